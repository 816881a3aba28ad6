"""torch-CPU restatement of the reference's PyTorch path, for timing only.

Test infrastructure: only bench.py's cpu_baseline leg uses this module, to time the
reference's own CPU algorithms on the host cores in the same run as the GPU
measurements. Nothing in the product imports it. Every function follows the reference
function named in its docstring step for step, in torch on the CPU with the threads
torch is given (torch.get_num_threads()); the numpy oracle in moddit_ref.py is what the
tests check against.
"""
from __future__ import annotations

import time
from typing import Callable, Dict, List

import torch


def compute_mts_as_written(S_T: torch.Tensor, bpf: int, diagonals=None,
                           rest: bool = False) -> torch.Tensor:
    """M^T S with the reference's Python loops (MoD/mod/cuda_lstsq.py:91-139): one
    accumulation per diagonal cell, then per-column sums, then the frame blocks.
    `diagonals` restricts the first loop to a subset (for a bounded timing sample); the
    column and frame loops then run only with `rest`."""
    H, n, _ = S_T.shape
    nd = 2 * n - 1
    out = torch.zeros(H, 3 * n, dtype=S_T.dtype)
    for kd in (range(nd) if diagonals is None else diagonals):
        off = kd - (n - 1)
        acc = torch.zeros(H, dtype=S_T.dtype)
        if off >= 0:
            for i in range(n - off):
                acc += S_T[:, i, i + off]
        else:
            for i in range(n + off):
                acc += S_T[:, i - off, i]
        out[:, kd] = acc
    if diagonals is not None and not rest:
        return out
    for c in range(n):
        out[:, nd + c] = S_T[:, :, c].sum(dim=1)
    acc = torch.zeros(H, dtype=S_T.dtype)
    for f in range(n // bpf):
        s = f * bpf
        acc += S_T[:, s:s + bpf, s:s + bpf].sum(dim=(1, 2))
    out[:, 3 * n - 1] = acc
    return out


def compute_mts_vectorized(S_T: torch.Tensor, bpf: int) -> torch.Tensor:
    """The same M^T S as whole-tensor torch operations (one index_add for all diagonals)."""
    H, n, _ = S_T.shape
    nd = 2 * n - 1
    r = torch.arange(n).view(n, 1)
    c = torch.arange(n).view(1, n)
    dk = ((c - r) + (n - 1)).reshape(-1)
    diag = torch.zeros(H, nd, dtype=S_T.dtype).index_add_(1, dk, S_T.reshape(H, -1))
    cols = S_T.sum(dim=1)
    nb = n // bpf
    blk = S_T[:, :nb * bpf, :nb * bpf].reshape(H, nb, bpf, nb, bpf)
    frame = torch.diagonal(blk, dim1=1, dim2=3).sum(dim=(1, 2, 3))
    return torch.cat([diag, cols, frame.view(H, 1)], dim=1)


def compute_mtm(n: int, bpf: int, lam: float, dtype=torch.float32) -> torch.Tensor:
    """Closed-form M^T M + lambda I (MoD/mod/cuda_lstsq.py:42-89)."""
    nd = 2 * n - 1
    F = 3 * n
    G = torch.zeros(F, F, dtype=dtype)
    offs = torch.arange(-(n - 1), n)
    idx = torch.arange(nd)
    G[idx, idx] = (n - offs.abs()).to(dtype)
    vi = nd + torch.arange(n)
    G[vi, vi] = float(n)
    cols = torch.arange(n).view(1, n)
    og = offs.view(nd, 1)
    dv = torch.where(og >= 0, cols >= og, cols < n + og).to(dtype)
    G[:nd, nd:nd + n] = dv
    G[nd:nd + n, :nd] = dv.t()
    nbk = n // bpf
    db = torch.where(offs.abs() < bpf, nbk * (bpf - offs.abs()), torch.zeros_like(offs)).to(dtype)
    G[:nd, -1] = db
    G[-1, :nd] = db
    vb = torch.where(torch.arange(n) < nbk * bpf, bpf, 0).to(dtype)
    G[nd:nd + n, -1] = vb
    G[-1, nd:nd + n] = vb
    G[-1, -1] = float(nbk * bpf * bpf)
    return G + torch.eye(F, dtype=dtype) * lam


def choose_topk(x_cur: torch.Tensor, x_last: torch.Tensor, n: int, T: int, top_k: int):
    """Line prediction and torch.topk(largest=False, sorted=False)
    (MoD/mod/attn_mask.py:351-370)."""
    nd = 2 * n - 1
    c_cur, c_last = x_cur[:, nd:nd + n] / 2, x_last[:, nd:nd + n] / 2
    d_cur, d_last = x_cur[:, :nd], x_last[:, :nd]
    pred = torch.cat([c_cur + (c_cur - c_last) / T, d_cur + (d_cur - d_last) / T], dim=1)
    return torch.topk(pred, k=min(top_k, pred.shape[1]), dim=1, largest=False, sorted=False)[1]


def mask_from_lines_loop(sel: torch.Tensor, block_diag: torch.Tensor, n: int, bpf: int,
                         lines=None) -> torch.Tensor:
    """The video mask of generate_mask_from_lines (MoD/mod/attn_mask.py:440-559): one
    pass of whole-(H,n,n) tensor operations per selected line, then the frame blocks.
    `lines` restricts the loop to the first `lines` selections (a bounded sample)."""
    H, k = sel.shape
    video = torch.zeros(H, n, n, dtype=torch.bool)
    diff = torch.arange(n).view(1, 1, n) - torch.arange(n).view(1, n, 1)
    ar = torch.arange(n).view(1, n)
    for t in range(k if lines is None else min(lines, k)):
        idx = sel[:, t]
        col_case = idx < n
        if bool(col_case.any()):
            col_eq = (ar == idx.view(H, 1)) & col_case.view(H, 1)
            video |= col_eq.unsqueeze(1).expand(-1, n, -1)
        diag_case = idx >= n
        if bool(diag_case.any()):
            offs = idx - (n - 1) - n
            video |= (diff.expand(H, n, n) == offs.view(H, 1, 1)) & diag_case.view(H, 1, 1)
    if bool(block_diag.any()):
        rb = (torch.arange(n) // bpf).view(n, 1)
        cb = (torch.arange(n) // bpf).view(1, n)
        video |= block_diag.view(H, 1, 1) & (rb == cb).unsqueeze(0)
    return video


def probability_map_chunk(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, qb0: int,
                          qb1: int, block_size: int, threshold: float):
    """Query blocks [qb0, qb1) of the chunked PyTorch map (MoD/mod/attn_mask.py:151-222,
    the triton_flash_sparsity.py:346-370 statistic): fp32 scores over all keys, softmax,
    P.V, and the fraction of probabilities below the threshold per (block, key block).
    q, k, v: (S, D) of one head, video-only layout."""
    S, D = k.shape
    nb = S // block_size
    s = torch.matmul(q[qb0 * block_size:qb1 * block_size], k.t()) * (D ** -0.5)
    p = torch.softmax(s, dim=-1)
    out = torch.matmul(p, v)
    m = p.lt(threshold).view(qb1 - qb0, block_size, nb, block_size).float().mean(dim=(1, 3))
    return out, m.to(torch.float16)


def block_sparse_attention_tile(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, t: int,
                                entries: List[int], origin: int = 0) -> torch.Tensor:
    """One 128-row query tile of block-sparse attention (the sparse engine's semantics,
    MoD/mod/attn_mask.py:296-317): each 64-row half attends, in fp32, to the 64-key tiles
    whose entry enables it. q, k, v: (S, D) of one head. Returns (rows, D)."""
    S, D = k.shape
    outs = []
    for half in range(2):
        r0 = max(origin + t * 128 + 64 * half, 0)
        r1 = min(origin + t * 128 + 64 * half + 64, S)
        if r0 >= r1:
            continue
        kts = [e >> 2 for e in entries if e & (1 << half)]
        if not kts:
            outs.append(torch.zeros(r1 - r0, D))
            continue
        idx = torch.cat([torch.arange(max(origin + kt * 64, 0), min(origin + kt * 64 + 64, S))
                         for kt in kts])
        s = torch.matmul(q[r0:r1], k.index_select(0, idx).t()) * (D ** -0.5)
        outs.append(torch.matmul(torch.softmax(s, dim=-1), v.index_select(0, idx)))
    return torch.cat(outs) if outs else torch.zeros(0, D)


def timed(fn: Callable[[], object]) -> float:
    t0 = time.perf_counter()
    fn()
    return time.perf_counter() - t0


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"
