"""numpy restatement of the MOD-DiT hot path (test infrastructure only).

Conventions: maps are (H, n, n); features X are (H, 3n) in the column order of M:
[2n-1 diagonals, offset k-(n-1) = col-row][n columns][1 frame-block-diagonal].
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

__all__ = [
    "bf16_round", "fp16_round", "build_M", "mtm_closed_form", "mts_loop", "mts_exact",
    "ridge_solve", "features_from_x", "reconstruct_map", "predict_lines",
    "choose_topk_lines", "generate_mask_from_lines", "video_mask_cells", "mask_cell",
    "tiles_from_mask",
    "token_mask_from_tiles", "token_mask_rows_from_tiles", "token_mask_from_blocks",
    "masked_attention",
    "probability_map", "replay_map", "replay_map_rows", "refresh_merge", "step_phase", "video_layout",
    "cogvideox_grid", "e4m3_decode", "e4m3_encode", "quantize_qkv", "attention_q8",
    "attention_q8_with_bound", "q8_exact_error_bound", "e4m3_flip_candidates",
    "FP8_MFMA_SUM_REL", "FP8_MFMA_ACC_REL",
    "MODE_SPARSE", "MODE_BLOCK_DIAGONAL", "MODE_FULL",
]

MODE_SPARSE, MODE_BLOCK_DIAGONAL, MODE_FULL = 0, 1, 2

# Summation error of one v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3 operands, fp32 C): the
# instruction does not add its 64 products in exact fp32; its result C_in + sum_k a_k b_k
# is within FP8_MFMA_SUM_REL * sum_k |a_k b_k| + FP8_MFMA_ACC_REL * |C_in| of the exact
# value (plus the final fp32 rounding). Characterised on MI355X with the calibration
# probe moddit_calib_mfma_precision over 11 operand distributions (worst observed 2^-11.5
# of sum |a b| and, beyond that, 2^-22.2 of |C_in|); tests/test_gpu_calib.py holds the
# instruction to these constants. The bf16 MFMA sums to fp32 accuracy (2^-23.5).
FP8_MFMA_SUM_REL = 2.0 ** -10
FP8_MFMA_ACC_REL = 2.0 ** -21


# --------------------------------------------------------------------------------------
# rounding helpers
# --------------------------------------------------------------------------------------
def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to bfloat16 (round-to-nearest-even), returned as fp32."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = u.astype(np.uint32).view(np.float32)
    return np.where(nan, np.float32(np.nan), out).astype(np.float32)


def fp16_round(x: np.ndarray) -> np.ndarray:
    """Round to IEEE half (numpy's cast is round-to-nearest-even), returned as fp32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


# --------------------------------------------------------------------------------------
# layouts (MoD/mod/triton_flash_sparsity.py:101-120)
# --------------------------------------------------------------------------------------
def video_layout(model_type: str, S: int, video_tokens: int, text_tokens: int, bs: int):
    """(video_blocks, q_offset, k_offset). cogvideox counts a partial last video block."""
    if model_type == "wan":
        return S // bs, 0, 0
    if model_type == "hunyuan":
        return video_tokens // bs, 0, 0
    if model_type == "cogvideox":
        return -(-video_tokens // bs), text_tokens, text_tokens
    raise ValueError(f"Unknown model_type: {model_type}")


def cogvideox_grid(text_tokens: int, video_tokens: int, bs: int):
    """(text_blocks, video_blocks, origin) of the padded text-first grid.

    This build's padding rule for shapes the reference rejects
    (MoD/mod/triton_flash_sparsity.py:157-160): text occupies whole blocks that end where
    the video starts, video occupies whole blocks from there; grid token g is sequence
    token g + origin, and grid tokens outside the sequence are padding."""
    tb = (text_tokens + bs - 1) // bs
    vb = (video_tokens + bs - 1) // bs
    return tb, vb, text_tokens - tb * bs


# --------------------------------------------------------------------------------------
# line model (MoD/mod/cuda_lstsq.py)
# --------------------------------------------------------------------------------------
def build_M(n: int, bpf: int) -> np.ndarray:
    """Explicit (n*n, 3n) indicator matrix of the line model (brute force, small n).

    Column k < 2n-1: cells with col-row = k-(n-1); column 2n-1+j: cells of column j;
    last column: cells inside the n//bpf frame-diagonal bpf x bpf blocks
    (MoD/mod/cuda_lstsq.py:52-86, cuda_lstsq_kernel.cu:17-162).
    """
    nd = 2 * n - 1
    F = 3 * n
    M = np.zeros((n * n, F), dtype=np.float64)
    for r in range(n):
        for c in range(n):
            cell = r * n + c
            M[cell, (c - r) + (n - 1)] = 1.0
            M[cell, nd + c] = 1.0
    nb = n // bpf
    for f in range(nb):
        for i in range(bpf):
            for j in range(bpf):
                M[(f * bpf + i) * n + (f * bpf + j), F - 1] = 1.0
    return M


def mtm_closed_form(n: int, bpf: int, lam: float) -> np.ndarray:
    """M^T M + lam I from the closed forms of MoD/mod/cuda_lstsq.py:42-89."""
    nd = 2 * n - 1
    F = 3 * n
    G = np.zeros((F, F), dtype=np.float64)
    offs = np.arange(-(n - 1), n)
    G[np.arange(nd), np.arange(nd)] = n - np.abs(offs)
    G[nd + np.arange(n), nd + np.arange(n)] = n
    cols = np.arange(n)[None, :]
    o = offs[:, None]
    dv = np.where(o >= 0, cols >= o, cols < n + o).astype(np.float64)
    G[:nd, nd:nd + n] = dv
    G[nd:nd + n, :nd] = dv.T
    nbk = n // bpf
    db = np.where(np.abs(offs) < bpf, nbk * (bpf - np.abs(offs)), 0).astype(np.float64)
    G[:nd, -1] = db
    G[-1, :nd] = db
    vb = np.where(np.arange(n) < nbk * bpf, bpf, 0).astype(np.float64)
    G[nd:nd + n, -1] = vb
    G[-1, nd:nd + n] = vb
    G[-1, -1] = nbk * bpf * bpf
    G += lam * np.eye(F)
    return G


def mts_loop(S: np.ndarray, bpf: int) -> np.ndarray:
    """M^T S as the reference's CPU fallback loops it, in fp32 (MoD/mod/cuda_lstsq.py:91-139).

    Small n only (pure-Python loop). Sums accumulate in fp32 in the reference's order.
    """
    S = np.asarray(S, dtype=np.float32)
    H, n, _ = S.shape
    nd = 2 * n - 1
    out = np.zeros((H, 3 * n), dtype=np.float32)
    for k in range(nd):
        off = k - (n - 1)
        tot = np.zeros(H, dtype=np.float32)
        if off >= 0:
            for i in range(n - off):
                tot = (tot + S[:, i, i + off]).astype(np.float32)
        else:
            for i in range(n + off):
                tot = (tot + S[:, i - off, i]).astype(np.float32)
        out[:, k] = tot
    for k in range(n):
        out[:, nd + k] = S[:, :, k].sum(axis=1, dtype=np.float32)
    nbk = n // bpf
    tot = np.zeros(H, dtype=np.float32)
    for f in range(nbk):
        s = f * bpf
        tot = (tot + S[:, s:s + bpf, s:s + bpf].sum(axis=(1, 2), dtype=np.float32)).astype(np.float32)
    out[:, 3 * n - 1] = tot
    return out


def mts_exact(S16: np.ndarray, bpf: int) -> np.ndarray:
    """M^T S of an fp16 map: exact sums, each rounded once to fp32.

    Every fp16 value is an integer multiple of 2^-24, so the sums are formed exactly in
    int64 units of 2^-24 and converted with one round-to-nearest. Equal to mts_loop
    wherever the fp32 loop is exact (diagonal and column sums of maps whose entries
    are multiples of 2^-12 with n * 2^12 < 2^24).
    """
    S16 = np.asarray(S16, dtype=np.float16)
    H, n, _ = S16.shape
    units = np.rint(S16.astype(np.float64) * 2.0 ** 24).astype(np.int64)
    nd = 2 * n - 1
    out = np.zeros((H, 3 * n), dtype=np.float32)
    r = np.arange(n)[:, None]
    c = np.arange(n)[None, :]
    dk = (c - r) + (n - 1)
    for h in range(H):
        dsum = np.zeros(nd, dtype=np.int64)
        np.add.at(dsum, dk.ravel(), units[h].ravel())
        csum = units[h].sum(axis=0)
        nbk = n // bpf
        bsum = np.int64(0)
        for f in range(nbk):
            s = f * bpf
            bsum += units[h, s:s + bpf, s:s + bpf].sum()
        vals = np.concatenate([dsum, csum, [bsum]]).astype(np.int64)
        out[h] = vals.astype(np.float32) * np.float32(2.0 ** -24)
    return out


def ridge_solve(S: np.ndarray, bpf: int, lam: float) -> np.ndarray:
    """X = (M^T M + lam I)^-1 M^T S in fp64 (the target of MoD/mod/cuda_lstsq.py:211-264)."""
    S = np.asarray(S, dtype=np.float64)
    H, n, _ = S.shape
    G = mtm_closed_form(n, bpf, lam)
    mts = np.stack([_mts_f64(S[h], bpf) for h in range(H)])
    return np.linalg.solve(G, mts.T).T


def _mts_f64(S2: np.ndarray, bpf: int) -> np.ndarray:
    n = S2.shape[0]
    nd = 2 * n - 1
    r = np.arange(n)[:, None]
    c = np.arange(n)[None, :]
    dk = ((c - r) + (n - 1)).ravel()
    d = np.bincount(dk, weights=S2.ravel(), minlength=nd)
    cs = S2.sum(axis=0)
    nbk = n // bpf
    b = sum(S2[f * bpf:(f + 1) * bpf, f * bpf:(f + 1) * bpf].sum() for f in range(nbk))
    return np.concatenate([d, cs, [b]])


def features_from_x(X: np.ndarray, n: int) -> Dict[str, np.ndarray]:
    """Feature slicing of MoD/mod/cuda_lstsq.py:249-261 (c = columns / 2)."""
    nd = 2 * n - 1
    X = np.asarray(X, dtype=np.float32)
    return {"d": X[:, :nd], "c": X[:, nd:nd + n] / np.float32(2), "b_d": X[:, -1]}


def reconstruct_map(X: np.ndarray, n: int, bpf: int) -> np.ndarray:
    """M X per head (MoD/mod/cuda_lstsq.py:271-357, with c given back as 2c)."""
    X = np.asarray(X, dtype=np.float64)
    H = X.shape[0]
    nd = 2 * n - 1
    out = np.zeros((H, n, n))
    r = np.arange(n)[:, None]
    c = np.arange(n)[None, :]
    for h in range(H):
        out[h] = X[h, (c - r) + (n - 1)] + X[h, nd + c]
        for f in range(n // bpf):
            out[h, f * bpf:(f + 1) * bpf, f * bpf:(f + 1) * bpf] += X[h, -1]
    return out


# --------------------------------------------------------------------------------------
# line selection (MoD/mod/attn_mask.py:336-370)
# --------------------------------------------------------------------------------------
def predict_lines(x_cur: np.ndarray, x_last: np.ndarray, n: int, T: int) -> np.ndarray:
    """v = cat(pred_c, pred_d), pred = cur + (cur - last) / T, all in fp32 (:358-362)."""
    nd = 2 * n - 1
    xc = np.asarray(x_cur, dtype=np.float32)
    xl = np.asarray(x_last, dtype=np.float32)
    c_cur = xc[:, nd:nd + n] / np.float32(2)
    c_last = xl[:, nd:nd + n] / np.float32(2)
    d_cur = xc[:, :nd]
    d_last = xl[:, :nd]
    Tf = np.float32(T)
    pc = c_cur + (c_cur - c_last) / Tf
    pd = d_cur + (d_cur - d_last) / Tf
    return np.concatenate([pc, pd], axis=1).astype(np.float32)


def choose_topk_lines(x_cur, x_last, n: int, T: int, top_k: int) -> np.ndarray:
    """Indices of the k = min(top_k, 3n-1) smallest predictions per head, ascending.

    topk(largest=False, sorted=False) (:363-369) with ties broken by lower index and NaN
    ordered last; -0.0 and +0.0 compare equal.
    """
    v = predict_lines(x_cur, x_last, n, T)
    k = min(int(top_k), v.shape[1])
    out = []
    for h in range(v.shape[0]):
        row = v[h].astype(np.float64)
        row = np.where(row == 0.0, 0.0, row)
        key_nan = np.isnan(row)
        order = np.lexsort((np.arange(row.size), np.where(key_nan, np.inf, row), key_nan))
        out.append(np.sort(order[:k]))
    return np.stack(out).astype(np.int64) if out else np.zeros((0, k), np.int64)


# --------------------------------------------------------------------------------------
# mask generation (MoD/mod/attn_mask.py:440-559)
# --------------------------------------------------------------------------------------
def generate_mask_from_lines(sel: np.ndarray, modes: Sequence[int], *, seq_len: int,
                             block_size: int, video_tokens: int, text_tokens: int,
                             bpf: int, model_type: str) -> np.ndarray:
    """Line-by-line restatement of generate_mask_from_lines (bool (H, nb, nb))."""
    H = len(modes)
    block_num = seq_len // block_size
    tb = text_tokens // block_size
    vb = video_tokens // block_size
    if model_type == "cogvideox":
        tb, vb, _ = cogvideox_grid(text_tokens, video_tokens, block_size)
        block_num = tb + vb
    mask = np.ones((H, block_num, block_num), dtype=bool)
    video = np.zeros((H, vb, vb), dtype=bool)
    sel = np.asarray(sel, dtype=np.int64)
    if sel.ndim == 1:
        sel = sel[:, None]
    full = np.array([m == MODE_FULL for m in modes])
    bd = np.array([m == MODE_BLOCK_DIAGONAL for m in modes])
    video[full] = True
    if vb > 0:
        row = np.arange(vb).reshape(1, vb, 1)
        col = np.arange(vb).reshape(1, 1, vb)
        diff = col - row
        for t in range(sel.shape[1]):
            idx = sel[:, t]
            active = ~full
            if not active.any():
                break
            col_case = (idx < vb) & active
            if col_case.any():
                eq = (np.arange(vb).reshape(1, vb) == idx.reshape(H, 1)) & col_case.reshape(H, 1)
                video |= np.broadcast_to(eq[:, None, :], (H, vb, vb))
            diag_case = (idx >= vb) & active
            if diag_case.any():
                offs = idx - (vb - 1) - vb
                video |= (diff == offs.reshape(H, 1, 1)) & diag_case.reshape(H, 1, 1)
        if bd.any():
            rb = (np.arange(vb) // bpf).reshape(vb, 1)
            cb = (np.arange(vb) // bpf).reshape(1, vb)
            video |= bd.reshape(H, 1, 1) & (rb == cb)[None]
    if model_type == "cogvideox":
        if tb > 0:
            mask[:, :tb, :] = True
            mask[:, :, :tb] = True
        mask[:, tb:, tb:] = video
    elif model_type == "hunyuan":
        mask[:, vb:, :] = True
        mask[:, :, vb:] = True
        mask[:, :vb, :vb] = video
    elif model_type == "wan":
        mask = video
    else:
        mask = np.ones_like(mask)
    return mask


def video_mask_cells(sel: np.ndarray, modes: Sequence[int], n: int, bpf: int) -> np.ndarray:
    """The per-cell definition of `mask_cell` evaluated for whole (H, n, n) video masks:
    cell (i, j) is set iff the head is 'full', column j is selected, diagonal j - i is
    selected, or the head is block-diagonal and i, j share a frame. For shapes where the
    line-by-line restatement is slow (n = 1800)."""
    sel = np.asarray(sel, dtype=np.int64)
    H = len(modes)
    out = np.zeros((H, n, n), dtype=bool)
    r = np.arange(n)[:, None]
    c = np.arange(n)[None, :]
    diag_idx = (c - r) + (n - 1)
    same_frame = (r // bpf) == (c // bpf)
    for h in range(H):
        if modes[h] == MODE_FULL:
            out[h] = True
            continue
        col = np.zeros(n, dtype=bool)
        dia = np.zeros(2 * n - 1, dtype=bool)
        idx = sel[h]
        col[idx[(idx >= 0) & (idx < n)]] = True
        dd = idx[(idx >= n) & (idx < 3 * n - 1)] - n
        dia[dd] = True
        out[h] = col[None, :] | dia[diag_idx]
        if modes[h] == MODE_BLOCK_DIAGONAL:
            out[h] |= same_frame
    return out


def mask_cell(sel_h: Sequence[int], mode: int, n: int, bpf: int, i: int, j: int) -> bool:
    """Independent per-cell definition of the video mask (used to cross-check)."""
    if mode == MODE_FULL:
        return True
    for idx in sel_h:
        if 0 <= idx < n and idx == j:
            return True
        if n <= idx < 3 * n - 1 and (j - i) == idx - n - (n - 1):
            return True
    return mode == MODE_BLOCK_DIAGONAL and i // bpf == j // bpf


# --------------------------------------------------------------------------------------
# attention engine tiles (MoD/mod/attn_mask.py:296-311)
# --------------------------------------------------------------------------------------
def tiles_from_mask(mask: np.ndarray, block_size: int, union_rows: bool,
                    kv_tiles: Optional[int] = None) -> Tuple[np.ndarray, List[List[List[int]]]]:
    """Per (head, 128-row query tile) ascending entries (key_tile << 2 | row bits).

    mask: bool (H, rows, cols) block mask (rows = query blocks, cols = key blocks).
    """
    H, rows, cols = mask.shape
    nq = (rows * block_size + 127) // 128
    per_col = block_size // 64
    cap = cols * per_col
    if kv_tiles is None:
        kv_tiles = cap
    counts = np.zeros((H, nq), dtype=np.int32)
    lists: List[List[List[int]]] = []
    for h in range(H):
        hl = []
        for t in range(nq):
            if block_size == 64:
                r0, r1 = 2 * t, 2 * t + 1
                m0 = mask[h, r0].astype(bool) if r0 < rows else np.zeros(cols, bool)
                m1 = mask[h, r1].astype(bool) if r1 < rows else np.zeros(cols, bool)
                js = np.nonzero((m0 | m1)[:kv_tiles])[0]
                bits = (np.full(js.size, 3) if union_rows
                        else m0[js].astype(np.int64) | (m1[js].astype(np.int64) << 1))
                ent = ((js << 2) | bits).tolist()
            else:
                js = np.nonzero(mask[h, t].astype(bool))[0]
                kts = np.stack([2 * js, 2 * js + 1], axis=1).reshape(-1)  # ascending
                kts = kts[kts < kv_tiles]
                ent = ((kts << 2) | 3).tolist()
            counts[h, t] = len(ent)
            hl.append(ent)
        lists.append(hl)
    return counts, lists


def token_mask_from_tiles(lists, H: int, q_len: int, kv_len: int, origin: int = 0) -> np.ndarray:
    """Token-level (H, q_len, kv_len) mask the block-sparse kernel realises.

    Tiles sit on a grid whose token 0 is sequence token `origin` (<= 0); the parts of a
    tile outside the sequence are dropped."""
    m = np.zeros((H, q_len, kv_len), dtype=bool)
    for h in range(H):
        for t, ent in enumerate(lists[h]):
            for e in ent:
                kt, bits = e >> 2, e & 3
                k0 = max(kt * 64 + origin, 0)
                k1 = min(kt * 64 + 64 + origin, kv_len)
                for half in range(2):
                    if bits & (1 << half):
                        q0 = max(t * 128 + 64 * half + origin, 0)
                        q1 = min(t * 128 + 64 * half + 64 + origin, q_len)
                        if q0 < q1 and k0 < k1:
                            m[h, q0:q1, k0:k1] = True
    return m


def token_mask_rows_from_tiles(counts_h: np.ndarray, entries_h: np.ndarray, rows: np.ndarray,
                               kv_len: int, origin: int = 0) -> np.ndarray:
    """Rows `rows` (token indices) of one head's token-level mask, (len(rows), kv_len),
    from tile arrays as the kernel reads them: counts (n_qtiles,), entries
    (n_qtiles, cap) with entry = key_tile << 2 | row bits on the grid starting at token
    `origin`. Equals token_mask_from_tiles(...)[h, rows] without forming all rows."""
    rows = np.asarray(rows, dtype=np.int64)
    out = np.zeros((rows.size, kv_len), dtype=bool)
    for i, r in enumerate(rows):
        g = r - origin  # grid row
        t, half = g // 128, (g % 128) // 64
        ent = np.asarray(entries_h[t, :counts_h[t]], dtype=np.int64)
        for kt in (ent[(ent >> half) & 1 == 1] >> 2):
            k0, k1 = max(kt * 64 + origin, 0), min(kt * 64 + 64 + origin, kv_len)
            if k0 < k1:
                out[i, k0:k1] = True
    return out


def token_mask_from_blocks(mask: np.ndarray, block_size: int) -> np.ndarray:
    """Expand an (H, nb, nb) block mask to tokens."""
    return np.repeat(np.repeat(mask, block_size, axis=1), block_size, axis=2)


# --------------------------------------------------------------------------------------
# attention and the sparsity map
# --------------------------------------------------------------------------------------
def masked_attention(q, k, v, token_mask: Optional[np.ndarray] = None, scale=None,
                     dtype=np.float32):
    """Softmax attention under a token mask; rows with no allowed key give 0 / -inf LSE.

    q, k, v: (H, S, D) (one batch element). Returns (out (H,Sq,D), lse (H,Sq)) in `dtype`.
    Textbook definition (MoD/mod/triton_flash_sparsity.py:346-370 without the map).
    """
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    D = q.shape[-1]
    if scale is None:
        scale = D ** -0.5
    s = np.matmul(q, np.swapaxes(k, -1, -2)).astype(dtype) * dtype(scale)
    if token_mask is not None:
        s = np.where(token_mask, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    empty = ~np.isfinite(m)
    m = np.where(empty, 0, m)
    p = np.exp(s - m)
    l = p.sum(axis=-1, keepdims=True)
    out = np.matmul(p, v) / np.where(l > 0, l, 1)
    out = np.where(l > 0, out, 0)
    with np.errstate(divide="ignore"):
        lse = np.where(l[..., 0] > 0, np.log(np.where(l[..., 0] > 0, l[..., 0], 1)) + m[..., 0], -np.inf)
    return out.astype(dtype), lse.astype(dtype)


def probability_map(q, k, threshold: float, block_size: int, q_off: int, k_off: int,
                    video_tokens: int) -> np.ndarray:
    """fp32 probability map: mean over each block of [softmax < threshold].

    tests/test_flash_sparsity.py:28-49 and triton_flash_sparsity.py:346-370 of the
    reference. q, k: (H, S, D).
    """
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    H, S, D = q.shape
    s = np.einsum("hqd,hkd->hqk", q, k) * np.float32(D ** -0.5)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    pv = p[:, q_off:q_off + video_tokens, k_off:k_off + video_tokens]
    nb = video_tokens // block_size
    blk = (pv < threshold).reshape(H, nb, block_size, nb, block_size)
    return blk.mean(axis=(2, 4)).astype(np.float32)


def replay_map(q, k, lse, *, scale: float, log_threshold: float, q_off: int, k_off: int,
               video_blocks: int, block_size: int, dtype: str = "bf16") -> np.ndarray:
    """Replayed fp16 map (MoD/mod/cuda_flash_sparsity_kernel.cu:82-163).

    q*scale is formed in fp32 and rounded to the input dtype (:86-92), scores are exact
    dot products (fp64, which equals the fp32 accumulation whenever that is exact, e.g.
    for dyadic inputs), the comparison is strict against fp32(lse + log_threshold)
    (:138-143), and the ratio count/bs^2 is rounded to fp16 (:158-163).
    q, k: (H, S, D) float values already representable in `dtype`; lse: (H, S).
    The last block may run past S (this build's padded grid): positions >= S count
    nothing, and the cell is still divided by block_size^2.
    """
    rnd = bf16_round if dtype == "bf16" else fp16_round
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    H, S = q.shape[0], q.shape[1]
    vt = video_blocks * block_size
    nq = min(vt, S - q_off)
    nk = min(vt, S - k_off)
    qs = rnd(q[:, q_off:q_off + nq] * np.float32(scale)).astype(np.float64)
    kk = k[:, k_off:k_off + nk].astype(np.float64)
    thr = (np.asarray(lse, dtype=np.float32)[:, q_off:q_off + nq] + np.float32(log_threshold)).astype(np.float32)
    out = np.zeros((H, video_blocks, video_blocks), dtype=np.float16)
    for h in range(H):
        below = np.zeros((vt, vt), dtype=bool)
        below[:nq, :nk] = (qs[h] @ kk[h].T) < thr[h][:, None].astype(np.float64)
        cnt = below.reshape(video_blocks, block_size, video_blocks, block_size).sum(axis=(1, 3))
        out[h] = (cnt.astype(np.float32) / np.float32(block_size * block_size)).astype(np.float16)
    return out


def replay_map_rows(q, k, lse, blocks, *, scale: float, log_threshold: float,
                    video_blocks: int, block_size: int, dtype: str = "bf16") -> np.ndarray:
    """Rows `blocks` (query block indices) of replay_map for a video-only layout
    (offsets 0, whole blocks): (H, len(blocks), video_blocks) fp16. Same arithmetic as
    replay_map, for shapes whose full map is too large to form on the host."""
    rnd = bf16_round if dtype == "bf16" else fp16_round
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    H = q.shape[0]
    bs = block_size
    vt = video_blocks * bs
    kk = k[:, :vt].astype(np.float64)
    out = np.zeros((H, len(blocks), video_blocks), dtype=np.float16)
    for h in range(H):
        for i, b in enumerate(blocks):
            r0, r1 = b * bs, b * bs + bs
            qs = rnd(q[h, r0:r1] * np.float32(scale)).astype(np.float64)
            thr = (np.asarray(lse, np.float32)[h, r0:r1] + np.float32(log_threshold)).astype(np.float32)
            below = (qs @ kk[h].T) < thr[:, None].astype(np.float64)
            cnt = below.reshape(bs, video_blocks, bs).sum(axis=(0, 2))
            out[h, i] = (cnt.astype(np.float32) / np.float32(bs * bs)).astype(np.float16)
    return out


# --------------------------------------------------------------------------------------
# int8 / fp8 attention (the quantised engine, block_sparse_sage2_attn_cuda at
# MoD/mod/attn_mask.py:306, restated as SageAttention2's published scheme: int8 Q.K^T
# with per-block scales on a mean-smoothed K, fp8 e4m3 P.V with per-channel V scales)
# --------------------------------------------------------------------------------------
def e4m3_decode(b: np.ndarray) -> np.ndarray:
    """OCP FP8 E4M3 (bias 7, max 448, 0x7f/0xff NaN) bytes -> float64."""
    b = np.asarray(b).astype(np.int64)
    sign = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e - 7))
    mag = np.where((b & 0x7F) == 0x7F, np.nan, mag)
    return sign * mag


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float -> OCP E4M3 bytes (|x| <= 448)."""
    x = np.asarray(x, dtype=np.float64)
    table = e4m3_decode(np.arange(128))  # non-negative codes 0..127 (127 is NaN)
    vals = table[:127]
    a = np.abs(x)
    idx = np.searchsorted(vals, a)  # vals[idx-1] < a <= vals[idx]
    idx = np.clip(idx, 1, 126)
    lo, hi = vals[idx - 1], vals[idx]
    pick_hi = (a - lo > hi - a) | ((a - lo == hi - a) & (idx % 2 == 0))
    code = np.where(pick_hi, idx, idx - 1)
    code = np.where(a >= vals[126], 126, code)
    code = np.where(a == 0, 0, code)
    return (code | np.where(x < 0, 0x80, 0)).astype(np.uint8)


def quantize_qkv(q, k, v, k_mean: Optional[np.ndarray] = None,
                 origin: int = 0) -> Dict[str, np.ndarray]:
    """Quantise one batch element's q/k/v (H, S, D) (values exact in fp32).

    Follows the fp32 operations of the definition in include/moddit.h: blocks of 32 and
    tiles of 64 positions on the grid that starts at token `origin` (tokens outside the
    sequence count as zero), scale = amax/127 (or 448), x * (127/amax) rounded
    half-to-even, K minus its per-channel mean (the mean is taken from `k_mean` when given,
    so the rest can be compared bit for bit), v8t column c = token origin + c.
    q_kmean = q . k_mean in fp64."""
    f32 = np.float32
    q = np.asarray(q, f32)
    k = np.asarray(k, f32)
    v = np.asarray(v, f32)
    H, S, D = q.shape
    if k_mean is None:
        k_mean = (k.astype(np.float64).mean(axis=1)).astype(f32)
    k_mean = np.asarray(k_mean, f32)
    G = S - origin
    nqb, nkt = (G + 31) // 32, (G + 63) // 64
    s_pad = nkt * 64

    def grid(x):  # (H, S, D) -> (H, s_pad, D) on the grid, zero outside the sequence
        g = np.zeros((H, s_pad, D), f32)
        g[:, -origin:-origin + S] = x
        return g

    out = dict(q8=np.zeros((H, S, D), np.int8), q_scale=np.zeros((H, nqb), f32),
               k8=np.zeros((H, S, D), np.int8), k_scale=np.zeros((H, nkt), f32),
               v8t=np.zeros((H, D, s_pad), np.uint8), v_scale=np.zeros((H, D), f32),
               k_mean=k_mean,
               q_kmean=np.einsum("hsd,hd->hs", q.astype(np.float64), k_mean.astype(np.float64)))

    def q_int(x, amax):
        inv = f32(127) / amax if amax > 0 else f32(1)
        return np.clip(np.rint((x * inv).astype(f32)), -127, 127).astype(np.int8)

    qg = grid(q)
    kg = grid((k - k_mean[:, None, :]).astype(f32))
    q8g = np.zeros((H, s_pad, D), np.int8)
    k8g = np.zeros((H, s_pad, D), np.int8)
    for h in range(H):
        for b in range(nqb):
            blk = qg[h, 32 * b:32 * b + 32]
            am = f32(np.abs(blk).max())
            q8g[h, 32 * b:32 * b + 32] = q_int(blk, am)
            out["q_scale"][h, b] = am / f32(127) if am > 0 else f32(1)
        for t in range(nkt):
            blk = kg[h, 64 * t:64 * t + 64]
            am = f32(np.abs(blk).max())
            k8g[h, 64 * t:64 * t + 64] = q_int(blk, am)
            out["k_scale"][h, t] = am / f32(127) if am > 0 else f32(1)
        vam = np.abs(v[h]).max(axis=0).astype(f32)
        vinv = np.where(vam > 0, f32(448) / np.where(vam > 0, vam, 1), f32(1)).astype(f32)
        out["v_scale"][h] = np.where(vam > 0, vam / f32(448), f32(1))
        out["v8t"][h, :, -origin:-origin + S] = e4m3_encode((v[h] * vinv[None, :]).astype(f32)).T
    out["q8"] = q8g[:, -origin:-origin + S]
    out["k8"] = k8g[:, -origin:-origin + S]
    return out


def attention_q8(qz: Dict[str, np.ndarray], token_mask: Optional[np.ndarray] = None,
                 scale: Optional[float] = None, slack: float = 1.5, shift: float = 7.0,
                 origin: int = 0):
    """Attention on quantised inputs (the output of `quantize_qkv` with the same `origin`),
    in fp64, modelling the kernel's arithmetic: scores int8.int8 * q_scale * k_scale (log2
    units); key tiles of 64 on the grid starting at token `origin` visited in ascending
    order, the row max moved only when a tile's max exceeds it by more than `slack`;
    P = exp2(s - m + shift) rounded to e4m3 for the P.V product, the row sum over the
    unrounded P, earlier tiles rescaled by 2^(m_old - m_new); O times v_scale.
    LSE (natural log) = ln(sum P) + (m - shift) ln 2 + scale * q_kmean.
    Returns (O (H, S, D), LSE (H, S)); rows without keys: O = 0, LSE = -inf."""
    out, lse, _ = _attention_q8_core(qz, token_mask, scale, slack, shift, origin, False, False)
    return out, lse


def e4m3_flip_candidates(p: np.ndarray, tol: np.ndarray) -> np.ndarray:
    """True where a non-negative value p could round to another e4m3 code than its own
    under a relative change of at most tol: p (1 - tol) and p (1 + tol) round to
    different codes (the rounding is monotone, so every value in between rounds to one
    of those two)."""
    p = np.asarray(p, np.float64)
    return e4m3_encode(p * (1 - tol)) != e4m3_encode(p * (1 + tol))


def attention_q8_with_bound(qz: Dict[str, np.ndarray], token_mask: Optional[np.ndarray] = None,
                            scale: Optional[float] = None, slack: float = 1.5,
                            shift: float = 7.0, origin: int = 0, emulate_fp32: bool = False,
                            p_jitter: float = 0.0, jitter_seed: int = 0,
                            mfma_jitter: float = 0.0):
    """`attention_q8` plus, per output element, a bound on how far an implementation of
    the same arithmetic in fp32 (the kernel) can be from this fp64 model:

      - a weight P whose fp64 value lies within fp32's error of an e4m3 rounding midpoint
        (P * (1 -/+ tol) round to different codes, tol = 4e-6 (1 + |s|): the score's fp32
        roundings and exp2's ulp, ~30x over) may round one code the other way: up to
        2^-3 (1 + 2^-4) P |v8| for a normal P, one subnormal step 2^-9 |v8| below 2^-6;
      - a row whose lazy-max decision (tile max > m + slack) lies within 4e-6 (1 + |m|)
        of its threshold may move its max at another tile, after which every P of the row
        can round the other way: 2^-3 (1 + 2^-4) sum_j P_j |v8_j| for that row;
      - the fp8 MFMA's own summation of each tile's 64 products P8 v8 onto the
        accumulator: FP8_MFMA_SUM_REL sum_tile P8 |v8| + FP8_MFMA_ACC_REL |acc| per tile;
      - fp32 accumulation of O and of the row sum l: (keys + 2 tiles + 256) 2^-24
        relative to |O| + sum_j P_j |v8_j| v_scale / l (recursive-summation bound);
      - the kernel's bf16 output rounding: 2^-9 of |O| plus the terms above, taken as
        2^-8 |O| + 2^-8 (terms).
    All P terms are rescaled with the accumulator and divided by l like O.
    emulate_fp32: compute the scores and exp2 in fp32 (an fp32 rendering of the same
    arithmetic, used on the CPU to exercise the bound); p_jitter: multiply every P by
    1 + p_jitter * U(-1, 1) (seeded) before it is rounded and summed (another rendering
    whose P differ by up to p_jitter, for the same purpose; the bound itself is computed
    from the unperturbed model); mfma_jitter: add mfma_jitter * U(-1, 1) times the fp8
    MFMA error model's allowance to each tile's P.V sum (a rendering whose MFMA sums err
    by up to mfma_jitter of what the model allows). Returns (O, LSE, bound)."""
    return _attention_q8_core(qz, token_mask, scale, slack, shift, origin, True, emulate_fp32,
                              p_jitter, jitter_seed, mfma_jitter)


def _attention_q8_core(qz, token_mask, scale, slack, shift, origin, want_bound, fp32,
                       p_jitter=0.0, jitter_seed=0, mfma_jitter=0.0):
    q8 = qz["q8"].astype(np.float64)
    k8 = qz["k8"].astype(np.float64)
    H, S, D = q8.shape
    if scale is None:
        scale = D ** -0.5
    pos = np.arange(S) - origin  # grid position of each token
    qs = qz["q_scale"].astype(np.float64)[:, pos // 32]
    ks = qz["k_scale"].astype(np.float64)[:, pos // 64]
    v = e4m3_decode(qz["v8t"][:, :, pos]).transpose(0, 2, 1)  # (H, S, D)
    vs = qz["v_scale"].astype(np.float64)
    out = np.zeros((H, S, D))
    lse = np.full((H, S), -np.inf)
    bound = np.zeros((H, S, D)) if want_bound else None
    nt = (S - origin + 63) // 64
    f32 = np.float32
    jrng = np.random.default_rng(jitter_seed)
    for h in range(H):
        if fp32:
            s_all = (((q8[h] @ k8[h].T).astype(f32) * qs[h][:, None].astype(f32))
                     * ks[h][None, :].astype(f32)) * f32(scale * np.log2(np.e))
            s_all = s_all.astype(np.float64)
        else:
            s_all = (q8[h] @ k8[h].T) * qs[h][:, None] * ks[h][None, :] * scale * np.log2(np.e)
        if token_mask is not None:
            s_all = np.where(token_mask[h], s_all, -np.inf)
        m = np.full(S, -np.inf)
        acc = np.zeros((S, D))
        l = np.zeros(S)
        av = np.abs(v[h])
        if want_bound:
            flip_acc = np.zeros((S, D))
            tot_acc = np.zeros((S, D))
            mfma_acc = np.zeros((S, D))
            near_max = np.zeros(S, bool)
            n_keys = np.zeros(S)
            n_tiles = np.zeros(S)
        for t in range(nt):
            k0, k1 = max(origin + 64 * t, 0), min(origin + 64 * t + 64, S)
            st = s_all[:, k0:k1]
            mx = st.max(axis=1)
            act = np.isfinite(mx)  # rows for which this tile holds a key
            need = act & (mx > m + slack)
            if want_bound:
                fin_m = np.isfinite(m)
                gap = np.where(act & fin_m, mx - np.where(fin_m, m, 0) - slack, np.inf)
                near_max |= np.abs(gap) <= 4e-6 * (1 + np.abs(np.where(act, mx, 0)))
            m_new = np.where(need, mx, m)
            fin_new = np.where(np.isfinite(m_new), m_new, 0)
            alpha = np.where(np.isfinite(m), np.exp2(np.where(np.isfinite(m), m - fin_new, 0)), 0.0)
            alpha = np.where(act, np.where(need, alpha, 1.0), 1.0)
            arg = st - (fin_new - shift)[:, None]
            if fp32:
                p = np.where(act[:, None], np.exp2(arg.astype(f32)).astype(np.float64), 0.0)
            else:
                p = np.where(act[:, None], np.exp2(arg), 0.0)
            p_model = p
            if p_jitter:
                p = p * (1 + p_jitter * jrng.uniform(-1, 1, p.shape))
            p8 = e4m3_decode(e4m3_encode(p))
            acc_in = acc * alpha[:, None]
            mfma_allow = (FP8_MFMA_SUM_REL * (p8 @ av[k0:k1])
                          + FP8_MFMA_ACC_REL * np.abs(acc_in)) if (want_bound or mfma_jitter) else 0
            acc = acc_in + p8 @ v[h, k0:k1]
            if mfma_jitter:
                acc = acc + mfma_jitter * jrng.uniform(-1, 1, acc.shape) * mfma_allow
            l = l * alpha + p.sum(axis=1)
            if want_bound:
                mfma_acc = mfma_acc * alpha[:, None] + mfma_allow
                p = p_model
                keyed = np.isfinite(st)
                tol = 4e-6 * (1 + np.abs(np.where(keyed, st, 0)))
                flip = e4m3_flip_candidates(p, tol) & keyed
                step = np.maximum(2.0 ** -3 * (1 + 2.0 ** -4) * p, 2.0 ** -9)
                flip_acc = flip_acc * alpha[:, None] + np.where(flip, step, 0.0) @ av[k0:k1]
                tot_acc = tot_acc * alpha[:, None] + p @ av[k0:k1]
                n_keys += keyed.sum(axis=1)
                n_tiles += act
            m = m_new
        o = acc * vs[h][None, :]
        ok = l > 0
        linv = np.where(ok, 1.0 / np.where(ok, l, 1), 0.0)[:, None]
        out[h] = o * linv
        lse[h] = np.where(ok, np.log(np.where(ok, l, 1)) + (np.where(ok, m, 0) - shift) * np.log(2)
                          + scale * qz["q_kmean"][h], -np.inf)
        if want_bound:
            tot = tot_acc * vs[h][None, :] * linv
            flip_o = np.where(near_max[:, None], 2.0 ** -3 * (1 + 2.0 ** -4) * tot,
                              flip_acc * vs[h][None, :] * linv)
            gam = (n_keys + 2 * n_tiles + 256)[:, None] * 2.0 ** -24
            mfma_o = mfma_acc * vs[h][None, :] * linv
            terms = flip_o + mfma_o + gam * (np.abs(out[h]) + tot)
            bound[h] = terms * (1 + 2.0 ** -8) + 2.0 ** -8 * np.abs(out[h])
    return out, lse, bound


def q8_exact_error_bound(q, k, v, q8, q_scale, k8, k_scale, k_mean, v_scale,
                         allowed: Optional[np.ndarray] = None, scale: Optional[float] = None,
                         drop: Sequence[str] = ()):
    """Exact attention of query rows q (R, D) over keys k, v (S, D) (the unquantised bf16
    values, fp64), and a bound on how far the int8 Q.K^T / fp8 P.V kernel's output can be
    from it, per element, derived from the rounding model of that arithmetic:

    q8 (R, D) int8 with per-row q_scale (R,) (each row's 32-row block scale), k8 (S, D)
    int8 with per-key k_scale (S,) (its 64-key tile's scale), k_mean (D,), v_scale (D,):
    the quantiser's outputs for these rows and keys. allowed (R, S): the executed mask.

      - int8 scores: the kernel's scores s8 = scale q8.k8 q_scale k_scale against the
        exact smoothed scores s = scale q.(k - k_mean) (the constant q.k_mean shift cancels
        in softmax) differ by e_j; with E = (max_j e_j - min_j e_j) / 2 over the row's keys
        plus 1e-5 (1 + max|s8|) for the kernel's fp32 scores and exp2, the weights satisfy
        w8_j / w_j in [e^-2E, e^2E], so sum_j (w8_j - w_j) v_j <= (e^2E - 1) sum_j w_j |v_j|;
      - e4m3 P and e4m3 V: each 2^-4 relative (normal values), so the P.V sum over the
        fp32 row sum of the unrounded P is off by <= (2^-3 + 2^-8) sum_j w8_j |v_j|, with
        sum_j w8_j |v_j| <= e^2E sum_j w_j |v_j|; below e4m3's normal range an absolute
        error instead: V below 2^-6 v_scale: 2^-10 v_scale (twice, both factors); P below
        2^-6: 2^-10 (1 + 2^-4) |v_j| / l with l >= 2^7 (P = 2^(y - m + 7), the lazy max
        m <= the row max y_max), for keys with y_j < y_max - 13 (log2 units) only;
      - the fp8 MFMA's summation (FP8_MFMA_SUM_REL of each tile's sum |P8 v8| and
        FP8_MFMA_ACC_REL of the accumulator per tile, which is at most the whole row's
        sum): (FP8_MFMA_SUM_REL + tiles FP8_MFMA_ACC_REL) (1 + 2^-4) e^2E sum_j w_j |v_j|;
      - fp32 accumulation (O and l over the keys): (keys + 2 tiles + 256) 2^-24
        relative to |o| + 2 e^2E sum_j w_j |v_j|;
      - bf16 output rounding: 2^-9 of |o| plus all the above.
    drop: names of terms to leave out ("score", "e4m3", "subnormal", "mfma",
    "accumulation", "output"), for tests that show each one is needed.
    Returns (o (R, D), bound (R, D), E (R,))."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    R, D = q.shape
    S = k.shape[0]
    if scale is None:
        scale = D ** -0.5
    if allowed is None:
        allowed = np.ones((R, S), bool)
    s = scale * (q @ (k - np.asarray(k_mean, np.float64)[None, :]).T)
    s8 = scale * (np.asarray(q8, np.float64) @ np.asarray(k8, np.float64).T) \
        * np.asarray(q_scale, np.float64)[:, None] * np.asarray(k_scale, np.float64)[None, :]
    e = np.where(allowed, s8 - s, np.nan)
    has = allowed.any(axis=1)
    E = np.where(has, (np.nanmax(np.where(has[:, None], e, 0), axis=1)
                       - np.nanmin(np.where(has[:, None], e, 0), axis=1)) / 2, 0.0)
    s8a = np.where(allowed, s8, -np.inf)
    E = E + 1e-5 * (1 + np.abs(np.where(allowed, s8, 0)).max(axis=1))
    sa = np.where(allowed, s, -np.inf)
    mx = np.where(has, sa.max(axis=1), 0)
    w = np.where(allowed, np.exp(sa - mx[:, None]), 0.0)
    w = w / np.where(has, w.sum(axis=1), 1)[:, None]
    av = np.abs(v)
    o = w @ v
    bv = w @ av
    y = s8a * np.log2(np.e)
    ymax = np.where(has, y.max(axis=1), 0)
    sub = allowed & (y < (ymax - 12.99)[:, None])
    sub_v = sub.astype(np.float64) @ av
    n_sub = sub.sum(axis=1)[:, None]
    keys = allowed.sum(axis=1)
    gam = ((keys + 2 * ((keys + 63) // 64) + 256) * 2.0 ** -24)[:, None]
    vsc = np.asarray(v_scale, np.float64)[None, :]
    grow = np.exp(2 * E)[:, None]
    on = {t: 0.0 if t in drop else 1.0
          for t in ("score", "e4m3", "subnormal", "mfma", "accumulation", "output")}
    tiles = ((keys + 63) // 64)[:, None]
    pre = (on["score"] * (grow - 1) * bv
           + on["e4m3"] * grow * (2.0 ** -3 + 2.0 ** -8) * bv
           + on["subnormal"] * (grow * 2.0 ** -9 * vsc
                                + 2.0 ** -17 * (1 + 2.0 ** -4) * (sub_v + n_sub * vsc * 2.0 ** -10))
           + on["mfma"] * (FP8_MFMA_SUM_REL + tiles * FP8_MFMA_ACC_REL) * (1 + 2.0 ** -4)
           * grow * bv
           + on["accumulation"] * gam * (np.abs(o) + 2 * grow * bv))
    out_r = on["output"] * 2.0 ** -9
    bound = np.where(has[:, None], pre * (1 + out_r) + out_r * np.abs(o), 0.0)
    return o, bound, E


def refresh_merge(prev: np.ndarray, cur: np.ndarray, mask: np.ndarray) -> np.ndarray:
    """torch.where(mask == False, prev, cur) (MoD/mod/attn_mask.py:671-675)."""
    return np.where(mask, cur, prev)


# --------------------------------------------------------------------------------------
# schedule (MoD/mod/attn_mask.py:598-712 with the processors' use_dense gate)
# --------------------------------------------------------------------------------------
def step_phase(step: int, W: int, T: int) -> str:
    """Phase of one call: 'dense' | 'map_fit' | 'map_fit_predict' | 'refresh' | 'sparse'.

    Processors run dense below W-2 (hunyuan/attention_processor.py:110-115); W-2 maps and
    fits (zero features); W-1 maps, fits and predicts; after W a refresh happens when
    (step-W) % T == T-1, otherwise the sparse engine runs.
    """
    if step < W - 2:
        return "dense"
    if step < W - 1:
        return "map_fit"
    if step == W - 1:
        return "map_fit_predict"
    if (step - W) % T == T - 1:
        return "refresh"
    return "sparse"
