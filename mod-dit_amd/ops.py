"""Torch-facing wrappers over the C ABI (include/moddit.h).

Tensors are only plumbing here: each function validates shapes, allocates outputs with
torch on the input's device, and launches the HIP kernel on torch's current stream.
Nothing in this module computes on the host, and nothing falls back to torch math.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import check, strides3

_DTYPES = {torch.bfloat16: _lib.BF16, torch.float16: _lib.FP16}


def _stream(t: torch.Tensor):
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _require_gpu(*tensors: torch.Tensor, what: str) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise ValueError(f"{what}: tensors must live on a GPU (got {t.device})")


def _attn_view(t: torch.Tensor) -> torch.Tensor:
    """(B,H,S,D) with unit dim stride, 16-byte aligned; copies only if needed."""
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:3]):
        t = t.contiguous()
    return t


def _attn_dtype(t: torch.Tensor) -> int:
    if t.dtype not in _DTYPES:
        raise TypeError(f"expected float16 or bfloat16 inputs, got {t.dtype}")
    return _DTYPES[t.dtype]


# --------------------------------------------------------------------------------------
# attention
# --------------------------------------------------------------------------------------
@dataclass
class TileList:
    """Per-(head, 128-row query tile) ascending lists of active 64-key tiles.

    entries[h, t, i] = (key_tile << 2) | row_bits for i < counts[h, t]; bit 0 enables the
    tile for query rows 0..63 of the query tile, bit 1 for rows 64..127.
    Tiles sit on a grid whose row/column 0 is token `origin` (-63..0); grid positions
    before token 0 or past the sequence end are padding (keys masked, rows not written).
    """

    counts: torch.Tensor   # (H, n_qtiles) int32
    entries: torch.Tensor  # (H, n_qtiles, cap) int32
    block_size: int
    union_rows: bool
    origin: int = 0

    @property
    def n_qtiles(self) -> int:
        return self.counts.shape[1]

    @property
    def cap(self) -> int:
        return self.entries.shape[2]

    def active_tile_pairs(self) -> torch.Tensor:
        """Executed (64-row query block, 64-key tile) pairs per head (device tensor)."""
        bits = (self.entries & 1) + ((self.entries >> 1) & 1)
        idx = torch.arange(self.cap, device=self.entries.device).view(1, 1, -1)
        valid = idx < self.counts.unsqueeze(-1)
        return (bits * valid).sum(dim=(1, 2))


def _attention(q, k, v, scale, return_lse, tiles: TileList | None, out=None):
    _require_gpu(q, k, v, what="attention")
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("query, key and value must have shape [B, H, S, D]")
    if k.shape != v.shape or q.shape[:2] != k.shape[:2] or q.shape[3] != k.shape[3]:
        raise ValueError(f"incompatible shapes q={tuple(q.shape)} k={tuple(k.shape)} v={tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("query, key, and value must have the same dtype")
    dt = _attn_dtype(q)
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    if D not in (64, 128):
        raise ValueError(f"head_dim must be 64 or 128, got {D}")
    q, k, v = _attn_view(q), _attn_view(k), _attn_view(v)
    if out is None:
        out = torch.empty((B, H, Sq, D), device=q.device, dtype=q.dtype)
    lse = torch.empty((B, H, Sq), device=q.device, dtype=torch.float32) if return_lse else None
    if scale is None:
        scale = D ** -0.5
    if tiles is not None and tiles.counts.shape[0] != H:
        raise ValueError(f"tile lists cover {tiles.counts.shape[0]} heads, attention has {H}")
    lib = _lib.load()
    if out.numel() == 0:
        return out, lse  # no query rows: nothing to compute (empty tensors have no storage)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), _ptr(lse), B, H, Sq, Skv, D,
            strides3(*q.stride()[:3]), strides3(*k.stride()[:3]), strides3(*v.stride()[:3]),
            strides3(*out.stride()[:3]), float(scale), dt)
    if tiles is None:
        check(lib.moddit_flash_fwd(*args, _stream(q)), "moddit_flash_fwd")
    else:
        check(lib.moddit_block_sparse_fwd(*args, tiles.counts.data_ptr(), tiles.entries.data_ptr(),
                                          tiles.n_qtiles, tiles.cap, int(tiles.origin), _stream(q)),
              "moddit_block_sparse_fwd")
    return out, lse


def flash_fwd(q, k, v, softmax_scale=None, return_lse=True, out=None):
    """Dense attention over all keys; returns (O (B,H,Sq,D), LSE (B,H,Sq) fp32 or None)."""
    return _attention(q, k, v, softmax_scale, return_lse, None, out)


def block_sparse_fwd(q, k, v, tiles: TileList, softmax_scale=None, return_lse=False, out=None):
    """Attention restricted to the active key tiles of `tiles`."""
    return _attention(q, k, v, softmax_scale, return_lse, tiles, out)


def flash_fwd_map(q, k, v, *, softmax_scale, log_threshold, video_offset, video_blocks,
                  block_size, return_lse=True, out=None):
    """Dense self-attention and the fp16 (B,H,n,n) sparsity map in one kernel.

    Returns (O, LSE or None, map). The map equals `sparsity_map` applied to this LSE."""
    _require_gpu(q, k, v, what="flash_fwd_map")
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("query, key and value must have identical shape [B, H, S, D]")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("query, key, and value must have the same dtype")
    dt = _attn_dtype(q)
    B, H, S, D = q.shape
    if D not in (64, 128):
        raise ValueError(f"head_dim must be 64 or 128, got {D}")
    q, k, v = _attn_view(q), _attn_view(k), _attn_view(v)
    if out is None:
        out = torch.empty((B, H, S, D), device=q.device, dtype=q.dtype)
    lse = torch.empty((B, H, S), device=q.device, dtype=torch.float32) if return_lse else None
    smap = torch.empty((B, H, video_blocks, video_blocks), device=q.device, dtype=torch.float16)
    check(_lib.load().moddit_flash_fwd_map(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), _ptr(lse), smap.data_ptr(),
        B, H, S, D, strides3(*q.stride()[:3]), strides3(*k.stride()[:3]),
        strides3(*v.stride()[:3]), strides3(*out.stride()[:3]), float(softmax_scale),
        float(log_threshold), int(video_offset), int(video_blocks), int(block_size), dt,
        _stream(q)), "moddit_flash_fwd_map")
    return out, lse, smap


# --------------------------------------------------------------------------------------
# int8 / fp8 attention (SageAttention2-style quantised engine)
# --------------------------------------------------------------------------------------
@dataclass
class QuantizedQKV:
    """Output of `quantize_qkv` (all on the device; see include/moddit.h)."""

    q8: torch.Tensor       # int8 (B,H,S,D)
    q_scale: torch.Tensor  # fp32 (B,H,ceil(G/32)), G = S - origin: 32-position grid blocks
    k8: torch.Tensor       # int8 (B,H,S,D), K minus its per-channel mean
    k_scale: torch.Tensor  # fp32 (B,H,ceil(G/64)): 64-position grid tiles
    v8t: torch.Tensor      # uint8 e4m3 (B,H,D,s_pad), column c = token origin + c
    v_scale: torch.Tensor  # fp32 (B,H,D)
    k_mean: torch.Tensor   # fp32 (B,H,D)
    q_kmean: torch.Tensor  # fp32 (B,H,S): q . k_mean, the LSE correction
    dtype: torch.dtype     # of the source tensors (and of the attention output)
    origin: int = 0        # first token of the attention grid the blocks lie on

    @property
    def shape(self):
        return tuple(self.q8.shape)


def quantize_qkv(q, k, v, grid_origin: int = 0) -> QuantizedQKV:
    """Quantise self-attention q/k/v (B,H,S,D) bf16/fp16 for the int8/fp8 kernels, with
    blocks on the attention grid that starts at token `grid_origin` (-63..0: the
    `TileList.origin` the block-sparse kernel will run on; 0 for dense attention)."""
    _require_gpu(q, k, v, what="quantize_qkv")
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("query, key and value must have identical shape [B, H, S, D]")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("query, key, and value must have the same dtype")
    dt = _attn_dtype(q)
    B, H, S, D = q.shape
    if D not in (64, 128):
        raise ValueError(f"head_dim must be 64 or 128, got {D}")
    if not -64 < grid_origin <= 0:
        raise ValueError(f"grid_origin must lie in (-64, 0], got {grid_origin}")
    q, k, v = _attn_view(q), _attn_view(k), _attn_view(v)
    dev = q.device
    G = S - grid_origin
    s_pad = (G + 63) // 64 * 64
    lib = _lib.load()
    ws = torch.empty(lib.moddit_quantize_workspace_floats(B, H, D), device=dev, dtype=torch.float32)
    out = QuantizedQKV(
        q8=torch.empty((B, H, S, D), device=dev, dtype=torch.int8),
        q_scale=torch.empty((B, H, (G + 31) // 32), device=dev, dtype=torch.float32),
        k8=torch.empty((B, H, S, D), device=dev, dtype=torch.int8),
        k_scale=torch.empty((B, H, s_pad // 64), device=dev, dtype=torch.float32),
        v8t=torch.empty((B, H, D, s_pad), device=dev, dtype=torch.uint8),
        v_scale=torch.empty((B, H, D), device=dev, dtype=torch.float32),
        k_mean=torch.empty((B, H, D), device=dev, dtype=torch.float32),
        q_kmean=torch.empty((B, H, S), device=dev, dtype=torch.float32),
        dtype=q.dtype, origin=int(grid_origin))
    if B * H * S == 0:
        return out  # no rows to quantise
    check(lib.moddit_quantize_qkv(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), B, H, S, D, strides3(*q.stride()[:3]),
        strides3(*k.stride()[:3]), strides3(*v.stride()[:3]), dt, int(grid_origin),
        ws.data_ptr(), out.q8.data_ptr(), out.q_scale.data_ptr(), out.k8.data_ptr(),
        out.k_scale.data_ptr(), out.v8t.data_ptr(), out.v_scale.data_ptr(),
        out.k_mean.data_ptr(), out.q_kmean.data_ptr(), _stream(q)),
        "moddit_quantize_qkv")
    return out


def _attention_q8(qz: QuantizedQKV, scale, return_lse, tiles: TileList | None, out=None,
                  q_len=None):
    B, H, S, D = qz.shape
    q_len = S if q_len is None else int(q_len)
    if not 0 <= q_len <= S:
        raise ValueError(f"q_len={q_len} must lie in [0, {S}]")
    if out is None:
        out = torch.empty((B, H, q_len, D), device=qz.q8.device, dtype=qz.dtype)
    if tuple(out.shape) != (B, H, q_len, D) or out.dtype != qz.dtype:
        raise ValueError(f"out must be {qz.dtype} of shape {(B, H, q_len, D)}")
    lse = torch.empty((B, H, q_len), device=out.device, dtype=torch.float32) if return_lse else None
    if scale is None:
        scale = D ** -0.5
    dt = _attn_dtype(out)
    lib = _lib.load()
    origin = 0 if tiles is None else int(tiles.origin)
    if qz.origin != origin:
        raise ValueError(f"q/k/v were quantised on the grid starting at {qz.origin}, the "
                         f"attention runs on the grid starting at {origin}")
    if tiles is not None and tiles.counts.shape[0] != H:
        raise ValueError(f"tile lists cover {tiles.counts.shape[0]} heads, attention has {H}")
    if out.numel() == 0:
        return out, lse  # no query rows
    head = (qz.q8.data_ptr(), qz.q_scale.data_ptr(), qz.k8.data_ptr(), qz.k_scale.data_ptr(),
            qz.v8t.data_ptr(), qz.v_scale.data_ptr(), qz.q_kmean.data_ptr(), out.data_ptr(),
            _ptr(lse), B, H, S)
    tail = (D, strides3(*out.stride()[:3]), float(scale), dt)
    if tiles is None:
        check(lib.moddit_flash_fwd_q8(*head, *tail, _stream(out)), "moddit_flash_fwd_q8")
    else:
        check(lib.moddit_block_sparse_fwd_q8(*head, q_len, *tail, tiles.counts.data_ptr(),
                                             tiles.entries.data_ptr(), tiles.n_qtiles, tiles.cap,
                                             origin, _stream(out)),
              "moddit_block_sparse_fwd_q8")
    return out, lse


def flash_fwd_q8(qz: QuantizedQKV, softmax_scale=None, return_lse=True, out=None):
    """Dense int8/fp8 attention on quantised q/k/v; returns (O, LSE or None)."""
    return _attention_q8(qz, softmax_scale, return_lse, None, out)


def block_sparse_fwd_q8(qz: QuantizedQKV, tiles: TileList, softmax_scale=None, return_lse=False,
                        out=None, q_len=None):
    """Block-sparse int8/fp8 attention over the active key tiles of `tiles`; with `q_len`
    only queries 0..q_len-1 attend (to all keys), and O / LSE hold q_len rows."""
    return _attention_q8(qz, softmax_scale, return_lse, tiles, out, q_len)


# --------------------------------------------------------------------------------------
# sparsity map replay
# --------------------------------------------------------------------------------------
def sparsity_map(query, key, lse, *, softmax_scale, log_threshold, q_video_offset,
                 k_video_offset, video_blocks, block_size):
    """fp16 (B,H,n,n) map of MoD/mod/cuda_flash_sparsity.py:71-99 on the HIP replay kernel."""
    _require_gpu(query, key, lse, what="sparsity_map")
    if query.ndim != 4 or key.ndim != 4 or query.shape != key.shape:
        raise RuntimeError("Q and K must have identical shape [B, H, S, D]")
    if lse.ndim != 3 or tuple(lse.shape) != tuple(query.shape[:3]):
        raise RuntimeError("LSE shape must match Q except for head_dim")
    if lse.dtype != torch.float32:
        raise RuntimeError("LSE must be float32")
    if query.dtype != key.dtype:
        raise RuntimeError("Q and K dtypes must match")
    dt = _attn_dtype(query)
    B, H, S, D = query.shape
    query, key = _attn_view(query), _attn_view(key)
    lse = lse.contiguous()
    out = torch.empty((B, H, video_blocks, video_blocks), device=query.device, dtype=torch.float16)
    lib = _lib.load()
    check(lib.moddit_sparsity_map(query.data_ptr(), key.data_ptr(), lse.data_ptr(), out.data_ptr(),
                                  B, H, S, D, strides3(*query.stride()[:3]),
                                  strides3(*key.stride()[:3]), float(softmax_scale),
                                  float(log_threshold), int(q_video_offset), int(k_video_offset),
                                  int(video_blocks), int(block_size), dt, _stream(query)),
          "moddit_sparsity_map")
    return out


def sparsity_map_merge(query, key, lse, tiles: TileList, map_inout, *, softmax_scale,
                       log_threshold, q_video_offset, k_video_offset, video_blocks, block_size):
    """Write the sparsity_map cells that `tiles` (exact rows, over the video block mask)
    list into `map_inout` (B,H,n,n) fp16 contiguous, in place; the other cells keep their
    values (the refresh step's merge at the cost of the active cells)."""
    _require_gpu(query, key, lse, map_inout, what="sparsity_map_merge")
    if query.ndim != 4 or key.ndim != 4 or query.shape != key.shape:
        raise RuntimeError("Q and K must have identical shape [B, H, S, D]")
    if lse.ndim != 3 or tuple(lse.shape) != tuple(query.shape[:3]):
        raise RuntimeError("LSE shape must match Q except for head_dim")
    if lse.dtype != torch.float32:
        raise RuntimeError("LSE must be float32")
    if query.dtype != key.dtype:
        raise RuntimeError("Q and K dtypes must match")
    B, H, S, D = query.shape
    if (map_inout.dtype != torch.float16 or not map_inout.is_contiguous()
            or tuple(map_inout.shape) != (B, H, video_blocks, video_blocks)):
        raise ValueError(f"map must be a contiguous fp16 tensor of shape "
                         f"{(B, H, video_blocks, video_blocks)}")
    if tiles.union_rows or tiles.block_size != block_size or tiles.origin != 0:
        raise ValueError("the merge needs exact-row tile lists of the video block mask at the "
                         "map's block size")
    if tiles.counts.shape[0] != H:
        raise ValueError(f"tile lists cover {tiles.counts.shape[0]} heads, the map has {H}")
    dt = _attn_dtype(query)
    query, key = _attn_view(query), _attn_view(key)
    lse = lse.contiguous()
    lib = _lib.load()
    check(lib.moddit_sparsity_map_merge(
        query.data_ptr(), key.data_ptr(), lse.data_ptr(), map_inout.data_ptr(), B, H, S, D,
        strides3(*query.stride()[:3]), strides3(*key.stride()[:3]), float(softmax_scale),
        float(log_threshold), int(q_video_offset), int(k_video_offset), int(video_blocks),
        int(block_size), dt, tiles.counts.data_ptr(), tiles.entries.data_ptr(),
        tiles.n_qtiles, tiles.cap, _stream(query)), "moddit_sparsity_map_merge")
    return map_inout


# --------------------------------------------------------------------------------------
# least squares
# --------------------------------------------------------------------------------------
def compute_mts(S_T: torch.Tensor, blocks_per_frame: int) -> torch.Tensor:
    """(H, 3n) fp32 M^T S of an (H,n,n) fp16 or fp32 map."""
    _require_gpu(S_T, what="compute_mts")
    if S_T.ndim != 3 or S_T.shape[1] != S_T.shape[2]:
        raise ValueError(f"S_T must have shape (H, n, n), got {tuple(S_T.shape)}")
    if S_T.dtype == torch.float16:
        dt = _lib.FP16
    elif S_T.dtype == torch.float32:
        dt = _lib.FP32
    else:
        raise TypeError(f"S_T must be float16 or float32, got {S_T.dtype}")
    S_T = S_T.contiguous()
    H, n, _ = S_T.shape
    lib = _lib.load()
    out = torch.empty((H, 3 * n), device=S_T.device, dtype=torch.float32)
    ws = None
    if dt == _lib.FP16 and H > 0:
        ws = torch.empty(lib.moddit_mts_workspace_bytes(H, n), device=S_T.device, dtype=torch.uint8)
    check(lib.moddit_mts(S_T.data_ptr(), dt, H, n, int(blocks_per_frame), _ptr(ws),
                         out.data_ptr(), _stream(S_T)), "moddit_mts")
    return out


def compute_mtm_host(n: int, blocks_per_frame: int, regularization: float) -> torch.Tensor:
    """Closed-form M^T M + lambda I as a CPU float64 (3n, 3n) tensor."""
    F = 3 * n
    out = torch.empty((F, F), dtype=torch.float64)
    check(_lib.load().moddit_mtm_host(int(n), int(blocks_per_frame), float(regularization),
                                      out.data_ptr()), "moddit_mtm_host")
    return out


def fit_schur_host(n: int, blocks_per_frame: int, regularization: float) -> torch.Tensor:
    """Closed-form (n+1, n+1) Schur complement of M^T M + lambda I, CPU float64."""
    out = torch.empty((n + 1, n + 1), dtype=torch.float64)
    check(_lib.load().moddit_fit_schur_host(int(n), int(blocks_per_frame), float(regularization),
                                            out.data_ptr()), "moddit_fit_schur_host")
    return out


def fit_lines(schur_inv: torch.Tensor, mts: torch.Tensor, n: int, blocks_per_frame: int,
              regularization: float) -> torch.Tensor:
    """Ridge fit X (H, 3n) fp32 of M^T S rows `mts` (H, 3n), given S^-1 (n+1, n+1) fp64."""
    _require_gpu(schur_inv, mts, what="fit_lines")
    H, F = mts.shape
    if F != 3 * n or mts.dtype != torch.float32:
        raise ValueError(f"fit_lines: mts must be (H, {3 * n}) fp32, got {tuple(mts.shape)} {mts.dtype}")
    if schur_inv.shape != (n + 1, n + 1) or schur_inv.dtype != torch.float64:
        raise ValueError(f"fit_lines: schur_inv must be ({n + 1}, {n + 1}) fp64")
    schur_inv, mts = schur_inv.contiguous(), mts.contiguous()
    lib = _lib.load()
    ws = torch.empty(max(lib.moddit_fit_workspace_doubles(H, n), 1), device=mts.device,
                     dtype=torch.float64)
    x = torch.empty_like(mts)
    check(lib.moddit_fit_lines(schur_inv.data_ptr(), mts.data_ptr(), x.data_ptr(), ws.data_ptr(),
                               H, int(n), int(blocks_per_frame), float(regularization),
                               _stream(mts)), "moddit_fit_lines")
    return x


# --------------------------------------------------------------------------------------
# line selection / modes / mask
# --------------------------------------------------------------------------------------
def select_lines(x_cur: torch.Tensor, x_last: torch.Tensor, n: int, predict_T: int,
                 top_k: int) -> torch.Tensor:
    """(H, k) int32 ascending indices of the k smallest predicted line scores."""
    _require_gpu(x_cur, x_last, what="select_lines")
    H, F = x_cur.shape
    if F != 3 * n or x_last.shape != x_cur.shape:
        raise ValueError("x_cur/x_last must be (H, 3n)")
    if predict_T is None:
        raise TypeError("predict_T must be an int")
    k = min(int(top_k), 3 * n - 1)
    sel = torch.empty((H, k), device=x_cur.device, dtype=torch.int32)
    check(_lib.load().moddit_select_lines(x_cur.contiguous().data_ptr(),
                                          x_last.contiguous().data_ptr(), H, n, int(predict_T),
                                          int(top_k), sel.data_ptr(), _stream(x_cur)),
          "moddit_select_lines")
    return sel


def check_bd(x: torch.Tensor, mode: torch.Tensor, threshold: float) -> torch.Tensor:
    """In place: mode[h] SPARSE -> BLOCK_DIAGONAL when x[h,-1] <= threshold."""
    _require_gpu(x, mode, what="check_bd")
    H, F = x.shape
    if mode.dtype != torch.uint8 or mode.shape != (H,) or not mode.is_contiguous():
        raise ValueError("mode must be a contiguous (H,) uint8 tensor")
    check(_lib.load().moddit_check_bd(x.contiguous().data_ptr(), H, F, float(threshold),
                                      mode.data_ptr(), _stream(x)), "moddit_check_bd")
    return mode


def _tile_shape(nb: int, block_size: int):
    tokens = nb * block_size
    return (tokens + 127) // 128, nb * (block_size // 64)


def mask_from_lines(sel, mode, *, n, blocks_per_frame, layout, nb, text_blocks, block_size,
                    union_rows=True, want_mask=True, want_tiles=True, grid_origin=0):
    """Bool mask (H,nb,nb) and/or TileList from selected lines (one fused kernel).

    grid_origin: token index of mask row/column 0 (see TileList)."""
    _require_gpu(sel, mode, what="mask_from_lines")
    H = mode.shape[0]
    sel = sel.to(torch.int32).contiguous()
    if sel.ndim != 2 or sel.shape[0] != H:
        raise ValueError("selected lines must be (H, k)")
    dev = sel.device
    mask = torch.empty((H, nb, nb), device=dev, dtype=torch.bool) if want_mask else None
    tiles = None
    nq, cap = _tile_shape(nb, block_size)
    if want_tiles:
        tiles = TileList(torch.empty((H, nq), device=dev, dtype=torch.int32),
                         torch.empty((H, nq, cap), device=dev, dtype=torch.int32),
                         block_size, bool(union_rows), int(grid_origin))
    check(_lib.load().moddit_mask_from_lines(
        sel.data_ptr(), H, sel.shape[1], mode.data_ptr(), int(n), int(blocks_per_frame),
        int(layout), int(nb), int(text_blocks), int(block_size), int(bool(union_rows)),
        _ptr(mask), _ptr(tiles.counts) if tiles else None, _ptr(tiles.entries) if tiles else None,
        nq, cap, _stream(sel)), "moddit_mask_from_lines")
    return mask, tiles


def mask_to_tiles(mask: torch.Tensor, block_size: int, union_rows=True, kv_tiles=None,
                  grid_origin=0) -> TileList:
    """TileList of a bool (H, rows, cols) block mask (strided views are read in place).

    grid_origin: token index of mask row/column 0 (see TileList)."""
    _require_gpu(mask, what="mask_to_tiles")
    if mask.ndim != 3:
        raise ValueError(f"mask must be (H, rows, cols), got {tuple(mask.shape)}")
    if mask.dtype != torch.bool:
        mask = mask != 0
    if mask.stride(2) != 1 or mask.stride(1) < mask.shape[2]:
        mask = mask.contiguous()
    H, rows, cols = mask.shape
    nq = (rows * block_size + 127) // 128
    cap = cols * (block_size // 64)
    if kv_tiles is None:
        kv_tiles = cap
    tiles = TileList(torch.empty((H, nq), device=mask.device, dtype=torch.int32),
                     torch.empty((H, nq, cap), device=mask.device, dtype=torch.int32),
                     block_size, bool(union_rows), int(grid_origin))
    check(_lib.load().moddit_mask_to_tiles(mask.data_ptr(), H, rows, cols, mask.stride(0),
                                           mask.stride(1), int(block_size), int(bool(union_rows)),
                                           int(kv_tiles), tiles.counts.data_ptr(),
                                           tiles.entries.data_ptr(), nq, cap, _stream(mask)),
          "moddit_mask_to_tiles")
    return tiles


def refresh_merge(prev: torch.Tensor, cur: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """where(mask, cur, prev) over (H,n,n) fp16 maps; mask may be a strided bool view."""
    _require_gpu(prev, cur, mask, what="refresh_merge")
    if prev.shape != cur.shape or prev.ndim != 3 or tuple(mask.shape) != tuple(prev.shape):
        raise ValueError("refresh_merge: prev/cur/mask must share shape (H, n, n)")
    if prev.dtype != torch.float16 or cur.dtype != torch.float16:
        raise TypeError("refresh_merge: maps must be float16")
    if mask.dtype != torch.bool:
        raise TypeError("refresh_merge: mask must be bool")
    if mask.stride(2) != 1:
        mask = mask.contiguous()
    prev, cur = prev.contiguous(), cur.contiguous()
    H, n, _ = prev.shape
    out = torch.empty_like(prev)
    check(_lib.load().moddit_refresh_merge(prev.data_ptr(), cur.data_ptr(), mask.data_ptr(),
                                           mask.stride(0), mask.stride(1), H, n, out.data_ptr(),
                                           _stream(prev)), "moddit_refresh_merge")
    return out
