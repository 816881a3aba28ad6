"""MOD-DiT sparse-attention step machine on gfx950 (drop-in for MoD/mod/attn_mask.py).

Public functions keep the reference's names, signatures and return values:
  SparseAttentionWithMap (:567-729)   per-call warmup / predict / refresh / sparse machine
  AttentionSparseEngine (:266-331)    dense or block-sparse attention from a block mask
  update_warmup (:117-146), extract_attention_features (:76-115)
  check_bd_values (:336-349), choose_topk_lines (:351-370)
  predict_mask_from_warmup (:373-436), generate_mask_from_lines (:440-559)

Differences that are deliberate:
  * no host synchronisation on the path: head modes stay on the device (HeadModes
    behaves like the reference's list of strings when read), the block-diagonal test,
    line selection, mask construction and the refresh merge are device kernels, and the
    engine never calls mask.all(): an all-True mask runs block-sparse like any other (with
    a Hunyuan padding mask its video queries then also see the padded keys of the last
    64-key tile, as in the reference's sparse branch, where its dense branch would stop at
    the valid keys);
  * selected lines come back in ascending index order (the reference's
    topk(sorted=False) order is unspecified); ties at the k-th value go to the lower
    index;
  * the mask kernel also emits the attention tile lists, so sparse steps do not
    convert the mask again;
  * refresh steps replay the sparsity map only at the blocks the current mask keeps
    and write them into a copy of the previous map: the reference's full replay followed
    by where(mask == False, prev, current) gives the same map, bit for bit;
  * sparse types other than 'mod-dit' ('radial', 'spargeattn') call third-party kernels
    in the reference and raise NotImplementedError here;
  * the engine's arithmetic is bf16 by default; the state key 'precision' = 'int8'
    selects the reference engine's quantised (SageAttention2-style) numerics.
"""
from __future__ import annotations

import logging
from collections.abc import Sequence
from typing import Dict, List, Optional, Tuple

import torch

from . import _lib, ops
from .flash_sparsity import (_validate_inputs, flash_attn_with_sparsity_map, log_threshold,
                             padded_grid)
from .lstsq import solve_lstsq
from .state import is_warmup_complete

_MODE_CODES = {"sparse": _lib.MODE_SPARSE, "block_diagonal": _lib.MODE_BLOCK_DIAGONAL,
               "full": _lib.MODE_FULL}
_MODE_NAMES = {v: k for k, v in _MODE_CODES.items()}
_LAYOUTS = {"wan": _lib.LAYOUT_WAN, "hunyuan": _lib.LAYOUT_HUNYUAN,
            "cogvideox": _lib.LAYOUT_COGVIDEOX}


class HeadModes(Sequence):
    """Per-head mask modes kept as a device uint8 tensor.

    Reads like the reference's list of 'sparse' / 'block_diagonal' / 'full' strings; the
    device-to-host copy happens only when an element is actually read.
    """

    def __init__(self, codes: torch.Tensor):
        self.codes = codes
        self._names: Optional[List[str]] = None

    def _host(self) -> List[str]:
        if self._names is None:
            self._names = [_MODE_NAMES[int(c)] for c in self.codes.tolist()]
        return self._names

    def __len__(self):
        return self.codes.shape[0]

    def __getitem__(self, i):
        return self._host()[i]

    def __eq__(self, other):
        return list(self) == list(other)

    def __repr__(self):
        return f"HeadModes({self._host()!r})"


def _mode_tensor(mode, num_heads: int, device) -> torch.Tensor:
    if isinstance(mode, HeadModes):
        return mode.codes
    if torch.is_tensor(mode):
        return mode.to(device=device, dtype=torch.uint8)
    codes = [_MODE_CODES.get(m, _lib.MODE_SPARSE) for m in list(mode)]
    if len(codes) != num_heads:
        raise ValueError(f"mode has {len(codes)} entries for {num_heads} heads")
    return torch.tensor(codes, dtype=torch.uint8, device=device)


# ======================================================================================
# feature extraction / warmup bookkeeping
# ======================================================================================
def extract_attention_features(warmup_state: Dict, S_T: torch.Tensor, blocks_per_frame: int,
                               layer_idx: int = 0, regularization: float = 1,
                               use_cuda: bool = True) -> Dict[str, torch.Tensor]:
    """Fit the line model to S_T (H, n, n); MoD/mod/attn_mask.py:76-115 (lambda = 1)."""
    num_heads, n = S_T.shape[0], S_T.shape[1]
    assert S_T.shape == (num_heads, n, n), f"S_T shape mismatch: {S_T.shape} vs ({num_heads}, {n}, {n})"
    return solve_lstsq(warmup_state=warmup_state, S_T=S_T, step=warmup_state["current_steps"],
                       layer_idx=layer_idx, blocks_per_frame=blocks_per_frame,
                       regularization=regularization, use_cuda=use_cuda)


def update_warmup(warmup_state: Dict, step: int, block_sparse_map: torch.Tensor):
    """MoD/mod/attn_mask.py:117-146."""
    if step == warmup_state["warmup_steps"] - 2:
        warmup_state["features_history"] = []
        warmup_state["current_steps"] = step
        warmup_state["prev_full_maps"] = block_sparse_map
    features = extract_attention_features(warmup_state=warmup_state, S_T=block_sparse_map,
                                          blocks_per_frame=warmup_state["blocks_per_frame"],
                                          use_cuda=warmup_state["use_cuda"])
    warmup_state["features_history"].append(features)
    warmup_state["current_steps"] = step + 1
    warmup_state["prev_full_maps"] = block_sparse_map


# ======================================================================================
# mask prediction
# ======================================================================================
def check_bd_values(values: torch.Tensor, mode: List[str], threshold: float = -7.5e-2):
    """Host-list form of MoD/mod/attn_mask.py:336-349 (reads `values` on the host).

    The step machine uses the device kernel (ops.check_bd) instead.
    """
    last = values[:, -1].tolist()
    for i in range(values.shape[0]):
        if mode[i] == "sparse" and last[i] <= threshold:
            mode[i] = "block_diagonal"
    return mode


def _x_of(features: Dict[str, torch.Tensor]) -> torch.Tensor:
    x = features.get("_x")
    if x is not None:
        return x
    d, c, b = features["d"], features["c"], features["b_d"]
    return torch.cat([d, c * 2, b.reshape(-1, 1)], dim=1).to(torch.float32).contiguous()


def _select_i32(history, top_k: int, predict_T) -> torch.Tensor:
    x_last, x_cur = _x_of(history[-2]), _x_of(history[-1])
    n = x_cur.shape[1] // 3
    return ops.select_lines(x_cur, x_last, n, predict_T, top_k)


def choose_topk_lines(history: List[Dict[str, torch.Tensor]], top_k: int = 10,
                      predict_T: int = None) -> torch.Tensor:
    """k smallest of cat(pred_c, pred_d) per head; MoD/mod/attn_mask.py:351-370.

    Returns (H, k) int64 indices (index < n: column, else diagonal offset idx-n-(n-1)),
    in ascending order.
    """
    return _select_i32(history, top_k, predict_T).long()


def _grid(warmup_state: Dict, seq_len: int):
    """(text_blocks, video_blocks, mask_blocks, origin) of the attention block grid.

    wan / hunyuan / other: the reference's grid (block b = tokens [b*bs, (b+1)*bs)).
    cogvideox: text-first with text and video each starting on a block boundary, the
    grid shifted by `origin` <= 0 tokens when the text is not block-aligned
    (flash_sparsity.padded_grid)."""
    bs = warmup_state["block_size"]
    model_type = warmup_state.get("model_type")
    if model_type == "cogvideox":
        tb, vb, origin = padded_grid(warmup_state["text_token_num"],
                                     warmup_state["video_token_num"], bs)
        return tb, vb, tb + vb, origin
    tb = warmup_state["text_token_num"] // bs
    vb = warmup_state["video_token_num"] // bs
    return tb, vb, seq_len // bs, 0


def _generate_mask_and_tiles(warmup_state: Dict, num_heads: int, n: int, blocks_per_frame: int,
                             selected_lines, mode, device, want_tiles=True):
    block_size = warmup_state["block_size"]
    text_block_num, video_block_num, block_num, origin = _grid(warmup_state, n)
    model_type = warmup_state.get("model_type")
    layout = _LAYOUTS.get(model_type, _lib.LAYOUT_OTHER)
    if layout == _lib.LAYOUT_WAN:
        nb = video_block_num
    else:
        nb = block_num
    if layout == _lib.LAYOUT_COGVIDEOX and block_num * block_size + origin < n:
        raise RuntimeError(
            f"cogvideox mask: text {warmup_state['text_token_num']} + video "
            f"{warmup_state['video_token_num']} tokens do not cover the sequence of {n}"
        )
    if layout == _lib.LAYOUT_HUNYUAN and block_num < video_block_num:
        raise RuntimeError("hunyuan mask: video blocks exceed the sequence")
    if not torch.is_tensor(selected_lines):
        selected_lines = torch.as_tensor(selected_lines)
    selected_lines = selected_lines.to(device=device)
    if selected_lines.dim() == 1:
        selected_lines = selected_lines.unsqueeze(1)
    modes = _mode_tensor(mode, num_heads, device)
    union = warmup_state.get("tile_rows", "union") == "union"
    n_video = max(video_block_num, 1)
    if block_size == 128 and origin <= -64:
        want_tiles = False  # the engine runs such grids on 64-token tiles (_as_64_token_grid)
    return ops.mask_from_lines(selected_lines, modes, n=n_video,
                               blocks_per_frame=max(int(blocks_per_frame), 1), layout=layout,
                               nb=nb, text_blocks=text_block_num, block_size=block_size,
                               union_rows=union, want_mask=True, want_tiles=want_tiles,
                               grid_origin=origin)


def generate_mask_from_lines(warmup_state: Dict, num_heads: int, n: int, blocks_per_frame: int,
                             selected_lines, mode, device) -> torch.Tensor:
    """Bool block mask from selected lines; MoD/mod/attn_mask.py:440-559."""
    mask, _ = _generate_mask_and_tiles(warmup_state, num_heads, n, blocks_per_frame,
                                       selected_lines, mode, device, want_tiles=False)
    return mask


def predict_mask_from_warmup(warmup_state: Dict, n: int, top_k: int = 10,
                             layer_idx: int = 0) -> Dict:
    """First mask after warmup; MoD/mod/attn_mask.py:373-436."""
    num_heads = warmup_state["num_heads"]
    blocks_per_frame = warmup_state["blocks_per_frame"]
    if not is_warmup_complete(warmup_state):
        device = torch.device("cuda") if torch.cuda.is_available() else torch.device("cpu")
        nb = _grid(warmup_state, n)[2]
        return {
            "mode": ["full"] * num_heads,
            "block_diagonal": [False] * num_heads,
            "selected_lines": [],
            "mask": torch.ones(num_heads, nb, nb, dtype=torch.bool, device=device),
        }
    history = warmup_state["features_history"]
    x_cur = _x_of(history[-1])
    device = x_cur.device
    modes = torch.zeros(num_heads, dtype=torch.uint8, device=device)
    ops.check_bd(x_cur, modes, threshold=1.0)
    mode = HeadModes(modes)
    selected = _select_i32(history, top_k, warmup_state.get("predict_T", None))
    mask, tiles = _generate_mask_and_tiles(warmup_state, num_heads, n, blocks_per_frame,
                                           selected, mode, device)
    return {"mode": mode, "selected_lines": selected.long(), "mask": mask, "_tiles": tiles}


# ======================================================================================
# attention engine
# ======================================================================================
def _log_sparsity(logger, layer_idx: int, mask: torch.Tensor) -> None:
    # The value needs a device read; only pay for it when the message is emitted.
    if logger is not None and logger.isEnabledFor(logging.INFO):
        logger.info(f"Layer {layer_idx}, Mask Sparsity: {1 - mask.float().mean():.3%}")


def _kv_valid(pre_defined_mask: torch.Tensor) -> int:
    """Number of valid keys: the first row of the processor's padding mask.

    Like the reference (MoD/mod/attn_mask.py:270,310), this reads one value on the host.
    """
    return int(pre_defined_mask[0].sum().item())


def _as_64_token_grid(mask: torch.Tensor, seq_len: int, origin: int):
    """(mask64, origin64) for a 128-token block mask on a grid starting `origin` in
    [-127, -64] tokens before token 0.

    The kernels run 64-key tiles on grids that start in (-64, 0]. This grid is the 64-token
    grid 64 tokens later whose first tile row and column are all padding: each 128-block
    row and column becomes two 64-token ones, the first of each is dropped, and the rest is
    cut to the tiles the sequence reaches. Run with exact rows, every 64-row half keeps its
    128-block row's mask, so the token-level mask is the same."""
    origin64 = origin + 64
    n64 = -(-(seq_len - origin64) // 64)
    m64 = mask.repeat_interleave(2, dim=1).repeat_interleave(2, dim=2)
    return m64[:, 1:n64 + 1, 1:n64 + 1], origin64


def _engine(query, key, value, mask, tiles, pre_defined_mask, video_token_num, block_size,
            union_rows, grid_origin=0, precision="bf16"):
    if mask.dim() == 2:
        mask = mask.unsqueeze(0).expand(query.shape[1], -1, -1)
    q8 = precision == "int8"
    if pre_defined_mask is None:
        if block_size == 128 and grid_origin <= -64:
            m64, grid_origin = _as_64_token_grid(mask, query.shape[2], grid_origin)
            tiles = ops.mask_to_tiles(m64, 64, union_rows=False, grid_origin=grid_origin)
        elif tiles is None:
            tiles = ops.mask_to_tiles(mask, block_size, union_rows=union_rows,
                                      grid_origin=grid_origin)
        if q8:
            qz = ops.quantize_qkv(query, key, value, grid_origin=grid_origin)
            out, _ = ops.block_sparse_fwd_q8(qz, tiles)
        else:
            out, _ = ops.block_sparse_fwd(query, key, value, tiles)
        return out
    # Hunyuan layout (MoD/mod/attn_mask.py:310-331): video queries run block-sparse over the
    # key tiles below ceil(valid/64) (so up to 63 padded text keys of the last tile take
    # part, as in the reference); text queries attend densely to the valid keys.
    S = query.shape[2]
    kv = _kv_valid(pre_defined_mask)
    kv_tiles = (kv + 63) // 64
    video = int(video_token_num)
    if video % block_size:
        raise ValueError(f"video_token_num={video} must be divisible by block_size={block_size}")
    out = torch.empty_like(query, memory_format=torch.contiguous_format)
    if video > 0:
        vt = ops.mask_to_tiles(mask[:, :video // block_size, :], block_size, union_rows=union_rows,
                               kv_tiles=kv_tiles)
        if q8:  # the whole sequence is quantised, as the reference passes the full key/value
            qz = ops.quantize_qkv(query, key, value)
            ops.block_sparse_fwd_q8(qz, vt, out=out[:, :, :video], q_len=video)
        else:
            kv_len = min(S, kv_tiles * 64)
            ops.block_sparse_fwd(query[:, :, :video], key[:, :, :kv_len], value[:, :, :kv_len], vt,
                                 out=out[:, :, :video])
    if video < S:
        ops.flash_fwd(query[:, :, video:], key[:, :, :kv], value[:, :, :kv], return_lse=False,
                      out=out[:, :, video:])
    return out


def AttentionSparseEngine(query, key, value, mask, pre_defined_mask=None, video_token_num=0,
                          block_size=128, union_rows: bool = True, precision: str = "bf16"):
    """Block-sparse attention under a bool block mask; MoD/mod/attn_mask.py:266-331.

    union_rows=True executes each pair of 64-row mask rows as one 128-row query tile over
    the union of their key blocks, which is what the reference engine runs (:299-303).
    precision='int8' runs the int8 Q.K^T / fp8 P.V kernels on the video queries (the
    reference's block_sparse_sage2_attn_cuda numerics, :306,312-317); text queries of a
    padded (Hunyuan) layout stay bf16, as the reference's flashinfer call is (:319-330).
    """
    if precision not in ("bf16", "int8"):
        raise ValueError(f"precision must be 'bf16' or 'int8', got {precision!r}")
    return _engine(query, key, value, mask, None, pre_defined_mask, video_token_num,
                   block_size, union_rows, precision=precision)


def _dense_engine(query, key, value, pre_defined_mask, video_token_num=0, precision="bf16"):
    """All-True mask: every query attends to the valid keys (MoD/mod/attn_mask.py:268-295).

    bf16: one dense call (the reference's video/text split there is the same computation).
    int8: the video queries run the int8/fp8 kernels over the valid keys, as the
    reference's sageattn call does (:271-276, K smoothed by the mean of those keys); the
    text queries of a padded layout stay bf16, as its flashinfer call is (:278-290).
    """
    kv = key.shape[2] if pre_defined_mask is None else _kv_valid(pre_defined_mask)
    if precision != "int8":
        out, _ = ops.flash_fwd(query, key[:, :, :kv], value[:, :, :kv], return_lse=False)
        return out
    if pre_defined_mask is None:
        out, _ = ops.flash_fwd_q8(ops.quantize_qkv(query, key, value), return_lse=False)
        return out
    S = query.shape[2]
    video = int(video_token_num)
    if not 0 <= video <= kv:
        raise ValueError(f"video_token_num={video} must lie in [0, valid keys={kv}]")
    if video % 32:
        # Q is quantised in 32-row blocks: a block straddling the video/text boundary would
        # take its scale from text rows too, where the reference quantises query[:video]
        raise ValueError(f"video_token_num={video} must be a multiple of 32 for the int8 path")
    out = torch.empty_like(query, memory_format=torch.contiguous_format)
    if video > 0:
        # rows video..kv-1 are text queries (every 32-row block lies on one side of the
        # boundary, so the video rows' scales are those of query[:video] alone); the bf16
        # call below overwrites them
        qz = ops.quantize_qkv(query[:, :, :kv], key[:, :, :kv], value[:, :, :kv])
        ops.flash_fwd_q8(qz, return_lse=False, out=out[:, :, :kv])
    if video < S:
        ops.flash_fwd(query[:, :, video:], key[:, :, :kv], value[:, :, :kv], return_lse=False,
                      out=out[:, :, video:])
    return out


# ======================================================================================
# step machine
# ======================================================================================
def _video_part(warmup_state: Dict, mask: torch.Tensor) -> torch.Tensor:
    bs = warmup_state["block_size"]
    mt = warmup_state["model_type"]
    if mt == "cogvideox":
        t = _grid(warmup_state, 0)[0]
        return mask[:, t:, t:]
    if mt == "hunyuan":
        v = warmup_state["video_token_num"] // bs
        return mask[:, :v, :v]
    return mask


def _refresh_map_step(query, key, value, warmup_state: Dict, current_mask: torch.Tensor):
    """Dense attention and the merged map of a refresh step (MoD/mod/attn_mask.py:659-675).

    The reference computes the whole map with flash_attn_with_sparsity_map and keeps it
    only where the current (video) mask is True: where(mask == False, prev, current).
    Here the replay runs over the mask's active blocks only, writing them into a copy of
    the previous map; the result is the same map, bit for bit."""
    bs = warmup_state["block_size"]
    thr, video_blocks, q_off, k_off = _validate_inputs(
        query, key, value, warmup_state["threshold"], bs, warmup_state["model_type"],
        warmup_state["video_token_num"], warmup_state["text_token_num"])
    sm_scale = query.shape[-1] ** -0.5
    out, lse = ops.flash_fwd(query, key, value, softmax_scale=sm_scale, return_lse=True)
    tiles = ops.mask_to_tiles(current_mask, bs, union_rows=False)
    merged = warmup_state["prev_full_maps"].clone(memory_format=torch.contiguous_format)
    ops.sparsity_map_merge(query, key, lse, tiles, merged.unsqueeze(0), softmax_scale=sm_scale,
                           log_threshold=log_threshold(thr), q_video_offset=q_off,
                           k_video_offset=k_off, video_blocks=video_blocks, block_size=bs)
    return out, merged


def SparseAttentionWithMap(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    warmup_state: Dict,
    logger: logging.Logger,
    pre_defined_mask: Optional[torch.Tensor] = None,
    current_step: int = 0,
    layer_idx: int = 0,
    use_dense: bool = False,
    in_test: bool = False,
    **kwargs,
):
    """One attention call of the MOD-DiT schedule; MoD/mod/attn_mask.py:567-729.

    Returns (output (1,H,S,D), mask_info) with the same branch-dependent mask_info as
    the reference: a dict on dense and sparse steps, the next-step mask (or None) on
    warmup steps.
    """
    if use_dense:
        output = _dense_engine(query, key, value, pre_defined_mask,
                               video_token_num=warmup_state.get("video_token_num", 0),
                               precision=warmup_state.get("precision", "bf16"))
        return output, {"mode": "warmup", "mask": None}
    sparse_type = warmup_state["sparse_type"]
    if sparse_type != "mod-dit":
        raise NotImplementedError(f"sparse_type {sparse_type!r} is not part of this build")

    num_heads = query.size(1)
    seq_len = query.size(2)
    W = warmup_state["warmup_steps"]
    if current_step < W:
        if current_step < W - 2:
            raise RuntimeError(
                "SparseAttentionWithMap: steps before warmup_steps-2 run dense attention; "
                "call with use_dense=True (the processors' use_dense gate)"
            )
        output, block_sparse_map = flash_attn_with_sparsity_map(
            query, key, value, threshold=warmup_state["threshold"],
            block_size=warmup_state["block_size"], model_type=warmup_state["model_type"],
            video_token_num=warmup_state["video_token_num"],
            text_token_num=warmup_state["text_token_num"])
        update_warmup(warmup_state, current_step, block_sparse_map.squeeze(0))
        if current_step == W - 1:
            info = predict_mask_from_warmup(warmup_state, seq_len, top_k=warmup_state["top_k"],
                                            layer_idx=layer_idx)
            warmup_state["mask"] = info["mask"]
            warmup_state["_tiles"] = info.get("_tiles")
            warmup_state["_tiles_for"] = info["mask"]
            _log_sparsity(logger, layer_idx, warmup_state["mask"])
            warmup_state["mode"] = info["mode"]
        return output, warmup_state["mask"]

    if warmup_state.get("mask", None) is None:
        raise RuntimeError("SparseAttentionWithMap: no mask was predicted during warmup")
    T = warmup_state["predict_T"]
    if (current_step - W) % T == T - 1:
        current_mask = _video_part(warmup_state, warmup_state["mask"])
        output, warmup_state["prev_full_maps"] = _refresh_map_step(
            query, key, value, warmup_state, current_mask)
        features = extract_attention_features(
            warmup_state=warmup_state, S_T=warmup_state["prev_full_maps"], layer_idx=layer_idx,
            blocks_per_frame=warmup_state["blocks_per_frame"], use_cuda=warmup_state["use_cuda"])
        warmup_state["features_history"].append(features)
        warmup_state["features_history"].pop(0)
        selected = _select_i32(warmup_state["features_history"], warmup_state["top_k"],
                               warmup_state.get("predict_T", None))
        next_mask, tiles = _generate_mask_and_tiles(
            warmup_state, num_heads, seq_len, warmup_state["blocks_per_frame"], selected,
            warmup_state["mode"], device=query.device)
        warmup_state["mask"] = next_mask
        warmup_state["_tiles"] = tiles
        warmup_state["_tiles_for"] = next_mask
    else:
        mask = warmup_state["mask"]
        union = warmup_state.get("tile_rows", "union") == "union"
        tiles = warmup_state.get("_tiles") if warmup_state.get("_tiles_for") is mask else None
        if tiles is not None and tiles.union_rows != union:
            tiles = None  # built for the other row granularity; the engine rebuilds them
        output = _engine(query, key, value, mask, tiles, pre_defined_mask,
                         warmup_state.get("video_token_num", 0), warmup_state["block_size"],
                         union,
                         grid_origin=_grid(warmup_state, seq_len)[3],
                         precision=warmup_state.get("precision", "bf16"))
    return output, {"mask": warmup_state["mask"]}
