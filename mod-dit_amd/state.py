"""Per-layer state of the MOD-DiT step machine (MoD/mod/state.py:3-71).

Same keys and validation as the reference, plus keys of this build:
  'tile_rows'  'union' (default): the attention engine runs each mask row pair as one
               128-row query tile over the union of both rows' key blocks, as the
               reference's engine does (MoD/mod/attn_mask.py:299-303);
               'exact': 64x64 blocks are honoured exactly.
  'precision'  arithmetic of the engine's attention on sparse steps and on
               use_dense calls: 'bf16' (default; bf16 MFMA, fp32 softmax) or 'int8'
               (int8 Q.K^T with smoothed K, fp8 e4m3 P.V: the SageAttention2-style
               numerics of the reference's engine, whose dense branch calls sageattn and
               sparse branch block_sparse_sage2_attn_cuda, MoD/mod/attn_mask.py:271-276,
               306,312-317). Map steps always run bf16.
  '_tiles'     the attention tile lists built together with 'mask'.
"""
from __future__ import annotations

from typing import Dict

_SPARSE_TYPES = {"full", "mod-dit", "radial", "svg", "spargeattn"}


def init_warmup_state() -> Dict:
    """Empty algorithm state (MoD/mod/state.py:3-22)."""
    return {
        "features_history": None,
        "current_steps": 0,
        "prev_full_maps": None,
        "prediction_features": {},
        "mask": None,
        "sparse_id": None,
    }


def create_adaptive_mask_state(
    model_type: str,
    num_heads: int,
    video_token_num: int,
    text_token_num: int,
    tokens_per_frame: int,
    num_frames: int,
    warmup_steps: int = 12,
    top_k: int = 10,
    predict_T: int = 5,
    threshold: float = 1.5e-4,
    block_size: int = 128,
    use_cuda: bool = True,
    sparse_type: str = "mod-dit",
    tile_rows: str = "union",
    precision: str = "bf16",
) -> Dict:
    """Build a layer state (MoD/mod/state.py:24-68)."""
    state = init_warmup_state()
    state["model_type"] = model_type
    state["num_heads"] = num_heads
    state["video_token_num"] = video_token_num
    state["text_token_num"] = text_token_num
    state["blocks_per_frame"] = tokens_per_frame // block_size
    state["frame_size"] = tokens_per_frame
    state["num_frames"] = num_frames
    state["warmup_steps"] = warmup_steps
    state["top_k"] = top_k
    state["threshold"] = float(threshold)
    state["block_size"] = block_size
    state["predict_T"] = predict_T
    state["use_cuda"] = use_cuda
    if sparse_type not in _SPARSE_TYPES:
        raise ValueError(
            f"{sparse_type} not support , only support [full mod-dit, radial, svg, spargeattn]"
        )
    state["sparse_type"] = sparse_type
    if tile_rows not in ("union", "exact"):
        raise ValueError(f"tile_rows must be 'union' or 'exact', got {tile_rows!r}")
    state["tile_rows"] = tile_rows
    if precision not in ("bf16", "int8"):
        raise ValueError(f"precision must be 'bf16' or 'int8', got {precision!r}")
    state["precision"] = precision
    return state


def is_warmup_complete(warmup_state: Dict) -> bool:
    """MoD/mod/state.py:70-72."""
    return warmup_state["current_steps"] >= warmup_state["warmup_steps"]
