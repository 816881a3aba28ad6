"""MI355X-native (gfx950) MOD-DiT sparse-attention hot path.

Layers:
  csrc/*.hip        HIP kernels + the C ABI of include/moddit.h -> libmoddit.so
  _lib.py           ctypes binding (loads libmoddit.so from this directory, no fallback)
  ops.py            torch-facing wrappers (validation, output allocation, current stream)
  flash_sparsity.py flash_attn_with_sparsity_map / cuda_sparsity_map drop-ins
  lstsq.py          solve_lstsq drop-in (closed-form M^T M, cached inverse, HIP fit)
  attn_mask.py      SparseAttentionWithMap and the rest of MoD/mod/attn_mask.py's API
  state.py          create_adaptive_mask_state / init_warmup_state / is_warmup_complete
"""
from . import _lib, ops
from .attn_mask import (
    AttentionSparseEngine,
    HeadModes,
    SparseAttentionWithMap,
    check_bd_values,
    choose_topk_lines,
    extract_attention_features,
    generate_mask_from_lines,
    predict_mask_from_warmup,
    update_warmup,
)
from .flash_sparsity import (_validate_inputs, cuda_sparsity_map, flash_attn_with_sparsity_map,
                             padded_grid)
from .lstsq import compute_mtm, compute_mts, solve_lstsq
from .ops import TileList
from .state import create_adaptive_mask_state, init_warmup_state, is_warmup_complete

__all__ = [
    "AttentionSparseEngine", "HeadModes", "SparseAttentionWithMap", "TileList",
    "check_bd_values", "choose_topk_lines", "compute_mtm", "compute_mts",
    "create_adaptive_mask_state", "cuda_sparsity_map", "extract_attention_features",
    "flash_attn_with_sparsity_map", "generate_mask_from_lines", "init_warmup_state",
    "is_warmup_complete", "padded_grid", "predict_mask_from_warmup", "solve_lstsq",
    "update_warmup",
]
