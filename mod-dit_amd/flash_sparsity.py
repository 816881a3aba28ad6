"""Dense flash attention plus the exact video x video block sparsity map.

Drop-in for MoD/mod/triton_flash_sparsity.py (public entry `flash_attn_with_sparsity_map`,
:274-341) and MoD/mod/cuda_flash_sparsity.py (`cuda_sparsity_map`, :71-99):

  pass 1  dense attention -> O and the natural-log row LSE (HIP MFMA kernel)
  pass 2  replay of the video x video QK tiles, counting probabilities below the
          threshold: count(bf16(q*scale).k < lse + ln(threshold)) / block_size^2 -> fp16

Two kernels on purpose: the single-kernel form (`ops.flash_fwd_map`, same results) runs
its replay sweep at the attention kernel's occupancy (two waves per SIMD) and is slower
on gfx950 than the standalone replay kernel at four.

There is a single backend (gfx950 HIP); the reference's Triton fallback and its
MOD_DIT_SPARSITY_BACKEND switch have no counterpart here.
"""
from __future__ import annotations

import math
from typing import Tuple

import torch

from . import ops


def padded_grid(text_token_num: int, video_token_num: int, block_size: int) -> Tuple[int, int, int]:
    """Block grid of a text-first (CogVideoX) sequence: (text_blocks, video_blocks, origin).

    Text and video each start on a block boundary: the grid begins `-origin` virtual
    tokens before token 0 so that the text fills ceil(text/bs) blocks ending exactly where
    the video begins, and the video fills ceil(video/bs) blocks, the last one padded past
    the sequence end. Virtual tokens are never attended to and produce no output. For
    block-aligned text and video this is the reference's own grid (origin 0). The
    reference rejects unaligned shapes (MoD/mod/triton_flash_sparsity.py:157-160).
    """
    tb = -(-text_token_num // block_size)
    vb = -(-video_token_num // block_size)
    return tb, vb, text_token_num - tb * block_size


def _video_layout(model_type: str, sequence_length: int, video_token_num: int,
                  text_token_num: int, block_size: int) -> Tuple[int, int, int]:
    """(video_blocks, q_offset, k_offset); MoD/mod/triton_flash_sparsity.py:101-120.

    cogvideox counts a trailing partial video block (see `padded_grid`)."""
    if model_type == "wan":
        if video_token_num not in (0, sequence_length):
            raise ValueError(
                f"wan expects video_token_num to be 0 or S={sequence_length}, got {video_token_num}"
            )
        return sequence_length // block_size, 0, 0
    if model_type == "hunyuan":
        return video_token_num // block_size, 0, 0
    if model_type == "cogvideox":
        return -(-video_token_num // block_size), text_token_num, text_token_num
    raise ValueError(
        f"Unknown model_type: {model_type}, expected 'wan', 'hunyuan', or 'cogvideox'"
    )


def _validate_inputs(query, key, value, threshold, block_size: int, model_type: str,
                     video_token_num: int, text_token_num: int):
    """Argument checks of MoD/mod/triton_flash_sparsity.py:123-178 (same errors/messages).

    Returns (threshold_value, video_blocks, q_offset, k_offset).
    """
    if query.ndim != 4:
        raise ValueError(f"query must have shape [B, H, S, D], got {tuple(query.shape)}")
    if key.shape != query.shape or value.shape != query.shape:
        raise ValueError("query, key, and value must have identical [B, H, S, D] shapes")
    if not query.is_cuda or not key.is_cuda or not value.is_cuda:
        raise ValueError("query, key, and value must be CUDA tensors")
    if query.device != key.device or query.device != value.device:
        raise ValueError("query, key, and value must be on the same CUDA device")
    if query.dtype != key.dtype or query.dtype != value.dtype:
        raise ValueError("query, key, and value must have the same dtype")
    if query.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"expected float16 or bfloat16 inputs, got {query.dtype}")
    if block_size not in (64, 128):
        raise ValueError(f"block_size must be 64 or 128, got {block_size}")

    _, _, sequence_length, head_dim = query.shape
    if head_dim not in (64, 128):
        raise ValueError(f"head_dim must be 64 or 128, got {head_dim}")
    if model_type == "wan":
        video_tokens = sequence_length
    else:
        if video_token_num <= 0:
            raise ValueError(f"video_token_num must be positive for {model_type}")
        video_tokens = video_token_num
    if video_tokens % block_size:
        # Text-first sequences whose video ends the sequence get a padded block grid
        # (`padded_grid`); every other layout keeps the reference's rule.
        if not (model_type == "cogvideox"
                and text_token_num + video_token_num == sequence_length):
            raise ValueError(
                f"video_token_num={video_tokens} must be divisible by block_size={block_size}"
            )
    if text_token_num < 0:
        raise ValueError("text_token_num must be non-negative")
    if model_type in ("hunyuan", "cogvideox") and video_token_num + text_token_num > sequence_length:
        raise ValueError("video and text regions exceed the sequence length")

    if torch.is_tensor(threshold):
        if threshold.numel() != 1:
            raise ValueError("threshold tensor must contain one element")
        threshold_value = float(threshold.detach().item())
    else:
        threshold_value = float(threshold)
    if math.isnan(threshold_value):
        raise ValueError("threshold must not be NaN")

    video_blocks, q_offset, k_offset = _video_layout(
        model_type, sequence_length, video_token_num, text_token_num, block_size
    )
    return threshold_value, video_blocks, q_offset, k_offset


def log_threshold(threshold_value: float) -> float:
    """ln(threshold), or -inf for a non-positive threshold (:328)."""
    return math.log(threshold_value) if threshold_value > 0 else float("-inf")


def cuda_sparsity_map(query, key, lse, *, softmax_scale, log_threshold, q_video_offset,
                      k_video_offset, video_blocks, block_size):
    """Replay pass with the signature of MoD/mod/cuda_flash_sparsity.py:71-99."""
    if block_size not in (64, 128):
        raise RuntimeError("block_size must be 64 or 128")
    if query.shape[-1] not in (64, 128):
        raise RuntimeError("head_dim must be 64 or 128")
    if video_blocks <= 0:
        raise RuntimeError("video_blocks must be positive")
    return ops.sparsity_map(query, key, lse, softmax_scale=softmax_scale,
                            log_threshold=log_threshold, q_video_offset=q_video_offset,
                            k_video_offset=k_video_offset, video_blocks=video_blocks,
                            block_size=block_size)


@torch.no_grad()
def flash_attn_with_sparsity_map(query, key, value, threshold, block_size: int,
                                 model_type: str = "hunyuan", video_token_num: int = 0,
                                 text_token_num: int = 0):
    """Attention output (B,H,S,D) and fp16 sparsity map (B,H,video_blocks,video_blocks)."""
    threshold_value, video_blocks, q_off, k_off = _validate_inputs(
        query, key, value, threshold, block_size, model_type, video_token_num, text_token_num
    )
    D = query.shape[-1]
    sm_scale = D ** -0.5
    out, lse = ops.flash_fwd(query, key, value, softmax_scale=sm_scale, return_lse=True)
    sparsity = ops.sparsity_map(query, key, lse, softmax_scale=sm_scale,
                                log_threshold=log_threshold(threshold_value),
                                q_video_offset=q_off, k_video_offset=k_off,
                                video_blocks=video_blocks, block_size=block_size)
    return out, sparsity
