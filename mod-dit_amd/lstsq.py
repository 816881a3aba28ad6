"""Ridge least-squares fit of the line model (drop-in for MoD/mod/cuda_lstsq.py:42-270).

min_X ||S - M X||^2 + lambda ||X||^2 with M's columns = [2n-1 block diagonals, n block
columns, 1 frame-block-diagonal] over an (n, n) block map. M^T M depends only on
(n, blocks_per_frame, lambda), and its diagonal x diagonal block is diagonal, so the
system reduces to the (n+1) x (n+1) Schur complement of that block. The complement is
built in closed form once, inverted once in fp64 on the device (Cholesky, falling back
to LU then pinv like :176-183) and cached in fp64. Every fit is then one M^T S
reduction kernel plus the three fp64 kernels of `ops.fit_lines`; the features agree
with the fp64 ridge solution to fp32 rounding (the reference's fp32 Cholesky of the
full 3n x 3n matrix does not).
"""
from __future__ import annotations

import threading
from typing import Dict

import torch

from . import ops

_FACTOR_CACHE: Dict[tuple, torch.Tensor] = {}
_FACTOR_CACHE_LOCK = threading.Lock()


def compute_mtm(n: int, blocks_per_frame: int, regularization: float = 1e-3) -> torch.Tensor:
    """Closed-form M^T M + lambda I, CPU float64 (MoD/mod/cuda_lstsq.py:42-89)."""
    return ops.compute_mtm_host(n, blocks_per_frame, regularization)


def compute_mts(S_T: torch.Tensor, blocks_per_frame: int) -> torch.Tensor:
    """(H, 3n) fp32 M^T S (MoD/mod/cuda_lstsq.py:91-139 semantics, HIP kernel)."""
    return ops.compute_mts(S_T, blocks_per_frame)


def _factor_cache_key(device: torch.device, n: int, blocks_per_frame: int, regularization: float):
    return (device.type, device.index, int(n), int(blocks_per_frame), float(regularization))


def get_factor(device: torch.device, n: int, blocks_per_frame: int,
               regularization: float) -> torch.Tensor:
    """Cached fp64 inverse of the (n+1, n+1) Schur complement on `device`
    (the factor cache of MoD/mod/cuda_lstsq.py:141-186)."""
    key = _factor_cache_key(device, n, blocks_per_frame, regularization)
    inv = _FACTOR_CACHE.get(key)
    if inv is not None:
        return inv
    with _FACTOR_CACHE_LOCK:
        inv = _FACTOR_CACHE.get(key)
        if inv is not None:
            return inv
        schur = ops.fit_schur_host(n, blocks_per_frame, regularization).to(device)
        try:
            inv = torch.cholesky_inverse(torch.linalg.cholesky(schur))
        except RuntimeError:
            try:
                inv = torch.linalg.inv(schur)
            except RuntimeError:
                inv = torch.linalg.pinv(schur)
        inv = inv.contiguous()
        _FACTOR_CACHE[key] = inv
        return inv


def fit(mts: torch.Tensor, n: int, blocks_per_frame: int, regularization: float) -> torch.Tensor:
    """Features X (H, 3n) fp32 of M^T S rows (H, 3n)."""
    sinv = get_factor(mts.device, n, blocks_per_frame, regularization)
    return ops.fit_lines(sinv, mts, n, blocks_per_frame, regularization)


def features_from_x(X: torch.Tensor, n: int) -> Dict[str, torch.Tensor]:
    """Feature dict of MoD/mod/cuda_lstsq.py:249-261; '_x' keeps the raw solution."""
    nd = 2 * n - 1
    return {
        "d": X[:, :nd],
        "c": X[:, nd:nd + n] / 2,
        "b_d": X[:, -1],
        "_x": X,
    }


def solve_lstsq(warmup_state, S_T, step, blocks_per_frame, layer_idx=0, regularization=1e-5,
                use_cuda=True):
    """Features of an (H, n, n) map (MoD/mod/cuda_lstsq.py:211-270).

    At step <= warmup_steps - 2 the reference returns zero features (:245, 265-270); the
    M^T S it computes there is discarded, so it is not computed here.
    """
    if not S_T.is_cuda:
        raise ValueError("solve_lstsq: S_T must be a GPU tensor (this build has no CPU path)")
    H, n = S_T.shape[0], S_T.shape[1]
    if step > warmup_state["warmup_steps"] - 2:
        X = fit(ops.compute_mts(S_T, blocks_per_frame), n, blocks_per_frame, regularization)
    else:
        X = torch.zeros((H, 3 * n), device=S_T.device, dtype=torch.float32)
    return features_from_x(X, n)
