"""Accuracy contracts of the int8 Q.K^T / fp8 P.V path, shared by the GPU tests.

Both bounds are derived from the rounding model of the kernels' arithmetic, not fitted to
measurements (the oracle functions document each term; tests/test_oracle.py checks that
they hold for renderings of the arithmetic and that each term is needed):

- kernel against the oracle's fp64 model of its arithmetic (oracle.attention_q8_with_bound):
  fp32 accumulation, the bf16 output rounding, and a one-code e4m3 re-rounding of a
  weight only where the model's weight lies within fp32's error of a rounding midpoint;
- kernel against exact attention on the unquantised inputs (oracle.q8_exact_error_bound):
  the int8 score error measured per row, e4m3 P and V, subnormals, accumulation, output.

The thresholds used before these bounds (max-abs 4e-3 / mean-abs 2e-4 against the model)
are printed beside them as metrics.
"""
import numpy as np
import torch

import oracle as O


def _f64(x):
    if torch.is_tensor(x):
        x = x.detach().float().cpu().numpy()
    return np.asarray(x, np.float64)


def check_q8_model(out, z, tm=None, origin=0, rows=slice(None), tag=""):
    """Kernel output `out` (H, R, D) against rows `rows` of the oracle's model of the
    int8/fp8 arithmetic on the same quantised inputs `z`, elementwise within the derived
    bound. Returns the model's (O, LSE) over all rows."""
    ref, lse, bound = O.attention_q8_with_bound(z, tm, origin=origin)
    got = _f64(out)
    err = np.abs(got - ref[:, rows])
    b = bound[:, rows]
    ratio = err / np.maximum(b, 1e-300)
    over = int((err > b).sum())
    rows_4e3 = int((err.max(axis=-1) > 4e-3).sum())
    print(f"{tag}: q8 vs model max-abs {err.max():.3e} mean-abs {err.mean():.3e}, worst "
          f"element at {ratio.max():.3f} of its bound ({over} over); rows above 4e-3: "
          f"{rows_4e3} of {err.size // err.shape[-1]}", flush=True)
    assert over == 0, (tag, float(ratio.max()), over)
    return ref, lse


def check_q8_exact(got_h, q_h, k_h, v_h, qz, b, h, rows, allowed, tag=""):
    """Rows `rows` of head h of the kernel's output `got_h` (R, D) against exact
    attention on the unquantised inputs (q_h, k_h, v_h: the head's (S, D) values),
    elementwise within oracle.q8_exact_error_bound, given the quantiser's outputs `qz`
    (batch element b) for these rows and keys. Returns (err, bound, E) arrays."""
    origin = qz.origin
    pos_r = np.asarray(rows) - origin
    pos_k = np.arange(k_h.shape[0]) - origin
    qs = qz.q_scale[b, h].cpu().numpy()[pos_r // 32]
    ks = qz.k_scale[b, h].cpu().numpy()[pos_k // 64]
    o, bound, E = O.q8_exact_error_bound(
        q_h[rows], k_h, v_h, qz.q8[b, h].cpu().numpy()[rows], qs, qz.k8[b, h].cpu().numpy(), ks,
        qz.k_mean[b, h].cpu().numpy(), qz.v_scale[b, h].cpu().numpy(), allowed=allowed)
    err = np.abs(_f64(got_h) - o)
    assert np.all(err <= bound), (tag, float((err / bound).max()), int((err > bound).sum()))
    return err, bound, E
