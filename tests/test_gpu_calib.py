"""The calibration library (libmoddit_calib.so, not part of the C ABI):

- the MFMA-ceiling measurement bench.py reports beside the published peak: it runs, and
  its rate, clock and cycles per MFMA are consistent with each other and with the part's
  limits (2.5 PFLOP/s bf16 and 5.0 POP/s int8/fp8 dense at the top clock);
- the single-MFMA summation precision that the int8/fp8 accuracy contract assumes."""
import numpy as np
import pytest

import bench
import oracle as O

pytestmark = pytest.mark.gpu

# kind -> (published dense peak at the top clock, ops per MFMA): the 32x32 shapes the
# kernels use and the 16x16 shapes of the same types
PEAK = {0: (2500.0, 32768), 1: (5000.0, 65536), 2: (5000.0, 131072),
        3: (2500.0, 16384), 4: (5000.0, 32768), 5: (5000.0, 65536)}


@pytest.mark.parametrize("kind", [0, 1, 2, 3, 4, 5])
def test_mfma_ceiling_is_consistent(kind):
    r = bench.mfma_ceiling(kind, iters=400, reps=2)
    assert r is not None, "libmoddit_calib.so missing or the measurement failed"
    peak, ops = PEAK[kind]
    assert 0.2 * peak < r["value"] <= 1.02 * peak, r
    assert 500 <= r["clock_mhz"] <= 2600, r
    # an MFMA cannot issue faster than its pass count: the published peak is 1024 SIMDs
    # x ops per MFMA / (minimum cycles per MFMA) at 2.4 GHz
    min_cycles = 1024 * ops * 2.4e9 / (peak * 1e12)
    assert r["cycles_per_mfma_per_simd"] >= 0.97 * min_cycles, (min_cycles, r)


# --------------------------------------------------------------------------------------
# summation precision of single MFMAs (the constants of the int8/fp8 accuracy contract)
# --------------------------------------------------------------------------------------
def _precision_probe():
    import ctypes

    from mod_dit_amd import _lib

    lib = ctypes.CDLL(str(_lib.LIB_PATH.parent / "libmoddit_calib.so"))
    fn = lib.moddit_calib_mfma_precision
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int, ctypes.c_int] + [ctypes.c_void_p] * 4
    return fn


def _mfma_once(fn, kind, A, B, C):
    """One MFMA per wave: A, B (W, 64, 32) bytes, C (W, 64, 16) fp32 -> C + A.B."""
    import torch

    a, b, c = (torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (A, B, C))
    o = torch.empty_like(c)
    assert fn(kind, A.shape[0], a.data_ptr(), b.data_ptr(), c.data_ptr(), o.data_ptr()) == 0
    return o.cpu().numpy().astype(np.float64)


def _exact_dot(kind, A, B, C):
    """(C + A.B, sum |a b|) in the probe's layout: A lane (m, h) and B lane (n, h) hold the
    same k positions; C element i of lane l is row 8 (i/4) + 4 (l/32) + i%4, column l%32."""
    W = A.shape[0]
    if kind == 2:
        av = O.e4m3_decode(A).reshape(W, 2, 32, 32)
        bv = O.e4m3_decode(B).reshape(W, 2, 32, 32)
    else:
        av = ((A.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
              .astype(np.float64).reshape(W, 2, 32, 16)[..., :8])
        bv = ((B.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
              .astype(np.float64).reshape(W, 2, 32, 16)[..., :8])
    prod = np.einsum("whmj,whnj->wmnhj", av, bv)
    l = np.arange(64)[:, None]
    i = np.arange(16)[None, :]
    rows, cols = 8 * (i // 4) + 4 * (l // 32) + i % 4, np.broadcast_to(l % 32, (64, 16))
    exact = prod.sum(axis=(3, 4))[:, rows, cols] + C.astype(np.float64)
    return exact, np.abs(prod).sum(axis=(3, 4))[:, rows, cols]


def test_fp8_mfma_sums_within_the_contract_constants():
    """v_mfma_scale_f32_32x32x64_f8f6f4 (the int8/fp8 kernel's P.V product) does not add
    its 64 products in exact fp32. The int8/fp8 accuracy contract models its result as
    within FP8_MFMA_SUM_REL * sum |a b| + FP8_MFMA_ACC_REL * |C| (+ fp32 rounding) of the
    exact C + A.B; this holds the instruction to those constants on integer operands
    (exact: checks the probe's operand layout), on uniform codes, Gaussian values,
    attention-like P x V, a dominant product, cancelling pairs, subnormals, and small
    products onto a large accumulator. The bf16 MFMA sums to fp32 accuracy."""
    fn = _precision_probe()
    rng = np.random.default_rng(3)
    W = 512
    enc = lambda x: O.e4m3_encode(np.clip(x, -448, 448))
    zero = np.zeros((W, 64, 16), np.float32)
    ints = O.e4m3_encode(np.arange(9.0))
    A = rng.choice(ints, size=(W, 64, 32)).astype(np.uint8) | (
        rng.integers(0, 2, (W, 64, 32)) * 0x80).astype(np.uint8)
    B = rng.choice(ints, size=(W, 64, 32)).astype(np.uint8)
    exact, _ = _exact_dot(2, A, B, zero)
    assert np.array_equal(_mfma_once(fn, 2, A, B, zero), exact)

    codes = rng.integers(0, 256, (2, W, 64, 32)).astype(np.uint8)
    codes = np.where((codes & 0x7F) == 0x7F, codes & 0xF0, codes).astype(np.uint8)
    dom_a = rng.normal(0, 1, (W, 64, 32))
    dom_a[..., 0] = 400.0
    dom_b = np.exp2(rng.uniform(-10, 0, (W, 64, 32)))
    dom_b[..., 0] = 400.0
    can_a = rng.normal(0, 1, (W, 64, 32))
    can_a[..., 1::2] = -can_a[..., 0::2]
    can_b = np.exp2(rng.uniform(-4, 4, (W, 64, 32)))
    can_b[..., 1::2] = can_b[..., 0::2]
    cases = {
        "uniform codes": (codes[0], codes[1], zero),
        "gaussian": (enc(rng.normal(0, 1, (W, 64, 32))), enc(rng.normal(0, 1, (W, 64, 32))), zero),
        "P x V": (enc(rng.normal(0, 100, (W, 64, 32))),
                  enc(np.exp2(rng.uniform(-20, 8.5, (W, 64, 32)))),
                  rng.normal(0, 1e4, (W, 64, 16)).astype(np.float32)),
        "dominant": (enc(dom_a), enc(dom_b), zero),
        "cancelling": (enc(can_a), enc(can_b), zero),
        "subnormals": (enc(rng.uniform(-2 ** -6, 2 ** -6, (W, 64, 32))),
                       enc(rng.normal(0, 100, (W, 64, 32))), zero),
        "large C": (enc(rng.normal(0, 1e-2, (W, 64, 32))), enc(rng.normal(0, 1, (W, 64, 32))),
                    rng.normal(0, 1e6, (W, 64, 16)).astype(np.float32)),
    }
    for name, (A, B, C) in cases.items():
        got = _mfma_once(fn, 2, A, B, C)
        exact, absum = _exact_dot(2, A, B, C)
        allow = (O.FP8_MFMA_SUM_REL * absum + O.FP8_MFMA_ACC_REL * np.abs(C.astype(np.float64))
                 + 2.0 ** -24 * np.abs(exact))
        err = np.abs(got - exact)
        ratio = (err / allow).max()
        print(f"fp8 MFMA {name}: worst error at {ratio:.3f} of the allowance "
              f"(err / sum|ab| up to 2^{np.log2((err / np.maximum(absum, 1e-300)).max() + 1e-300):.2f})",
              flush=True)
        assert np.all(err <= allow), (name, ratio)

    a = O.bf16_round(rng.normal(0, 1, (W, 64, 16)).astype(np.float32))
    b = O.bf16_round(rng.normal(0, 1, (W, 64, 16)).astype(np.float32))
    A = (a.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(W, 64, 32)
    B = (b.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(W, 64, 32)
    C = rng.normal(0, 10, (W, 64, 16)).astype(np.float32)
    exact, absum = _exact_dot(0, A, B, C)
    err = np.abs(_mfma_once(fn, 0, A, B, C) - exact)
    assert np.all(err <= 2.0 ** -22 * (absum + np.abs(C))), err.max()
