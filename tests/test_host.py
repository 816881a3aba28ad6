"""Host-side checks that need no GPU: the C-ABI library, validation, state, modes."""
import ctypes
import re
import types

import numpy as np
import pytest
import torch

import mod_dit_amd as md
import oracle as O
from mod_dit_amd import _lib

HEADER = _lib.LIB_PATH.parents[1] / "include" / "moddit.h"


def _declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moddit_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_symbols()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_lib.EXPORTED)
    assert lib.moddit_version().startswith(b"moddit-mi355x")


def test_calibration_library_stays_outside_the_c_abi():
    """bench.py's MFMA-ceiling kernel lives in its own library: the drop-in library and
    its header carry no calibration entry point."""
    calib = _lib.LIB_PATH.parent / "libmoddit_calib.so"
    assert calib.exists(), "build() builds libmoddit_calib.so next to libmoddit.so"
    lib = ctypes.CDLL(str(calib))
    assert hasattr(lib, "moddit_calib_mfma")
    assert not hasattr(_lib.load(), "moddit_calib_mfma")
    assert "moddit_calib_mfma" not in _declared_symbols()
    fn = lib.moddit_calib_mfma
    fn.restype = ctypes.c_int
    d = ctypes.c_double()
    # argument errors are reported before any HIP call
    assert fn(6, 0, 10, 1, ctypes.byref(d), ctypes.byref(d), ctypes.byref(d)) == 2
    assert fn(-1, 0, 10, 1, ctypes.byref(d), ctypes.byref(d), ctypes.byref(d)) == 2
    assert fn(0, 0, 0, 1, ctypes.byref(d), ctypes.byref(d), ctypes.byref(d)) == 2
    assert fn(0, 0, 10, 1, None, ctypes.byref(d), ctypes.byref(d)) == 2


def test_mtm_host_matches_oracle_closed_form_and_brute_force():
    for n, bpf in [(4, 2), (9, 4), (64, 16)]:
        got = md.compute_mtm(n, bpf, 1.0).numpy()
        assert np.array_equal(got, O.mtm_closed_form(n, bpf, 1.0))
    M = O.build_M(9, 4)
    assert np.array_equal(md.compute_mtm(9, 4, 0.5).numpy(), M.T @ M + 0.5 * np.eye(27))


def test_fit_schur_host_is_the_schur_complement_of_mtm():
    """S = C - W^T A^-1 W for G = M^T M + lambda I = [[A, W], [W^T, C]] with A the
    diagonal x diagonal block, which must be diagonal; the fit's elimination rests on it.
    Checked against the explicit indicator matrix M (brute force) and the closed form."""
    for n, bpf, lam in [(4, 2, 1.0), (9, 4, 0.5), (37, 5, 1.0), (64, 16, 1.0), (61, 60, 1.0)]:
        G = O.build_M(n, bpf) if n <= 16 else None
        G = G.T @ G + lam * np.eye(3 * n) if G is not None else O.mtm_closed_form(n, bpf, lam)
        nd = 2 * n - 1
        A = G[:nd, :nd]
        assert np.array_equal(A, np.diag(np.diag(A)))
        W, C = G[:nd, nd:], G[nd:, nd:]
        want = C - W.T @ (W / np.diag(A)[:, None])
        got = md.ops.fit_schur_host(n, bpf, lam).numpy()
        np.testing.assert_allclose(got, want, rtol=0, atol=1e-12 * np.abs(want).max())
        # eliminating A and solving S reproduces the full solve
        rng = np.random.default_rng(n)
        rhs = rng.normal(size=3 * n)
        x_full = np.linalg.solve(G, rhs)
        x_cb = np.linalg.solve(got, rhs[nd:] - W.T @ (rhs[:nd] / np.diag(A)))
        x_d = (rhs[:nd] - W @ x_cb) / np.diag(A)
        np.testing.assert_allclose(np.concatenate([x_d, x_cb]), x_full, rtol=0,
                                   atol=1e-9 * np.abs(x_full).max())
    lib = _lib.load()
    assert lib.moddit_fit_schur_host(0, 1, 1.0, None) == _lib.MODDIT_EINVAL
    assert lib.moddit_fit_workspace_doubles(24, 1800) == 2 * 24 * 1801


def test_c_abi_rejects_bad_arguments_before_any_launch():
    lib = _lib.load()
    rc = lib.moddit_mtm_host(0, 1, 1.0, None)
    assert rc == _lib.MODDIT_EINVAL
    assert b"mtm" in lib.moddit_last_error()
    s = _lib.strides3(0, 0, 0)
    rc = lib.moddit_flash_fwd(16, 16, 16, 16, None, 1, 1, 64, 64, 96, s, s, s, s, 0.1, 0, None)
    assert rc == _lib.MODDIT_EUNSUPPORTED and b"head_dim" in lib.moddit_last_error()
    rc = lib.moddit_sparsity_map(16, 16, 16, 16, 1, 1, 128, 64, s, s, 0.1, -1.0, 0, 0, 2, 32, 0, None)
    assert rc == _lib.MODDIT_EINVAL and b"block_size" in lib.moddit_last_error()
    # the merged replay's lists must cover the video region's 128-row query tiles
    rc = lib.moddit_sparsity_map_merge(16, 16, 16, 16, 1, 1, 256, 64, s, s, 0.1, -1.0, 0, 0, 4,
                                       64, 0, 16, 16, 1, 4, None)
    assert rc == _lib.MODDIT_EINVAL and b"needs 2" in lib.moddit_last_error()
    rc = lib.moddit_sparsity_map_merge(16, 16, 16, 16, 1, 1, 256, 64, s, s, 0.1, -1.0, 0, 0, 4,
                                       64, 0, None, None, 2, 4, None)
    assert rc == _lib.MODDIT_EINVAL and b"tile lists" in lib.moddit_last_error()
    # the last map block must hold at least one token of the sequence
    rc = lib.moddit_sparsity_map(16, 16, 16, 16, 1, 1, 128, 64, s, s, 0.1, -1.0, 64, 64, 2, 64, 0,
                                 None)
    assert rc == _lib.MODDIT_EINVAL and b"exceeds" in lib.moddit_last_error()
    # grid origin outside (-64, 0]
    for origin in (1, -64):
        rc = lib.moddit_block_sparse_fwd(16, 16, 16, 16, None, 1, 1, 64, 64, 64, s, s, s, s, 0.1, 0,
                                         16, 16, 1, 1, origin, None)
        assert rc == _lib.MODDIT_EINVAL and b"grid_origin" in lib.moddit_last_error()
    # n_qtiles must cover the shifted grid: 64 rows from origin -30 need one 128-row tile
    rc = lib.moddit_block_sparse_fwd(16, 16, 16, 16, None, 1, 1, 100, 100, 64, s, s, s, s, 0.1, 0,
                                     16, 16, 1, 1, -30, None)
    assert rc == _lib.MODDIT_EINVAL and b"needs 2" in lib.moddit_last_error()
    rc = lib.moddit_select_lines(16, 16, 1, 6000, 10, 5, 16, None)
    assert rc == _lib.MODDIT_EINVAL and b"exceeds" in lib.moddit_last_error()
    rc = lib.moddit_mask_from_lines(16, 1, 1, 16, 4, 2, _lib.LAYOUT_WAN, 5, 0, 64, 1,
                                    None, None, None, 0, 0, None)
    assert rc == _lib.MODDIT_EINVAL and b"nb == n" in lib.moddit_last_error()
    # int8/fp8 path: quantiser grid origin and head_dim, LSE without q . mean_k, query prefix
    P = 16  # a non-null, 16-byte aligned stand-in pointer (never dereferenced)
    q8_out = [P] * 9
    rc = lib.moddit_quantize_qkv(P, P, P, 1, 1, 64, 64, s, s, s, 0, 1, *q8_out, None)
    assert rc == _lib.MODDIT_EINVAL and b"grid_origin" in lib.moddit_last_error()
    rc = lib.moddit_quantize_qkv(P, P, P, 1, 1, 64, 96, s, s, s, 0, 0, *q8_out, None)
    assert rc == _lib.MODDIT_EUNSUPPORTED and b"head_dim" in lib.moddit_last_error()
    rc = lib.moddit_flash_fwd_q8(P, P, P, P, P, P, None, P, P, 1, 1, 64, 64, s, 0.1, 0, None)
    assert rc == _lib.MODDIT_EINVAL and b"q_kmean" in lib.moddit_last_error()
    rc = lib.moddit_block_sparse_fwd_q8(P, P, P, P, P, P, P, P, P, 1, 1, 64, 65, 64, s, 0.1, 0,
                                        P, P, 1, 1, 0, None)
    assert rc == _lib.MODDIT_EINVAL and b"q_len" in lib.moddit_last_error()
    rc = lib.moddit_block_sparse_fwd_q8(P, P, P, P, P, P, P, P, P, 1, 1, 300, 300, 64, s, 0.1, 0,
                                        P, P, 1, 1, 0, None)
    assert rc == _lib.MODDIT_EINVAL and b"needs 3" in lib.moddit_last_error()
    # fp16 M^T S: n beyond the int64 accumulators' range, unaligned workspace
    rc = lib.moddit_mts(P, _lib.FP16, 1, (1 << 20) + 1, 4, P, P, None)
    assert rc == _lib.MODDIT_EINVAL and b"exceeds" in lib.moddit_last_error()
    rc = lib.moddit_mts(P, _lib.FP16, 1, 64, 4, P + 8, P, None)
    assert rc == _lib.MODDIT_EINVAL and b"aligned" in lib.moddit_last_error()
    # the frame-block output sums n * min(bpf, n) cells: at most 2^23 stay exact in int64
    rc = lib.moddit_mts(P, _lib.FP16, 1, 4096, 4096, P, P, None)
    assert rc == _lib.MODDIT_EINVAL and b"frame-block cells" in lib.moddit_last_error()
    rc = lib.moddit_mts(P, _lib.FP16, 1, 4096, 2049, P, P, None)
    assert rc == _lib.MODDIT_EINVAL and b"frame-block cells" in lib.moddit_last_error()
    with pytest.raises(_lib.ModditError, match="mtm"):
        _lib.check(lib.moddit_mtm_host(-1, 1, 1.0, None), "moddit_mtm_host")


def test_state_matches_reference_fields_and_errors():
    st = md.create_adaptive_mask_state("wan", 40, 69120, 512, 3840, 18, block_size=64)
    assert st["blocks_per_frame"] == 60 and st["threshold"] == 1.5e-4
    assert st["features_history"] is None and st["mask"] is None
    assert st["tile_rows"] == "union"
    assert not md.is_warmup_complete(st)
    with pytest.raises(ValueError, match="not support"):
        md.create_adaptive_mask_state("wan", 1, 64, 0, 64, 1, sparse_type="bogus")


class _FakeCuda:
    """Duck-typed stand-in carrying only what _validate_inputs reads."""

    def __init__(self, shape, dtype=torch.float16, is_cuda=True):
        self.shape = torch.Size(shape)
        self.ndim = len(shape)
        self.dtype = dtype
        self.is_cuda = is_cuda
        self.device = torch.device("cuda", 0)


# the reference's test_input_validation cases (tests/test_flash_sparsity.py:178-201)
@pytest.mark.parametrize(
    "mutation,error_type,match",
    [
        ({"block_size": 32}, ValueError, "block_size"),
        ({"video_token_num": 65}, ValueError, "divisible"),
        ({"model_type": "unknown"}, ValueError, "Unknown model_type"),
        ({"threshold": float("nan")}, ValueError, "NaN"),
    ],
)
def test_input_validation(mutation, error_type, match):
    q = _FakeCuda((1, 1, 128, 64))
    args = dict(query=q, key=q, value=q, threshold=1e-3, block_size=64, model_type="hunyuan",
                video_token_num=64, text_token_num=64)
    args.update(mutation)
    with pytest.raises(error_type, match=match):
        md._validate_inputs(**args)


def test_input_validation_more_cases():
    q = _FakeCuda((1, 1, 128, 64))
    with pytest.raises(TypeError, match="float16 or bfloat16"):
        f = _FakeCuda((1, 1, 128, 64), dtype=torch.float32)
        md._validate_inputs(f, f, f, 1e-3, 64, "wan", 0, 0)
    with pytest.raises(ValueError, match="CUDA tensors"):
        c = _FakeCuda((1, 1, 128, 64), is_cuda=False)
        md._validate_inputs(c, c, c, 1e-3, 64, "wan", 0, 0)
    with pytest.raises(ValueError, match="head_dim"):
        d = _FakeCuda((1, 1, 128, 96))
        md._validate_inputs(d, d, d, 1e-3, 64, "wan", 0, 0)
    with pytest.raises(ValueError, match="exceed"):
        md._validate_inputs(q, q, q, 1e-3, 64, "hunyuan", 128, 64)
    thr, vb, qo, ko = md._validate_inputs(q, q, q, 1e-3, 64, "cogvideox", 64, 64)
    assert (vb, qo, ko) == (1, 64, 64)
    assert md._validate_inputs(q, q, q, 0.0, 64, "wan", 0, 0)[:2] == (0.0, 2)


def test_head_modes_reads_like_reference_list():
    hm = md.HeadModes(torch.tensor([0, 1, 2, 0], dtype=torch.uint8))
    assert list(hm) == ["sparse", "block_diagonal", "full", "sparse"]
    assert hm == ["sparse", "block_diagonal", "full", "sparse"]
    assert len(hm) == 4 and hm[1] == "block_diagonal"


def test_check_bd_values_host_form():
    vals = torch.tensor([[0.0, 2.0], [0.0, 1.0], [0.0, 0.5]])
    assert md.check_bd_values(vals, ["sparse"] * 3, threshold=1) == ["sparse", "block_diagonal",
                                                                     "block_diagonal"]


def test_product_path_refuses_cpu_tensors():
    with pytest.raises(ValueError, match="GPU"):
        md.ops.compute_mts(torch.zeros(1, 4, 4, dtype=torch.float16), 2)
    st = md.create_adaptive_mask_state("wan", 1, 256, 0, 128, 2, block_size=64)
    with pytest.raises(ValueError, match="GPU"):
        md.solve_lstsq(st, torch.zeros(1, 4, 4, dtype=torch.float16), 11, 2)


def test_use_dense_int8_rejects_more_video_queries_than_valid_keys():
    """The int8 dense path quantises the first valid-key-count tokens together; more
    video queries than valid keys is refused before any launch."""
    S, video = 512, 384
    st = md.create_adaptive_mask_state("hunyuan", 1, video, S - video, 128, 3, block_size=64,
                                       precision="int8")
    pdm = torch.zeros(S, S, dtype=torch.bool)
    pdm[:, :300] = True  # fewer valid keys than video tokens
    q = torch.zeros(1, 1, S, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="video_token_num=384"):
        md.SparseAttentionWithMap(q, q, q, st, None, pre_defined_mask=pdm, use_dense=True)


def test_use_dense_int8_rejects_a_q_block_across_the_video_text_boundary():
    """Q is quantised in 32-row blocks; with a video length that is not a multiple of 32
    one block would mix video and text rows (the reference quantises query[:video]
    alone), so the int8 dense path refuses it before any launch."""
    S, video = 512, 400
    st = md.create_adaptive_mask_state("hunyuan", 1, video, S - video, 80, 5, block_size=16,
                                       precision="int8")
    pdm = torch.zeros(S, S, dtype=torch.bool)
    pdm[:, :450] = True
    q = torch.zeros(1, 1, S, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="multiple of 32"):
        md.SparseAttentionWithMap(q, q, q, st, None, pre_defined_mask=pdm, use_dense=True)


def _fake_amdsmi(samples, cap_uw=1_400_000_000):
    """A stand-in amdsmi module that serves `samples` (power W, clock MHz) in order."""
    it = iter(samples)
    calls = {"init": 0, "shutdown": 0}

    def metrics(_h):
        pw, clk = next(it, samples[-1])
        return {"current_socket_power": pw, "current_gfxclk": clk}

    m = types.SimpleNamespace(
        amdsmi_init=lambda: calls.__setitem__("init", calls["init"] + 1),
        amdsmi_shut_down=lambda: calls.__setitem__("shutdown", calls["shutdown"] + 1),
        amdsmi_get_processor_handles=lambda: ["gpu0"],
        amdsmi_get_power_cap_info=lambda _h: {"power_cap": cap_uw},
        amdsmi_get_gpu_metrics_info=metrics)
    return m, calls


def test_board_sampler_collects_and_filters(monkeypatch):
    """bench.BoardSampler on a stand-in amdsmi: 0xFFFF-style missing fields never enter the
    record, amdsmi is initialised and shut down once, the cap is read in watts."""
    import sys
    import time as _time

    import bench

    fake, calls = _fake_amdsmi([(0xFFFF, 1800)] * 3 + [(1300, 1850), (1320, 1870)] * 50)
    monkeypatch.setitem(sys.modules, "amdsmi", fake)
    with bench.BoardSampler(period_s=0.005, skip_s=0.0) as b:
        _time.sleep(0.1)
    r = b.result()
    assert calls == {"init": 1, "shutdown": 1}
    assert r is not None and r["samples"] == len(b.samples) >= 2
    assert all(x[1] != 0xFFFF for x in b.samples)
    assert 1300 <= r["power_w"] <= 1320 and r["power_w_max"] <= 1320
    assert 1850 <= r["gfxclk_mhz"] <= 1870 and r["power_cap_w"] == 1400.0


def test_board_sampler_result_drops_the_lag_window():
    """Samples taken in the first skip_s seconds still show the load before the region."""
    import bench

    b = bench.BoardSampler(skip_s=1.0)
    b.samples = [(0.0, 500.0, 900.0), (0.6, 900.0, 2300.0), (1.2, 1320.0, 1870.0),
                 (1.7, 1330.0, 1860.0)]
    r = b.result()
    assert r["samples"] == 2 and r["power_w"] == 1325.0 and r["gfxclk_mhz"] == 1865
    b.samples = [(0.2, 500.0, 900.0)]
    assert b.result() is None


def test_board_sampler_without_amdsmi_reports_none(monkeypatch):
    import sys

    import bench

    monkeypatch.setitem(sys.modules, "amdsmi", None)  # import raises ImportError
    with bench.BoardSampler() as b:
        pass
    assert b.result() is None


def test_64_token_grid_of_a_128_block_mask_realises_the_same_token_mask():
    """attn_mask._as_64_token_grid: for random 128-token block masks on text-first grids
    starting 64..127 tokens early, the exact-row 64-tile lists of the converted mask
    realise the token mask of the original 128-block lists (oracle token masks)."""
    from mod_dit_amd.attn_mask import _as_64_token_grid

    rng = np.random.default_rng(5)
    checked = 0
    for _ in range(40):
        text = int(rng.integers(1, 64)) + 128 * int(rng.integers(0, 3))  # text % 128 in 1..63
        video = int(rng.integers(1, 900))
        tb, vb, origin = O.cogvideox_grid(text, video, 128)
        assert -127 <= origin <= -65
        S = text + video
        H = int(rng.integers(1, 3))
        nb = tb + vb
        m = rng.random((H, nb, nb)) < float(rng.uniform(0.1, 0.9))
        _, lists = O.tiles_from_mask(m, 128, False)
        want = O.token_mask_from_tiles(lists, H, S, S, origin=origin)
        m64, origin64 = _as_64_token_grid(torch.from_numpy(m), S, origin)
        assert -64 < origin64 <= 0 and m64.shape[1] == -(-(S - origin64) // 64)
        _, lists64 = O.tiles_from_mask(m64.numpy(), 64, False)
        got = O.token_mask_from_tiles(lists64, H, S, S, origin=origin64)
        assert np.array_equal(got, want), (text, video)
        checked += 1
    assert checked == 40
