"""Pins the CPU oracle against closed forms, brute force and invariants (CPU only).

Each check is chosen so that a plausible mistake in the oracle (a dropped term, a wrong
sign or index, a transposed operand) fails it; none of them retypes the oracle's own
formula.
"""
import math

import numpy as np
import pytest

import oracle as O


# ------------------------------------------------------------------ line model -------
@pytest.mark.parametrize("n,bpf", [(3, 1), (4, 2), (7, 3), (8, 4), (9, 4), (12, 5)])
def test_mtm_closed_form_equals_explicit_MtM(n, bpf):
    M = O.build_M(n, bpf)
    lam = 1.0
    assert np.array_equal(O.mtm_closed_form(n, bpf, lam), M.T @ M + lam * np.eye(3 * n))


def test_build_M_counts():
    # every cell sits on exactly one diagonal and one column
    n, bpf = 6, 2
    M = O.build_M(n, bpf)
    nd = 2 * n - 1
    assert np.all(M[:, :nd].sum(axis=1) == 1)
    assert np.all(M[:, nd:nd + n].sum(axis=1) == 1)
    assert M[:, -1].sum() == (n // bpf) * bpf * bpf


def _dyadic_map(rng, H, n, bs=64):
    counts = rng.integers(0, bs * bs + 1, size=(H, n, n))
    return (counts / float(bs * bs)).astype(np.float16)


@pytest.mark.parametrize("n,bpf", [(5, 2), (16, 4), (17, 5)])
def test_mts_exact_equals_brute_force(n, bpf):
    rng = np.random.default_rng(0)
    S = _dyadic_map(rng, 3, n)
    M = O.build_M(n, bpf)
    brute = np.stack([M.T @ S[h].astype(np.float64).ravel() for h in range(3)])
    got = O.mts_exact(S, bpf)
    assert np.array_equal(got.astype(np.float64), brute.astype(np.float32).astype(np.float64))


def test_mts_exact_arbitrary_fp16_is_correctly_rounded():
    # arbitrary-signed fp16 values incl. subnormals: exact sum, one rounding
    rng = np.random.default_rng(1)
    n, bpf = 9, 3
    bits = rng.integers(0, 0x7C00, size=(2, n, n)).astype(np.uint16)
    bits |= (rng.integers(0, 2, size=bits.shape) << 15).astype(np.uint16)
    S = bits.view(np.float16)
    from fractions import Fraction

    got = O.mts_exact(S, bpf)
    M = O.build_M(n, bpf)
    for h in range(2):
        vals = [Fraction(float(x)) for x in S[h].ravel()]
        for f in [0, n, 2 * n - 2, 2 * n - 1 + 3, 3 * n - 1]:
            exact = sum(v for v, w in zip(vals, M[:, f]) if w)
            assert got[h, f] == np.float32(float(exact))  # float(Fraction) is correctly rounded


@pytest.mark.parametrize("n,bpf", [(6, 2), (10, 3)])
def test_mts_loop_equals_exact_on_map_domain(n, bpf):
    rng = np.random.default_rng(2)
    S = _dyadic_map(rng, 2, n)
    loop = O.mts_loop(S, bpf)
    exact = O.mts_exact(S, bpf)
    # diagonal and column sums are exact in fp32 for map-domain values
    assert np.array_equal(loop[:, :-1], exact[:, :-1])
    np.testing.assert_allclose(loop[:, -1], exact[:, -1], rtol=1e-6)


def test_ridge_solve_recovers_planted_features():
    n, bpf, lam = 8, 2, 1.0
    rng = np.random.default_rng(3)
    xstar = rng.normal(size=(2, 3 * n))
    M = O.build_M(n, bpf)
    S = np.stack([(M @ xstar[h]).reshape(n, n) for h in range(2)])
    X = O.ridge_solve(S, bpf, lam)
    G = M.T @ M + lam * np.eye(3 * n)
    want = np.linalg.solve(G, (M.T @ M) @ xstar.T).T
    np.testing.assert_allclose(X, want, rtol=1e-9, atol=1e-9)
    # normal equations: (M^T M + lam I) X = M^T S
    res = G @ X.T - np.stack([M.T @ S[h].ravel() for h in range(2)]).T
    assert np.abs(res).max() < 1e-9
    # S = 0 -> X = 0
    assert np.all(O.ridge_solve(np.zeros((1, n, n)), bpf, lam) == 0)


def test_reconstruct_is_M_times_X():
    n, bpf = 7, 3
    rng = np.random.default_rng(4)
    X = rng.normal(size=(2, 3 * n))
    M = O.build_M(n, bpf)
    rec = O.reconstruct_map(X, n, bpf)
    for h in range(2):
        np.testing.assert_allclose(rec[h].ravel(), M @ X[h], rtol=1e-12)


def test_features_slicing_halves_columns():
    n = 5
    X = np.arange(2 * 3 * n, dtype=np.float32).reshape(2, 3 * n)
    f = O.features_from_x(X, n)
    assert np.array_equal(f["d"], X[:, :2 * n - 1])
    assert np.array_equal(f["c"] * 2, X[:, 2 * n - 1:3 * n - 1])
    assert np.array_equal(f["b_d"], X[:, -1])


# ------------------------------------------------------------------ selection --------
def test_first_prediction_is_cur_times_one_plus_inv_T():
    # at W-1 the previous features are zeros (MoD/mod/cuda_lstsq.py:265-270)
    n, T = 6, 10
    rng = np.random.default_rng(5)
    xc = rng.normal(size=(2, 3 * n)).astype(np.float32)
    v = O.predict_lines(xc, np.zeros_like(xc), n, T)
    c = xc[:, 2 * n - 1:3 * n - 1] / 2
    np.testing.assert_allclose(v[:, :n], c * (1 + 1 / T), rtol=1e-6)
    np.testing.assert_allclose(v[:, n:], xc[:, :2 * n - 1] * (1 + 1 / T), rtol=1e-6)


def test_choose_topk_matches_sorted_order_with_ties_nan_and_signed_zero():
    n, T, k = 5, 3, 6
    xc = np.zeros((1, 3 * n), np.float32)
    xl = np.zeros((1, 3 * n), np.float32)
    # craft predictions directly through cur with last = cur (pred = cur)
    vals = np.array([0.5, -1.0, 0.5, np.nan, -0.0, 0.0, 2.0, -1.0, 3.0, 0.5, 0.25, 0.0, 7.0, -5.0],
                    dtype=np.float32)
    nd = 2 * n - 1
    # v[:n] = X[nd:nd+n]/2, v[n:] = X[:nd]
    xc[0, nd:nd + n] = vals[:n] * 2
    xc[0, :nd] = vals[n:n + nd]
    xl[:] = xc
    got = O.choose_topk_lines(xc, xl, n, T, k)[0]
    keyed = sorted(range(len(vals)), key=lambda i: (math.isnan(vals[i]), 0.0 if vals[i] == 0 else vals[i], i))
    assert list(got) == sorted(keyed[:k])


# ------------------------------------------------------------------ mask -------------
@pytest.mark.parametrize("seed", range(4))
def test_generate_mask_restatement_equals_cell_definition(seed):
    rng = np.random.default_rng(10 + seed)
    n, bpf, H, k = 11, 3, 4, 5
    sel = rng.integers(0, 3 * n - 1, size=(H, k))
    modes = [O.MODE_SPARSE, O.MODE_BLOCK_DIAGONAL, O.MODE_FULL, O.MODE_SPARSE]
    m = O.generate_mask_from_lines(sel, modes, seq_len=n * 64, block_size=64,
                                   video_tokens=n * 64, text_tokens=0, bpf=bpf, model_type="wan")
    for h in range(H):
        for i in range(n):
            for j in range(n):
                assert m[h, i, j] == O.mask_cell(sel[h], modes[h], n, bpf, i, j)


def test_generate_mask_layouts():
    n, bpf, bs = 4, 2, 64
    sel = np.array([[0], [n + (n - 1)]])  # head 0: column 0; head 1: main diagonal
    modes = [O.MODE_SPARSE, O.MODE_SPARSE]
    hy = O.generate_mask_from_lines(sel, modes, seq_len=(n + 2) * bs, block_size=bs,
                                    video_tokens=n * bs, text_tokens=2 * bs, bpf=bpf,
                                    model_type="hunyuan")
    assert hy.shape == (2, n + 2, n + 2)
    assert hy[:, n:, :].all() and hy[:, :, n:].all()
    assert hy[0, :n, 0].all() and not hy[0, :n, 1:n].any()
    assert np.array_equal(hy[1, :n, :n], np.eye(n, dtype=bool))
    cg = O.generate_mask_from_lines(sel, modes, seq_len=(n + 2) * bs, block_size=bs,
                                    video_tokens=n * bs, text_tokens=2 * bs, bpf=bpf,
                                    model_type="cogvideox")
    assert cg[:, :2, :].all() and cg[:, :, :2].all()
    assert np.array_equal(cg[1, 2:, 2:], np.eye(n, dtype=bool))
    other = O.generate_mask_from_lines(sel, modes, seq_len=n * bs, block_size=bs,
                                       video_tokens=n * bs, text_tokens=0, bpf=bpf,
                                       model_type="unknown")
    assert other.all()


def test_block_diagonal_covers_partial_last_frame():
    # i // bpf == j // bpf also holds in the tail past the last full frame (:535-539)
    n, bpf = 5, 2
    m = O.generate_mask_from_lines(np.full((1, 1), 10**6), [O.MODE_BLOCK_DIAGONAL], seq_len=n * 64,
                                   block_size=64, video_tokens=n * 64, text_tokens=0, bpf=bpf,
                                   model_type="wan")
    assert m[0, 4, 4] and not m[0, 3, 4]


# ------------------------------------------------------------------ tiles ------------
@pytest.mark.parametrize("nb,bs", [(7, 64), (8, 64), (3, 128)])
def test_tiles_realise_the_mask(nb, bs):
    rng = np.random.default_rng(20 + nb)
    mask = rng.random((2, nb, nb)) < 0.4
    L = nb * bs
    counts, exact = O.tiles_from_mask(mask, bs, union_rows=False)
    tm = O.token_mask_from_tiles(exact, 2, L, L)
    assert np.array_equal(tm, O.token_mask_from_blocks(mask, bs))
    _, union = O.tiles_from_mask(mask, bs, union_rows=True)
    tu = O.token_mask_from_tiles(union, 2, L, L)
    assert (tu | ~tm).all()  # union is a superset
    if bs == 64:
        # union == OR of the two rows of each pair (MoD/mod/attn_mask.py:299-303)
        for t in range((nb + 1) // 2):
            rows = mask[:, 2 * t:2 * t + 2].any(axis=1)
            assert np.array_equal(tu[:, t * 128, ::64], rows)
    for h in range(2):
        for t in range(counts.shape[1]):
            keys = [e >> 2 for e in exact[h][t]]
            assert keys == sorted(keys) and len(keys) == counts[h, t]


def _as_arrays(counts, lists):
    H, nq = counts.shape
    cap = max(1, max((len(e) for hl in lists for e in hl), default=1))
    ent = np.zeros((H, nq, cap), np.int64)
    for h in range(H):
        for t in range(nq):
            ent[h, t, :counts[h, t]] = lists[h][t]
    return ent


@pytest.mark.parametrize("nb,bs,union,kv_tiles,text,video", [
    (9, 64, False, None, 0, 0), (9, 64, True, 13, 0, 0), (4, 128, False, 7, 0, 0),
    (8, 64, False, None, 50, 450),
])
def test_token_mask_rows_equal_the_full_token_mask(nb, bs, union, kv_tiles, text, video):
    """Row sampling of the executed mask (used at full shape, where the whole token mask
    cannot be formed) equals the rows of the full token mask, incl. dropped key tiles
    beyond kv_tiles and a shifted grid."""
    rng = np.random.default_rng(nb + bs)
    origin = 0
    if text:
        tb, vb, origin = O.cogvideox_grid(text, video, bs)
        nb = tb + vb
        S = text + video
    else:
        S = nb * bs
    mask = rng.random((2, nb, nb)) < 0.35
    counts, lists = O.tiles_from_mask(mask, bs, union_rows=union, kv_tiles=kv_tiles)
    ent = _as_arrays(counts, lists)
    full = O.token_mask_from_tiles(lists, 2, S, S, origin=origin)
    rows = np.unique(np.r_[0, S - 1, rng.integers(0, S, 40)])
    for h in range(2):
        got = O.token_mask_rows_from_tiles(counts[h], ent[h], rows, S, origin=origin)
        assert np.array_equal(got, full[h, rows])
    if kv_tiles is not None:  # nothing at or beyond the key-tile limit
        assert not full[:, :, kv_tiles * 64 + origin:].any()


@pytest.mark.parametrize("text,video,bs", [(50, 450, 64), (226, 1350, 64), (100, 700, 128),
                                           (128, 512, 64)])
def test_cogvideox_grid_puts_text_and_video_on_block_boundaries(text, video, bs):
    tb, vb, origin = O.cogvideox_grid(text, video, bs)
    assert -bs < origin <= 0 and (origin == 0) == (text % bs == 0)
    assert tb * bs + origin == text  # video starts on grid block tb
    assert (tb - 1) * bs < text - origin <= tb * bs and (vb - 1) * bs < video <= vb * bs


@pytest.mark.parametrize("text,video", [(50, 450), (30, 300), (64, 130)])
def test_padded_grid_tiles_realise_the_cropped_block_mask(text, video):
    # the tile mask on a shifted grid equals the grid-token expansion of the block mask,
    # cropped to the sequence: built here with np.repeat and slicing, not with the tiles
    rng = np.random.default_rng(text + video)
    tb, vb, origin = O.cogvideox_grid(text, video, 64)
    nb, S = tb + vb, text + video
    mask = rng.random((2, nb, nb)) < 0.4
    _, exact = O.tiles_from_mask(mask, 64, union_rows=False)
    tm = O.token_mask_from_tiles(exact, 2, S, S, origin=origin)
    grid = O.token_mask_from_blocks(mask, 64)
    assert np.array_equal(tm, grid[:, -origin:-origin + S, -origin:-origin + S])


def test_generate_mask_cogvideox_padded_grid_equals_cell_definition():
    rng = np.random.default_rng(77)
    text, video, bs, bpf, H = 50, 450, 64, 2, 3
    tb, n, _ = O.cogvideox_grid(text, video, bs)
    sel = rng.integers(0, 3 * n - 1, size=(H, 4))
    modes = [O.MODE_SPARSE, O.MODE_BLOCK_DIAGONAL, O.MODE_SPARSE]
    m = O.generate_mask_from_lines(sel, modes, seq_len=text + video, block_size=bs,
                                   video_tokens=video, text_tokens=text, bpf=bpf,
                                   model_type="cogvideox")
    assert m.shape == (H, tb + n, tb + n)
    assert m[:, :tb, :].all() and m[:, :, :tb].all()
    for h in range(H):
        for i in range(n):
            for j in range(n):
                assert m[h, tb + i, tb + j] == O.mask_cell(sel[h], modes[h], n, bpf, i, j)


def test_replay_partial_last_block_counts_only_tokens_in_the_sequence():
    # brute force with explicit loops over the valid rectangle of every cell
    rng = np.random.default_rng(5)
    H, D, bs, off, video = 1, 64, 64, 40, 150  # 3 blocks, the last holds 22 tokens
    S = off + video
    q = rng.integers(-4, 5, size=(H, S, D)).astype(np.float32) / 8
    k = rng.integers(-4, 5, size=(H, S, D)).astype(np.float32) / 8
    s = np.einsum("hqd,hkd->hqk", q.astype(np.float64), k.astype(np.float64)) / 8
    lse = np.log(np.exp(s).sum(-1)).astype(np.float32)
    vb = 3
    rep = O.replay_map(q, k, lse, scale=1 / 8, log_threshold=math.log(1e-2), q_off=off,
                       k_off=off, video_blocks=vb, block_size=bs)
    thr = lse[0] + np.float32(math.log(1e-2))
    for i in range(vb):
        for j in range(vb):
            c = 0
            for r in range(i * bs, min((i + 1) * bs, video)):
                for cc in range(j * bs, min((j + 1) * bs, video)):
                    c += s[0, off + r, off + cc] < thr[off + r]
            assert rep[0, i, j] == np.float16(np.float32(c) / np.float32(bs * bs)), (i, j)
    assert rep[0, 2, 2] * bs * bs <= 22 * 22


# ------------------------------------------------------------------ attention / map --
def test_masked_attention_all_true_is_dense_and_local_is_blockwise():
    rng = np.random.default_rng(30)
    H, S, D = 2, 128, 16
    q, k, v = (rng.normal(size=(H, S, D)).astype(np.float32) for _ in range(3))
    dense, lse = O.masked_attention(q, k, v, None, dtype=np.float64)
    full, lse_full = O.masked_attention(q, k, v, np.ones((H, S, S), bool), dtype=np.float64)
    np.testing.assert_allclose(full, dense, rtol=1e-12)
    # brute force softmax
    s = np.einsum("hqd,hkd->hqk", q.astype(np.float64), k.astype(np.float64)) / math.sqrt(D)
    p = np.exp(s - s.max(-1, keepdims=True))
    np.testing.assert_allclose(dense, (p / p.sum(-1, keepdims=True)) @ v, rtol=1e-10)
    np.testing.assert_allclose(lse, np.log(np.exp(s).sum(-1)), rtol=1e-10)
    # block-diagonal (64) mask = independent attention per block
    bm = O.token_mask_from_blocks(np.eye(2, dtype=bool)[None].repeat(H, 0), 64)
    loc, _ = O.masked_attention(q, k, v, bm, dtype=np.float64)
    for b in range(2):
        sl = slice(64 * b, 64 * b + 64)
        ref, _ = O.masked_attention(q[:, sl], k[:, sl], v[:, sl], None, dtype=np.float64)
        np.testing.assert_allclose(loc[:, sl], ref, rtol=1e-10)
    # a row with no allowed key gives zeros and -inf LSE
    em = np.ones((H, S, S), bool)
    em[:, 3] = False
    out, l = O.masked_attention(q, k, v, em, dtype=np.float64)
    assert np.all(out[:, 3] == 0) and np.all(np.isneginf(l[:, 3]))


def test_probability_map_zero_threshold_is_zero():
    # reference known answer: tests/test_flash_sparsity.py:142-154
    rng = np.random.default_rng(31)
    q = rng.normal(size=(1, 128, 64)).astype(np.float32)
    m = O.probability_map(q, q, 0.0, 64, 0, 0, 128)
    assert np.count_nonzero(m) == 0


def test_replay_equals_probability_map_on_dyadic_inputs():
    # d=64 -> scale 1/8 exact; q,k in {-4..4}/8 -> bf16-exact scaled q and exact scores;
    # LSE from exact softmax; cells are equal when no score sits at the threshold
    rng = np.random.default_rng(32)
    H, S, D, bs, thr = 2, 256, 64, 64, 1e-3
    q = rng.integers(-4, 5, size=(H, S, D)).astype(np.float32) / 8
    k = rng.integers(-4, 5, size=(H, S, D)).astype(np.float32) / 8
    s = np.einsum("hqd,hkd->hqk", q.astype(np.float64), k.astype(np.float64)) / 8
    lse = np.log(np.exp(s).sum(-1))
    assert np.abs(s - (lse[..., None] + math.log(thr))).min() > 1e-5
    rep = O.replay_map(q, k, lse.astype(np.float32), scale=1 / 8, log_threshold=math.log(thr),
                       q_off=0, k_off=0, video_blocks=S // bs, block_size=bs)
    prob = O.probability_map(q, k, thr, bs, 0, 0, S)
    np.testing.assert_array_equal(rep.astype(np.float32), prob.astype(np.float16).astype(np.float32))


def test_replay_rounds_count_ratio_to_fp16():
    # 64x64 blocks: ratios are multiples of 2^-12; counts >= 2048 lose their last bit
    r = (np.arange(0, 4097) / 4096.0).astype(np.float32).astype(np.float16).astype(np.float64)
    assert np.all(r[:2049] * 4096 == np.arange(2049))
    assert np.all((r * 4096) % 1 == 0)


def test_bf16_round_half_to_even():
    x = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8], np.float32)
    np.testing.assert_array_equal(O.bf16_round(x), np.array([1.0, 1.0 + 2 ** -6, -1.0], np.float32))


# ------------------------------------------------------------------ schedule ---------
def test_step_schedule_W12_T10():
    phases = [O.step_phase(s, 12, 10) for s in range(50)]
    assert phases[:10] == ["dense"] * 10
    assert phases[10] == "map_fit" and phases[11] == "map_fit_predict"
    assert [s for s, p in enumerate(phases) if p == "refresh"] == [21, 31, 41]
    assert phases.count("sparse") == 50 - 12 - 3


# ------------------------------------------------------------------ int8 / fp8 path --
def test_e4m3_known_answers_and_ties():
    # OCP FP8 E4M3: 0x38 = 1.0, 0x7e = 448 (max), 0x08 = 2^-6 (min normal), 0x01 = 2^-9
    dec = O.e4m3_decode(np.array([0x38, 0x7E, 0x08, 0x01, 0xB8, 0x00, 0x7F], np.uint8))
    assert dec[:6].tolist() == [1.0, 448.0, 2.0 ** -6, 2.0 ** -9, -1.0, 0.0] and np.isnan(dec[6])
    # every finite code round-trips; midpoints round to the even code
    codes = np.arange(256, dtype=np.uint8)
    vals = O.e4m3_decode(codes)
    ok = np.isfinite(vals) & (codes != 0x80)
    assert np.array_equal(O.e4m3_encode(vals[ok]), codes[ok])
    assert O.e4m3_encode(np.array([1.0625]))[0] == 0x38      # tie between 0x38 and 0x39
    assert O.e4m3_encode(np.array([1.1875]))[0] == 0x3A      # tie between 0x39 and 0x3a
    assert O.e4m3_encode(np.array([1.0625 + 1e-9]))[0] == 0x39


@pytest.mark.parametrize("origin", [0, -14])
def test_quantize_qkv_bounds(origin):
    rng = np.random.default_rng(8)
    H, S, D = 2, 200, 64
    q = O.bf16_round(rng.standard_normal((H, S, D)) * 2)
    k = O.bf16_round(rng.standard_normal((H, S, D)) + 3.0)  # channel offset removed by the mean
    v = O.bf16_round(rng.standard_normal((H, S, D)))
    z = O.quantize_qkv(q, k, v, origin=origin)
    pos = np.arange(S) - origin  # grid position of each token
    qs = z["q_scale"][:, pos // 32][:, :, None]
    assert np.abs(q - z["q8"] * qs).max() <= 0.5001 * qs.max()
    assert np.abs(z["q8"]).max() == 127
    ks = z["k_scale"][:, pos // 64][:, :, None]
    kd = z["k8"] * ks + z["k_mean"][:, None, :]
    assert np.abs(k - kd).max() <= 0.5001 * ks.max() + 1e-5
    vd = O.e4m3_decode(z["v8t"][:, :, pos]).transpose(0, 2, 1) * z["v_scale"][:, None, :]
    assert np.all(np.abs(v - vd) <= 2.0 ** -4 * np.abs(v) + 2.0 ** -9 * z["v_scale"].max())
    outside = np.ones(z["v8t"].shape[2], bool)
    outside[pos] = False
    assert np.all(z["v8t"][:, :, outside] == 0)  # grid positions outside the sequence
    np.testing.assert_allclose(z["k_mean"], k.mean(axis=1), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(z["q_kmean"], np.einsum("hsd,hd->hs", q, z["k_mean"].astype(np.float64)),
                               rtol=1e-12, atol=1e-12)


def test_quantize_qkv_shifted_grid_is_zero_padding():
    # on the grid starting at -14, Q and V are quantised as the sequence with 14 zero tokens
    # in front on the unshifted grid; K as its mean-free part padded with zeros
    rng = np.random.default_rng(18)
    H, S, D, pad = 2, 150, 64, 14
    q, k, v = (O.bf16_round(rng.standard_normal((H, S, D)) * 1.5) for _ in range(3))
    km = k.mean(axis=1).astype(np.float32)
    z = O.quantize_qkv(q, k, v, origin=-pad)
    zp = lambda x: np.concatenate([np.zeros((H, pad, D), np.float32), x], axis=1)
    ref = O.quantize_qkv(zp(q), zp(k - km[:, None, :]), zp(v), k_mean=np.zeros_like(km))
    assert np.array_equal(z["q8"], ref["q8"][:, pad:])
    assert np.array_equal(z["q_scale"], ref["q_scale"])
    assert np.array_equal(z["v8t"][:, :, :S + pad], ref["v8t"][:, :, :S + pad])
    assert np.array_equal(z["k_scale"], ref["k_scale"])
    assert np.abs(z["k8"].astype(int) - ref["k8"][:, pad:]).max() <= 1  # k - mean rounded once


@pytest.mark.parametrize("origin", [0, -14])
def test_attention_q8_is_close_to_exact_attention(origin):
    # the quantisation error averages over the keys a row attends to: with 2048 keys it is
    # inside the bf16 bound (at 256 keys fp8 P alone reaches max-abs 0.011, all three 0.034)
    rng = np.random.default_rng(9)
    H, S, D = 2, 2048, 64
    q, k, v = (O.bf16_round(rng.standard_normal((H, S, D))) for _ in range(3))
    k = k + O.bf16_round(rng.standard_normal((H, 1, D)) * 0.5)  # a channel offset
    z = O.quantize_qkv(q, k, v, origin=origin)
    ref, ref_lse = O.masked_attention(q, k, v, None, dtype=np.float64)
    got, lse = O.attention_q8(z, origin=origin)
    err = np.abs(got - ref)
    assert err.max() < 2e-2 and err.mean() < 2e-3, (err.max(), err.mean())
    # the LSE of the unsmoothed scores: without the q . mean_k term it is off by ~0.2
    assert np.abs(lse - ref_lse).max() < 1e-2
    assert np.abs(lse - D ** -0.5 * z["q_kmean"] - ref_lse).max() > 0.1
    # uniform scores (q = 0): the output is the mean of the dequantised V
    z0 = O.quantize_qkv(np.zeros_like(q), k, v, origin=origin)
    pos = np.arange(S) - origin
    vd = O.e4m3_decode(z0["v8t"][:, :, pos]).transpose(0, 2, 1) * z0["v_scale"][:, None, :]
    o0, l0 = O.attention_q8(z0, origin=origin)
    np.testing.assert_allclose(o0, np.broadcast_to(vd.mean(1, keepdims=True), vd.shape),
                               rtol=0, atol=1e-12)
    np.testing.assert_allclose(l0, np.log(S), rtol=0, atol=1e-12)


def test_attention_q8_lazy_max_and_masks():
    # Against exact masked attention on the dequantised values, the only error left is the
    # e4m3 rounding of P (relative 2^-4 for normal values; absolute 2^-10 below 2^-6, where
    # the row sum is at least 2^(7-1.5)): |O - O_exact| <= 2^-4 sum_k w_k |v_k| +
    # 2^-15.5 sum_k |v_k|, whatever the slack; the LSE is exact (row sums of unrounded P).
    # A row with no keys has O = 0 and LSE = -inf.
    rng = np.random.default_rng(19)
    H, S, D = 1, 256, 64
    q, k, v = (O.bf16_round(rng.standard_normal((H, S, D)) * 2) for _ in range(3))
    z = O.quantize_qkv(q, k, v)
    tm = np.ones((H, S, S), bool)
    tm[:, 3, :] = False
    tm[:, :, 200:] = False
    r = np.arange(S)
    qd = z["q8"] * z["q_scale"][:, r // 32][:, :, None].astype(np.float64)
    kd = z["k8"] * z["k_scale"][:, r // 64][:, :, None].astype(np.float64)
    vd = O.e4m3_decode(z["v8t"][:, :, :S]).transpose(0, 2, 1) * z["v_scale"][:, None, :]
    ref_o, ref_l = O.masked_attention(qd, kd, vd, tm, dtype=np.float64)
    w, _ = O.masked_attention(qd, kd, np.eye(S)[None].repeat(H, 0), tm, dtype=np.float64)
    bound = 2.0 ** -4 * (w @ np.abs(vd)) + 2.0 ** -15.5 * (tm.astype(float) @ np.abs(vd))
    keep = np.ones(S, bool)
    keep[3] = False
    # (slack <= log2(448) - 7 keeps P = 2^(s - m + 7) inside e4m3's range)
    for slack in (0.0, 0.75, 1.5):
        o, l = O.attention_q8(z, tm, slack=slack)
        assert np.all(o[:, 3] == 0) and np.isneginf(l[:, 3]).all()
        assert np.all(np.abs(o - ref_o)[:, keep] <= bound[:, keep] + 1e-12), slack
        np.testing.assert_allclose(l[:, keep] - D ** -0.5 * z["q_kmean"][:, keep], ref_l[:, keep],
                                   rtol=0, atol=1e-9)
    # the bound is not loose by orders of magnitude: the rounding error does show
    assert np.abs(o - ref_o)[:, keep].max() > 0.05 * bound[:, keep].max()


@pytest.mark.parametrize("bs,D", [(64, 64), (128, 128)])
def test_replay_map_rows_equal_rows_of_the_full_replay(bs, D):
    rng = np.random.default_rng(bs + D)
    H, nb = 2, 4
    S = nb * bs
    q = O.bf16_round(rng.normal(size=(H, S, D)).astype(np.float32))
    k = O.bf16_round(rng.normal(size=(H, S, D)).astype(np.float32))
    _, lse = O.masked_attention(q, k, k, None, dtype=np.float64)
    lse = lse.astype(np.float32)
    kw = dict(scale=D ** -0.5, log_threshold=np.log(1e-3), video_blocks=nb, block_size=bs)
    full = O.replay_map(q, k, lse, q_off=0, k_off=0, **kw)
    blocks = [3, 0, 2]
    assert np.array_equal(O.replay_map_rows(q, k, lse, blocks, **kw), full[:, blocks])


@pytest.mark.parametrize("n,bpf,k", [(7, 3, 4), (30, 6, 20), (64, 16, 48)])
def test_video_mask_cells_equal_the_line_by_line_restatement(n, bpf, k):
    rng = np.random.default_rng(n + k)
    modes = [O.MODE_SPARSE, O.MODE_BLOCK_DIAGONAL, O.MODE_FULL, O.MODE_SPARSE]
    sel = np.stack([np.sort(rng.choice(3 * n - 1, size=k, replace=False)) for _ in modes])
    want = O.generate_mask_from_lines(sel, modes, seq_len=n * 64, block_size=64,
                                      video_tokens=n * 64, text_tokens=0, bpf=bpf,
                                      model_type="wan")
    assert np.array_equal(O.video_mask_cells(sel, modes, n, bpf), want)
    for h in (0, 1):  # and the scalar cell definition on a sample of cells
        for i, j in rng.integers(0, n, size=(50, 2)):
            assert want[h, i, j] == O.mask_cell(sel[h], modes[h], n, bpf, i, j)


# --------------------------------------------------------------------------------------
# error bounds of the int8/fp8 path (the GPU tests' contracts)
# --------------------------------------------------------------------------------------
def test_e4m3_flip_candidates_flag_every_value_a_small_change_can_reround():
    codes = O.e4m3_decode(np.arange(1, 126))  # positive finite codes
    mids = (codes[:-1] + codes[1:]) / 2
    tol = np.full(mids.shape, 1e-6)
    assert O.e4m3_flip_candidates(mids, tol).all()  # rounding midpoints
    assert not O.e4m3_flip_candidates(codes[1:-1], np.full(codes.size - 2, 1e-6)).any()
    assert not O.e4m3_flip_candidates(mids * (1 + 3e-6), tol).any()  # beyond tol
    # the property the kernel bound rests on: any relative change up to tol that changes
    # the rounding happens only at a flagged value
    rng = np.random.default_rng(21)
    p = np.exp2(rng.uniform(-12, 8.5, 200000))
    p[:5000] = mids[rng.integers(0, mids.size, 5000)] * (1 + rng.uniform(-5e-6, 5e-6, 5000))
    tol = 4e-6
    delta = rng.uniform(-tol, tol, p.size)
    moved = O.e4m3_encode(p * (1 + delta)) != O.e4m3_encode(p)
    assert moved.sum() > 100
    assert np.all(O.e4m3_flip_candidates(p, np.full(p.size, tol))[moved])


def _q8_case(seed, S=512, D=64, qscale=1.0, keys_per_row=None, density=1.0, origin=0):
    rng = np.random.default_rng(seed)
    q = O.bf16_round(rng.standard_normal((1, S, D)) * qscale)
    k = O.bf16_round(rng.standard_normal((1, S, D)) + 0.5)
    v = O.bf16_round(rng.standard_normal((1, S, D)))
    if keys_per_row is None:
        tm = rng.random((1, S, S)) < density
    else:
        tm = np.zeros((1, S, S), bool)
        for r in range(S):
            tm[0, r, rng.choice(S, keys_per_row, replace=False)] = True
    tm[:, :, 0] |= ~tm.any(axis=2)
    return q, k, v, tm, origin


_Q8_CASES = [dict(seed=1), dict(seed=2, keys_per_row=3, qscale=2.0),
             dict(seed=3, D=128, qscale=2.0, density=0.3),
             dict(seed=4, qscale=4.0, density=0.1, origin=-14)]


@pytest.mark.parametrize("case", range(len(_Q8_CASES)))
def test_q8_model_bound_covers_fp32_renderings_and_catches_larger_errors(case):
    # The kernel-vs-model contract: renderings of the same arithmetic whose P differ from
    # the fp64 model's by less than the flip tolerance (fp32 scores and exp2; a seeded
    # relative jitter of 2e-6) stay inside attention_q8_with_bound's bound; P errors of
    # 1e-3 (250x the tolerance) re-round weights that the bound does not allow for.
    q, k, v, tm, origin = _q8_case(**_Q8_CASES[case])
    z = O.quantize_qkv(q, k, v, origin=origin)
    o, lse, b = O.attention_q8_with_bound(z, tm, origin=origin)
    o0, lse0 = O.attention_q8(z, tm, origin=origin)
    assert np.array_equal(o, o0) and np.array_equal(lse, lse0)
    o32, _, _ = O.attention_q8_with_bound(z, tm, origin=origin, emulate_fp32=True)
    assert np.all(np.abs(o32 - o) <= b)
    oj, _, _ = O.attention_q8_with_bound(z, tm, origin=origin, p_jitter=2e-6, jitter_seed=case)
    assert np.all(np.abs(oj - o) <= b)
    ob, _, _ = O.attention_q8_with_bound(z, tm, origin=origin, p_jitter=1e-3, jitter_seed=case)
    assert (np.abs(ob - o) > b).sum() > 0
    # fp8 MFMA sums that err by up to the instruction's characterised allowance stay
    # inside; eight times that allowance does not
    om, _, _ = O.attention_q8_with_bound(z, tm, origin=origin, mfma_jitter=1.0, jitter_seed=case)
    assert np.all(np.abs(om - o) <= b)
    om8, _, _ = O.attention_q8_with_bound(z, tm, origin=origin, mfma_jitter=8.0,
                                          jitter_seed=case)
    assert (np.abs(om8 - o) > b).sum() > 0


def _exact_bound(q, k, v, z, tm, origin=0, drop=()):
    S = q.shape[1]
    pos = np.arange(S) - origin
    return O.q8_exact_error_bound(q[0], k[0], v[0], z["q8"][0], z["q_scale"][0][pos // 32],
                                  z["k8"][0], z["k_scale"][0][pos // 64], z["k_mean"][0],
                                  z["v_scale"][0], allowed=tm[0], drop=drop)


@pytest.mark.parametrize("case", range(len(_Q8_CASES)))
def test_q8_exact_bound_holds_for_the_modelled_arithmetic(case):
    # The kernel-vs-exact contract: the model of the kernel's arithmetic (int8 scores,
    # lazy max, e4m3 P and V, output rounded to bf16 like the kernel's) against exact
    # attention on the unquantised inputs stays inside q8_exact_error_bound, and not by
    # orders of magnitude (rows over many keys reach ~0.1 of it: the bound takes the
    # score errors as coherent; rows over few keys ~0.7).
    q, k, v, tm, origin = _q8_case(**_Q8_CASES[case])
    z = O.quantize_qkv(q, k, v, origin=origin)
    o8, _ = O.attention_q8(z, tm, origin=origin)
    o8 = O.bf16_round(o8[0].astype(np.float32)).astype(np.float64)
    o, b, E = _exact_bound(q, k, v, z, tm, origin)
    ref, _ = O.masked_attention(q, k, v, tm, dtype=np.float64)
    np.testing.assert_allclose(o, ref[0], rtol=0, atol=1e-12)
    r = np.abs(o8 - o) / b
    assert r.max() <= 1.0 and r.max() > 0.05, r.max()
    assert np.all(E >= 0)
    # renderings with fp32 scores and exp2, and with fp8 MFMA sums erring by the
    # instruction's characterised allowance, stay inside too
    for kw in (dict(emulate_fp32=True), dict(mfma_jitter=1.0, jitter_seed=case)):
        o2 = O.attention_q8_with_bound(z, tm, origin=origin, **kw)[0][0]
        o2 = O.bf16_round(o2.astype(np.float32)).astype(np.float64)
        assert np.all(np.abs(o2 - o) <= b), kw


def test_q8_exact_bound_needs_each_rounding_term():
    # Planted omissions: each term of the bound is needed by some input.
    # (1) e4m3 rounding of P and V: rows with three keys.
    q, k, v, tm, _ = _q8_case(seed=2, keys_per_row=3, qscale=2.0)
    z = O.quantize_qkv(q, k, v)
    o8 = O.bf16_round(O.attention_q8(z, tm)[0][0].astype(np.float32)).astype(np.float64)
    o, b, _ = _exact_bound(q, k, v, z, tm)
    _, b_no, _ = _exact_bound(q, k, v, z, tm, drop=("e4m3",))
    assert np.all(np.abs(o8 - o) <= b) and (np.abs(o8 - o) > b_no).sum() > 100
    # (2) values below e4m3's normal range: V entries of 1e-5 where the channel max is ~4
    # (a subnormal step, 2^-9 v_scale, is comparable to the value), read by one key each
    rng = np.random.default_rng(6)
    S, D = 256, 64
    q = O.bf16_round(rng.standard_normal((1, S, D)))
    k = O.bf16_round(rng.standard_normal((1, S, D)))
    v = O.bf16_round(rng.standard_normal((1, S, D)))
    v[:, 10:20] = O.bf16_round(np.full((1, 10, D), 1e-5, np.float32))
    tm = np.zeros((1, S, S), bool)
    tm[0, np.arange(S), 10 + np.arange(S) % 10] = True
    z = O.quantize_qkv(q, k, v)
    o8 = O.bf16_round(O.attention_q8(z, tm)[0][0].astype(np.float32)).astype(np.float64)
    o, b, _ = _exact_bound(q, k, v, z, tm)
    _, b_no, _ = _exact_bound(q, k, v, z, tm, drop=("subnormal",))
    assert np.all(np.abs(o8 - o) <= b) and (np.abs(o8 - o) > b_no).sum() > 100
    # (3) int8 scores: a 32-row block with one huge channel (that K leaves at zero) gets
    # coarse Q steps; rows of two keys with values +-1 turn the score error into output
    rng = np.random.default_rng(4)
    q = rng.standard_normal((1, S, D)) * 2
    q[:, ::32, 0] = 100.0
    k = rng.standard_normal((1, S, D))
    k[:, :, 0] = 0.0
    v = rng.standard_normal((1, S, D))
    q, k, v = (O.bf16_round(x.astype(np.float32)) for x in (q, k, v))
    tm = np.zeros((1, S, S), bool)
    for r in range(S):
        tm[0, r, rng.choice(S, 2, replace=False)] = True
    z = O.quantize_qkv(q, k, v)
    o8 = O.bf16_round(O.attention_q8(z, tm)[0][0].astype(np.float32)).astype(np.float64)
    o, b, _ = _exact_bound(q, k, v, z, tm)
    _, b_no, _ = _exact_bound(q, k, v, z, tm, drop=("score",))
    assert np.all(np.abs(o8 - o) <= b) and (np.abs(o8 - o) > b_no).sum() > 100
