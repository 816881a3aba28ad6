"""Seeded random configurations through the attention kernels and the mask builder (GPU).

Each case draws heads, sequence length (aligned or ragged), head size, dtype, block size,
tile rows, mask density and, for text-first layouts, a shifted block grid. It checks:

- dense and block-sparse attention against fp64 attention under the executed mask, to
  the north-star bound (max-abs <= 2e-2, mean-abs <= 2e-3) and an LSE bound of 2e-3;
- the int8/fp8 block-sparse kernel against the oracle's model of its arithmetic,
  elementwise within the bound derived from that arithmetic (tests/q8_contract.py), and
  2e-4 on the LSE;
- masks and tile lists generated from selected lines, bit-exactly;
- the replay map of exact (quarter-integer) scores against the oracle's replay of the
  same LSE, bit-exactly, for the wan, hunyuan and cogvideox layouts (partial last video
  blocks included), batches of 1-2;
- the fused dense + map kernel against the separate replay of its own LSE (bit-exact)
  and fp64 attention;
- the quantiser bit-exact on random shapes, grids and layouts; M^T S of fp32 maps within
  the worst-case fp32 summation bound; the refresh merge on strided masks (bit-exact);
- M^T S on arbitrary finite fp16 (bit-exact), the fit against the fp64 ridge solution
  (2e-6 of max|X|), and line selection with ties, signed zeros and NaN (bit-exact);
- batches of 1-3 in both input layouts with strided outputs, and dense attention with
  different query and key lengths;
- whole SparseAttentionWithMap schedules (W-2 .. W+T+1) on random wan, text-first
  cogvideox and hunyuan (padding mask) layers in bf16 and int8: every step's output
  against fp64 attention or the quantised oracle under the mask the state holds.

The draws are fixed by the case index, so a failure names a reproducible configuration.
"""
import numpy as np
import pytest
import torch

import mod_dit_amd as md
import oracle as O
from mod_dit_amd import ops
from q8_contract import check_q8_model

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().float().cpu().numpy()


def _randn(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype).to(DEV)


def _lists(tiles):
    c = tiles.counts.cpu().numpy()
    e = tiles.entries.cpu().numpy()
    return [[[int(x) for x in e[h, t, :c[h, t]]] for t in range(c.shape[1])] for h in range(c.shape[0])]


def _draw_attention(i):
    rng = np.random.default_rng(5000 + i)
    H = int(rng.integers(1, 4))
    D = int(rng.choice([64, 128]))
    dtype = [torch.bfloat16, torch.float16][int(rng.integers(0, 2))]
    union = bool(rng.integers(0, 2))
    shifted = bool(rng.random() < 0.3)
    bs = 64 if shifted else int(rng.choice([64, 128]))
    if shifted:
        text = int(rng.integers(1, 200))
        video = 64 * int(rng.integers(2, 30)) + int(rng.integers(0, 64))
        S = text + video
        tb, vb, origin = O.cogvideox_grid(text, video, bs)
        nb = tb + vb
    else:
        S = int(rng.integers(65, 2600))
        origin = 0
        nb = -(-S // bs)
    density = float(rng.uniform(0.05, 0.9))
    m = rng.random((H, nb, nb)) < density
    if rng.random() < 0.5:
        m[:, int(rng.integers(0, nb)), :] = False  # a block row that attends to nothing
    return dict(H=H, D=D, dtype=dtype, union=union, bs=bs, S=S, origin=origin, mask=m,
                seed=7000 + 10 * i)


@pytest.mark.parametrize("i", range(16))
def test_random_dense_and_block_sparse(i):
    c = _draw_attention(i)
    H, S, D, dtype = c["H"], c["S"], c["D"], c["dtype"]
    tag = (f"case {i}: H={H} S={S} D={D} {dtype} bs={c['bs']} union={c['union']} "
           f"origin={c['origin']} density={c['mask'].mean():.2f}")
    print(tag, flush=True)
    q, k, v = (_randn((1, H, S, D), c["seed"] + j, dtype) for j in range(3))
    qn, kn, vn = _np(q[0]), _np(k[0]), _np(v[0])
    out, lse = ops.flash_fwd(q, k, v)
    ref, ref_lse = O.masked_attention(qn, kn, vn, None, dtype=np.float64)
    err = np.abs(_np(out[0]).astype(np.float64) - ref)
    assert err.max() <= 2e-2 and err.mean() <= 2e-3, (tag, "dense", err.max(), err.mean())
    np.testing.assert_allclose(_np(lse[0]), ref_lse, rtol=0, atol=2e-3)

    tiles = ops.mask_to_tiles(torch.from_numpy(c["mask"]).to(DEV), c["bs"],
                              union_rows=c["union"], grid_origin=c["origin"])
    out, lse = ops.block_sparse_fwd(q, k, v, tiles, return_lse=True)
    tm = O.token_mask_from_tiles(_lists(tiles), H, S, S, origin=c["origin"])
    ref, ref_lse = O.masked_attention(qn, kn, vn, tm, dtype=np.float64)
    err = np.abs(_np(out[0]).astype(np.float64) - ref)
    print(f"  sparse max-abs {err.max():.3e} mean-abs {err.mean():.3e}", flush=True)
    assert err.max() <= 2e-2 and err.mean() <= 2e-3, (tag, "sparse", err.max(), err.mean())
    got_lse = _np(lse[0])
    assert np.array_equal(np.isfinite(got_lse), np.isfinite(ref_lse)), tag
    fin = np.isfinite(ref_lse)
    if fin.any():
        assert np.abs(got_lse[fin] - ref_lse[fin]).max() <= 2e-3, tag
    # rows whose block row is empty are written as zeros
    assert np.all(_np(out[0])[~np.isfinite(ref_lse)] == 0), tag


@pytest.mark.parametrize("i", range(8))
def test_random_int8_block_sparse_against_quantised_oracle(i):
    c = _draw_attention(100 + i)
    H, S, D = c["H"], c["S"], c["D"]
    dtype = torch.bfloat16
    tag = (f"case {i}: H={H} S={S} D={D} bs={c['bs']} union={c['union']} origin={c['origin']} "
           f"density={c['mask'].mean():.2f}")
    print(tag, flush=True)
    q, k, v = (_randn((1, H, S, D), c["seed"] + j, dtype) for j in range(3))
    tiles = ops.mask_to_tiles(torch.from_numpy(c["mask"]).to(DEV), c["bs"],
                              union_rows=c["union"], grid_origin=c["origin"])
    qz = ops.quantize_qkv(q, k, v, grid_origin=c["origin"])
    out, lse = ops.block_sparse_fwd_q8(qz, tiles, return_lse=True)
    zn = dict(q8=qz.q8[0].cpu().numpy(), q_scale=qz.q_scale[0].cpu().numpy(),
              k8=qz.k8[0].cpu().numpy(), k_scale=qz.k_scale[0].cpu().numpy(),
              v8t=qz.v8t[0].cpu().numpy(), v_scale=qz.v_scale[0].cpu().numpy(),
              k_mean=qz.k_mean[0].cpu().numpy(), q_kmean=qz.q_kmean[0].cpu().numpy())
    tm = O.token_mask_from_tiles(_lists(tiles), H, S, S, origin=c["origin"])
    ref, ref_lse = check_q8_model(out[0], zn, tm, origin=c["origin"], tag=tag)
    got_lse = _np(lse[0])
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isfinite(got_lse), fin), tag
    if fin.any():
        assert np.abs(got_lse[fin] - ref_lse[fin]).max() <= 2e-4, tag


@pytest.mark.parametrize("i", range(12))
def test_random_mask_from_lines_bit_exact(i):
    rng = np.random.default_rng(9000 + i)
    model_type = ["wan", "hunyuan", "cogvideox", "other"][int(rng.integers(0, 4))]
    bs = int(rng.choice([64, 128]))
    union = bool(rng.integers(0, 2))
    H = int(rng.integers(1, 6))
    bpf = int(rng.integers(1, 40))
    n = bpf * int(rng.integers(1, 12)) + int(rng.integers(0, bpf))
    n = max(n, 2)
    k = int(rng.integers(1, 3 * n))
    tb = int(rng.integers(1, 6)) if model_type in ("hunyuan", "cogvideox") else 0
    nb = n + tb
    sel = np.stack([rng.choice(3 * n - 1, size=k, replace=False) for _ in range(H)]).astype(np.int32)
    modes = rng.integers(0, 3, size=H).astype(np.uint8)
    tag = f"case {i}: {model_type} bs={bs} union={union} H={H} n={n} bpf={bpf} k={k} text={tb}"
    print(tag, flush=True)
    st = {"block_size": bs, "text_token_num": tb * bs, "video_token_num": n * bs,
          "model_type": model_type, "tile_rows": "union" if union else "exact"}
    mask, tiles = md.attn_mask._generate_mask_and_tiles(
        st, H, nb * bs, bpf, torch.from_numpy(sel).to(DEV), torch.from_numpy(modes).to(DEV),
        torch.device(DEV))
    ref = O.generate_mask_from_lines(sel, list(modes), seq_len=nb * bs, block_size=bs,
                                     video_tokens=n * bs, text_tokens=tb * bs, bpf=bpf,
                                     model_type=model_type)
    got = mask.cpu().numpy()
    assert got.shape == ref.shape and np.array_equal(got, ref), tag
    c_ref, l_ref = O.tiles_from_mask(ref, bs, union)
    c_got = tiles.counts.cpu().numpy()
    assert np.array_equal(c_got, c_ref), tag
    assert _lists(tiles) == [[[int(x) for x in t] for t in h] for h in l_ref], tag


# ---------------------------------------------------------------- replay map / fused pass
def _draw_map(i):
    rng = np.random.default_rng(11000 + i)
    model_type = ["wan", "hunyuan", "cogvideox"][int(rng.integers(0, 3))]
    bs = int(rng.choice([64, 128]))
    D = int(rng.choice([64, 128]))
    dtype = [torch.bfloat16, torch.float16][int(rng.integers(0, 2))]
    if model_type == "wan":
        text, video = 0, bs * int(rng.integers(2, 9))
    elif model_type == "hunyuan":
        text, video = int(rng.integers(1, 2 * bs)), bs * int(rng.integers(2, 9))
    else:  # text first; the video may end in a partial block
        text, video = int(rng.integers(1, 2 * bs)), int(rng.integers(2 * bs, 9 * bs))
    S = text + video
    B = int(rng.integers(1, 3))
    H = int(rng.integers(1, 3))
    # scores exact in fp32: multiples of 1/4 in [-2, 2] (d=64 and d=128 alike)
    qn = rng.integers(-8, 9, size=(B, H, S, D)).astype(np.float32) / 4
    kn = rng.integers(-8, 9, size=(B, H, S, D)).astype(np.float32) / 4
    thr = float(rng.choice([1e-2, 1e-3, 1e-4]))
    return dict(model_type=model_type, bs=bs, D=D, dtype=dtype, text=text, video=video, S=S,
                B=B, H=H, qn=qn, kn=kn, thr=thr)


@pytest.mark.parametrize("i", range(12))
def test_random_replay_map_bit_exact(i):
    """The replay map of exact scores against the oracle's replay of the same LSE."""
    import math

    c = _draw_map(i)
    tag = (f"case {i}: {c['model_type']} bs={c['bs']} D={c['D']} {c['dtype']} text={c['text']} "
           f"video={c['video']} B={c['B']} H={c['H']} thr={c['thr']}")
    print(tag, flush=True)
    q = torch.from_numpy(c["qn"]).to(c["dtype"]).to(DEV)
    k = torch.from_numpy(c["kn"]).to(c["dtype"]).to(DEV)
    D, bs = c["D"], c["bs"]
    scale = D ** -0.5
    s = np.einsum("bhqd,bhkd->bhqk", c["qn"].astype(np.float64), c["kn"].astype(np.float64)) * scale
    lse = np.log(np.exp(s).sum(-1)).astype(np.float32)
    vb, qo, ko = O.video_layout(c["model_type"], c["S"], c["video"], c["text"], bs)
    ln_thr = math.log(c["thr"])
    got = md.cuda_sparsity_map(q, k, torch.from_numpy(lse).to(DEV), softmax_scale=scale,
                               log_threshold=ln_thr, q_video_offset=qo, k_video_offset=ko,
                               video_blocks=vb, block_size=bs)
    dt = "bf16" if c["dtype"] == torch.bfloat16 else "fp16"
    for b in range(c["B"]):
        ref = O.replay_map(c["qn"][b], c["kn"][b], lse[b], scale=scale, log_threshold=ln_thr,
                           q_off=qo, k_off=ko, video_blocks=vb, block_size=bs, dtype=dt)
        assert np.array_equal(got[b].cpu().numpy(), ref), (tag, b)


@pytest.mark.parametrize("i", range(10))
def test_random_merged_replay_equals_full_replay_then_merge(i):
    """The refresh step's map (MoD/mod/attn_mask.py:659-675): the replay run only at the
    mask's active blocks and written into the previous map equals the full replay merged
    with where(mask == False, prev, full), bit for bit, for the three layouts, both block
    sizes, batches of one or two, and masks from empty (case 0) to all-True (case 1)."""
    import math

    c = _draw_map(300 + i)
    D, bs, B, H = c["D"], c["bs"], c["B"], c["H"]
    q = torch.from_numpy(c["qn"]).to(c["dtype"]).to(DEV)
    k = torch.from_numpy(c["kn"]).to(c["dtype"]).to(DEV)
    scale = D ** -0.5
    vb, qo, ko = O.video_layout(c["model_type"], c["S"], c["video"], c["text"], bs)
    rng = np.random.default_rng(500 + i)
    density = 0.0 if i == 0 else (1.0 if i == 1 else float(rng.uniform(0.05, 0.6)))
    mask = rng.random((H, vb, vb)) < density
    tag = (f"case {i}: {c['model_type']} bs={bs} D={D} {c['dtype']} text={c['text']} "
           f"video={c['video']} B={B} H={H} density={mask.mean():.2f}")
    print(tag, flush=True)
    lse = torch.randn((B, H, c["S"]), generator=torch.Generator().manual_seed(i)).to(DEV)
    ln_thr = math.log(c["thr"])
    kw = dict(softmax_scale=scale, log_threshold=ln_thr, q_video_offset=qo, k_video_offset=ko,
              video_blocks=vb, block_size=bs)
    full = ops.sparsity_map(q, k, lse, **kw)
    prev = torch.rand((B, H, vb, vb), generator=torch.Generator().manual_seed(50 + i))
    prev = prev.to(torch.float16).to(DEV)
    tiles = ops.mask_to_tiles(torch.from_numpy(mask).to(DEV), bs, union_rows=False)
    merged = prev.clone()
    ops.sparsity_map_merge(q, k, lse, tiles, merged, **kw)
    want = torch.where(torch.from_numpy(mask).to(DEV)[None], full, prev)
    assert torch.equal(merged, want), tag
    for b in range(B):
        ref = O.refresh_merge(prev[b].cpu().numpy(), full[b].cpu().numpy(), mask)
        assert np.array_equal(merged[b].cpu().numpy(), ref), (tag, b)


@pytest.mark.parametrize("i", range(6))
def test_random_fused_map_pass_equals_two_kernels(i):
    """The fused dense + map kernel: the map equals the separate replay of its own LSE."""
    import math

    c = _draw_map(100 + i)
    tag = (f"case {i}: {c['model_type']} bs={c['bs']} D={c['D']} {c['dtype']} text={c['text']} "
           f"video={c['video']} B={c['B']} H={c['H']}")
    print(tag, flush=True)
    q = torch.from_numpy(c["qn"]).to(c["dtype"]).to(DEV)
    k = torch.from_numpy(c["kn"]).to(c["dtype"]).to(DEV)
    v = _randn(tuple(q.shape), 12000 + i, c["dtype"])
    vb, qo, _ = O.video_layout(c["model_type"], c["S"], c["video"], c["text"], c["bs"])
    scale = c["D"] ** -0.5
    ln_thr = math.log(c["thr"])
    out, lse, smap = ops.flash_fwd_map(q, k, v, softmax_scale=scale, log_threshold=ln_thr,
                                       video_offset=qo, video_blocks=vb, block_size=c["bs"])
    sep = md.cuda_sparsity_map(q, k, lse, softmax_scale=scale, log_threshold=ln_thr,
                               q_video_offset=qo, k_video_offset=qo, video_blocks=vb,
                               block_size=c["bs"])
    assert torch.equal(sep, smap), tag
    for b in range(c["B"]):
        ref, ref_lse = O.masked_attention(c["qn"][b], c["kn"][b], _np(v[b]), None,
                                          dtype=np.float64)
        err = np.abs(_np(out[b]).astype(np.float64) - ref)
        assert err.max() <= 2e-2 and err.mean() <= 2e-3, (tag, b, err.max(), err.mean())
        np.testing.assert_allclose(_np(lse[b]), ref_lse, rtol=0, atol=2e-3)


# ---------------------------------------------------------------- M^T S, fit, selection
@pytest.mark.parametrize("i", range(10))
def test_random_mts_bit_exact(i):
    rng = np.random.default_rng(13000 + i)
    n = int(rng.integers(2, 900))
    bpf = int(rng.integers(1, max(2, n // 2)))
    H = int(rng.integers(1, 4))
    print(f"case {i}: n={n} bpf={bpf} H={H}", flush=True)
    bits = rng.integers(0, 0x7C00, size=(H, n, n)).astype(np.uint16)
    bits |= (rng.integers(0, 2, size=bits.shape) << 15).astype(np.uint16)
    S = bits.view(np.float16)
    got = md.compute_mts(torch.from_numpy(S.copy()).to(DEV), bpf).cpu().numpy()
    assert np.array_equal(got, O.mts_exact(S, bpf)), (n, bpf, H)


@pytest.mark.parametrize("i", range(6))
def test_random_fit_matches_fp64_ridge(i):
    rng = np.random.default_rng(14000 + i)
    bpf = int(rng.integers(2, 40))
    frames = int(rng.integers(2, 12))
    n = bpf * frames
    H = int(rng.integers(1, 5))
    print(f"case {i}: n={n} bpf={bpf} H={H}", flush=True)
    S = (rng.integers(0, 4097, size=(H, n, n)) / 4096.0).astype(np.float16)
    st = md.create_adaptive_mask_state("wan", H, n * 64, 0, bpf * 64, frames, block_size=64)
    feats = md.solve_lstsq(st, torch.from_numpy(S).to(DEV), step=st["warmup_steps"],
                           blocks_per_frame=bpf, regularization=1.0)
    X = O.ridge_solve(S.astype(np.float64), bpf, 1.0)
    got = feats["_x"].cpu().numpy().astype(np.float64)
    err = np.abs(got - X).max() / np.abs(X).max()
    print(f"  max err / max|X| = {err:.3e}", flush=True)
    assert err <= 2e-6, (n, bpf, H, err)


@pytest.mark.parametrize("i", range(10))
def test_random_select_lines_bit_exact(i):
    rng = np.random.default_rng(15000 + i)
    n = int(rng.integers(2, 700))
    k = int(rng.integers(1, 3 * n + 20))
    T = int(rng.integers(1, 20))
    H = int(rng.integers(1, 6))
    print(f"case {i}: n={n} k={k} T={T} H={H}", flush=True)
    xc = rng.normal(size=(H, 3 * n)).astype(np.float32)
    xl = rng.normal(size=(H, 3 * n)).astype(np.float32)
    # ties (quantised values), signed zeros and a NaN
    if rng.random() < 0.5:
        xc = np.round(xc * 4) / 4
        xl = np.round(xl * 4) / 4
    xc[0, int(rng.integers(0, 3 * n))] = 0.0
    xl[0, int(rng.integers(0, 3 * n))] = -0.0
    if rng.random() < 0.3:
        xc[H - 1, int(rng.integers(0, 3 * n))] = np.nan
    got = ops.select_lines(torch.from_numpy(xc).to(DEV), torch.from_numpy(xl).to(DEV), n, T, k)
    ref = O.choose_topk_lines(xc, xl, n, T, k)
    assert np.array_equal(got.cpu().numpy(), ref), (n, k, T, H)


# ---------------------------------------------------------------- whole schedules
def _schedule_wan_cogvideox(i, seed, vary_dtype_and_threshold=False):
    """One random wan / text-first cogvideox schedule (see the tests below)."""
    rng = np.random.default_rng(seed + i)
    model_type = ["wan", "cogvideox"][int(rng.integers(0, 2))]
    bs = int(rng.choice([64, 128]))
    tile_rows = ["exact", "union"][int(rng.integers(0, 2))]
    precision = ["bf16", "int8"][int(rng.integers(0, 2))]
    H = int(rng.integers(1, 4))
    D = int(rng.choice([64, 128]))
    F = int(rng.integers(2, 5))
    if model_type == "wan":
        text, tpf = 0, bs * int(rng.integers(2, 7))
    else:
        text, tpf = int(rng.integers(1, 150)), int(rng.integers(bs, 5 * bs))
    video = F * tpf
    S = text + video
    W, T = int(rng.integers(3, 6)), int(rng.integers(2, 4))
    n_v = -(-video // bs)
    top_k = int(rng.integers(1, max(2, 3 * n_v // 2)))
    dtype, thr = torch.bfloat16, 1e-3
    if vary_dtype_and_threshold:
        dtype = [torch.bfloat16, torch.float16][int(rng.integers(0, 2))]
        thr = float(10.0 ** rng.uniform(-4.5, -1.5))
    origin = O.cogvideox_grid(text, video, bs)[2] if model_type == "cogvideox" else 0
    tag = (f"case {i}: {model_type} bs={bs} {tile_rows} {precision} H={H} D={D} F={F} "
           f"tpf={tpf} text={text} W={W} T={T} top_k={top_k} {dtype} thr={thr:.2e}")
    print(tag, flush=True)
    st = md.create_adaptive_mask_state(model_type, H, video, text, tpf, F, warmup_steps=W,
                                       top_k=top_k, predict_T=T, threshold=thr,
                                       block_size=bs, tile_rows=tile_rows, precision=precision)
    base = [torch.randn(1, H, S, D, generator=torch.Generator().manual_seed(seed + 1000 + 10 * i + j))
            for j in range(3)]
    checked = 0
    for step in range(W - 2, W + T + 2):
        g = torch.Generator().manual_seed(seed + 2000 + 100 * i + step)
        q, k, v = ((b + 0.3 * torch.randn(b.shape, generator=g)).to(dtype).to(DEV)
                   for b in base)
        phase = O.step_phase(step, W, T)
        out, _ = md.SparseAttentionWithMap(q, k, v, st, None, current_step=step)
        qn, kn, vn = _np(q[0]), _np(k[0]), _np(v[0])
        if phase != "sparse":
            ref, _ = O.masked_attention(qn, kn, vn, None, dtype=np.float64)
            err = np.abs(_np(out[0]).astype(np.float64) - ref)
            assert err.max() <= 2e-2 and err.mean() <= 2e-3, (tag, step, phase, err.max())
            continue
        mask = st["mask"].cpu().numpy()
        _, lists = O.tiles_from_mask(mask, bs, tile_rows == "union")
        tm = O.token_mask_from_tiles(lists, H, S, S, origin=origin)
        if precision == "int8":
            # the kernels' 64-tile grid: 64 tokens later when 128-blocks start >= 64 early
            grid = origin + 64 if bs == 128 and origin <= -64 else origin
            qz = ops.quantize_qkv(q, k, v, grid_origin=grid)
            zn = dict(q8=qz.q8[0].cpu().numpy(), q_scale=qz.q_scale[0].cpu().numpy(),
                      k8=qz.k8[0].cpu().numpy(), k_scale=qz.k_scale[0].cpu().numpy(),
                      v8t=qz.v8t[0].cpu().numpy(), v_scale=qz.v_scale[0].cpu().numpy(),
                      k_mean=qz.k_mean[0].cpu().numpy(), q_kmean=qz.q_kmean[0].cpu().numpy())
            check_q8_model(out[0], zn, tm, origin=grid, tag=f"{tag} step {step}")
        else:
            ref, _ = O.masked_attention(qn, kn, vn, tm, dtype=np.float64)
            err = np.abs(_np(out[0]).astype(np.float64) - ref)
            bound = 2e-2 + (2.0 ** -9) * np.abs(ref)  # half a bf16 ulp where |o| is large
            assert np.all(err <= bound) and err.mean() <= 2e-3, (tag, step, err.max(), err.mean())
        print(f"  sparse step {step}: max-abs {err.max():.3e} mean-abs {err.mean():.3e}",
              flush=True)
        checked += 1
    assert checked >= 2, tag


@pytest.mark.parametrize("i", range(16))
def test_random_schedule_sparse_steps(i):
    """SparseAttentionWithMap over W-2 .. W+T+1 (map, fit, predict, sparse, refresh,
    sparse) on a random wan or text-first cogvideox layer in bf16 at threshold 1e-3.
    Every sparse step's output is checked against fp64 attention (bf16) or the oracle's
    model of the quantised arithmetic (int8) under the mask the state holds, as the
    kernels execute it; every map step's output against fp64 dense attention."""
    _schedule_wan_cogvideox(i, 16000)


@pytest.mark.parametrize("i", range(10))
def test_random_schedule_fp16_inputs_and_thresholds(i):
    """As above with bf16 or fp16 inputs (the reference runs CogVideoX in fp16) and map
    thresholds drawn from 3e-5 .. 3e-2."""
    _schedule_wan_cogvideox(i, 27000, vary_dtype_and_threshold=True)


def _zn(qz, b=0):
    """One batch element of a QuantizedQKV as the oracle's numpy dict."""
    return dict(q8=qz.q8[b].cpu().numpy(), q_scale=qz.q_scale[b].cpu().numpy(),
                k8=qz.k8[b].cpu().numpy(), k_scale=qz.k_scale[b].cpu().numpy(),
                v8t=qz.v8t[b].cpu().numpy(), v_scale=qz.v_scale[b].cpu().numpy(),
                k_mean=qz.k_mean[b].cpu().numpy(), q_kmean=qz.q_kmean[b].cpu().numpy())


@pytest.mark.parametrize("i", range(10))
def test_random_hunyuan_schedule_with_padding_mask(i):
    """Hunyuan layout (video first, a text tail of which only the first tokens are valid,
    the processor's padding mask): dense steps over the valid keys, map steps without the
    padding mask, sparse steps with video rows block-sparse over the key tiles below
    ceil(valid/64) and text rows dense over the valid keys."""
    rng = np.random.default_rng(19000 + i)
    bs = int(rng.choice([64, 128]))
    tile_rows = ["exact", "union"][int(rng.integers(0, 2))]
    precision = ["bf16", "int8"][int(rng.integers(0, 2))]
    H = int(rng.integers(1, 4))
    D = int(rng.choice([64, 128]))
    F = int(rng.integers(2, 4))
    tpf = bs * int(rng.integers(2, 6))
    video = F * tpf
    text = bs * int(rng.integers(1, 4))
    valid = video + int(rng.integers(0, text + 1))
    S = video + text
    W, T = int(rng.integers(3, 6)), int(rng.integers(2, 4))
    top_k = int(rng.integers(1, max(2, 3 * (video // bs) // 2)))
    tag = (f"case {i}: bs={bs} {tile_rows} {precision} H={H} D={D} F={F} tpf={tpf} "
           f"text={text} valid={valid} W={W} T={T} top_k={top_k}")
    print(tag, flush=True)
    st = md.create_adaptive_mask_state("hunyuan", H, video, text, tpf, F, warmup_steps=W,
                                       top_k=top_k, predict_T=T, threshold=1e-3,
                                       block_size=bs, tile_rows=tile_rows, precision=precision)
    pdm = torch.zeros(S, S, dtype=torch.bool, device=DEV)
    pdm[:, :valid] = True
    checked = 0
    for step in range(W + T + 1):
        g = torch.Generator().manual_seed(20000 + 100 * i + step)
        q, k, v = (torch.randn(1, H, S, D, generator=g).to(torch.bfloat16).to(DEV)
                   for _ in range(3))
        qn, kn, vn = _np(q[0]), _np(k[0]), _np(v[0])
        phase = O.step_phase(step, W, T)
        out, _ = md.SparseAttentionWithMap(q, k, v, st, None, pre_defined_mask=pdm,
                                           current_step=step, use_dense=step < W - 2)
        if phase == "dense":
            tm = np.zeros((H, S, S), bool)
            tm[:, :, :valid] = True
            ref, _ = O.masked_attention(qn, kn, vn, tm, dtype=np.float64)
        elif phase != "sparse":
            ref, _ = O.masked_attention(qn, kn, vn, None, dtype=np.float64)
        if phase == "dense" and precision == "int8":
            # the reference's dense branch: sageattn on the video queries over the valid
            # keys (K smoothed by their mean), bf16 text queries
            got = _np(out[0]).astype(np.float64)
            err_text = np.abs(got[:, video:] - ref[:, video:])
            assert err_text.max() <= 2e-2 and err_text.mean() <= 2e-3, (tag, step, "text rows")
            qz = ops.quantize_qkv(q[:, :, :valid], k[:, :, :valid], v[:, :, :valid])
            check_q8_model(got[:, :video], _zn(qz), rows=slice(0, video),
                           tag=f"{tag} step {step} {phase}")
            continue
        if phase != "sparse":
            err = np.abs(_np(out[0]).astype(np.float64) - ref)
            assert err.max() <= 2e-2 and err.mean() <= 2e-3, (tag, step, phase, err.max())
            continue
        mask = st["mask"].cpu().numpy()
        nbv = video // bs
        kv_tiles = (valid + 63) // 64
        _, lists = O.tiles_from_mask(mask[:, :nbv, :], bs, tile_rows == "union",
                                     kv_tiles=kv_tiles)
        tm = np.zeros((H, S, S), bool)
        tm[:, :video, :] = O.token_mask_from_tiles(lists, H, video, S)
        tm[:, video:, :valid] = True
        ref, _ = O.masked_attention(qn, kn, vn, tm, dtype=np.float64)
        got = _np(out[0]).astype(np.float64)
        err_text = np.abs(got[:, video:] - ref[:, video:])
        assert err_text.max() <= 2e-2 and err_text.mean() <= 2e-3, (tag, step, "text rows")
        if precision == "int8":
            check_q8_model(got[:, :video], _zn(ops.quantize_qkv(q, k, v)), tm,
                           rows=slice(0, video), tag=f"{tag} step {step}")
        else:
            err = np.abs(got[:, :video] - ref[:, :video])
            bound = 2e-2 + (2.0 ** -9) * np.abs(ref[:, :video])
            assert np.all(err <= bound) and err.mean() <= 2e-3, (tag, step, err.max(), err.mean())
        print(f"  sparse step {step}: video max-abs {err.max():.3e}", flush=True)
        checked += 1
    assert checked >= 1, tag


# ---------------------------------------------------------------- batches, layouts, lengths
@pytest.mark.parametrize("i", range(10))
def test_random_batches_layouts_and_cross_lengths(i):
    """Batches of 1-3 in (B,H,S,D) or the processors' (B,S,H,D)-strided layout, outputs
    into strided views; dense attention with a key length different from the query
    length; block-sparse with one per-head mask shared by the batch (every batch element
    checked on its own against fp64 under the executed mask)."""
    rng = np.random.default_rng(21000 + i)
    B = int(rng.integers(1, 4))
    H = int(rng.integers(1, 4))
    D = int(rng.choice([64, 128]))
    dtype = [torch.bfloat16, torch.float16][int(rng.integers(0, 2))]
    Sq = int(rng.integers(1, 1500))
    Skv = int(rng.integers(1, 1500))
    bshd = bool(rng.integers(0, 2))
    tag = f"case {i}: B={B} H={H} D={D} {dtype} Sq={Sq} Skv={Skv} bshd={bshd}"
    print(tag, flush=True)
    g = torch.Generator().manual_seed(22000 + i)

    def make(S):
        if bshd:
            return torch.randn((B, S, H, D), generator=g).to(dtype).to(DEV).transpose(1, 2)
        return torch.randn((B, H, S, D), generator=g).to(dtype).to(DEV)

    q, k, v = make(Sq), make(Skv), make(Skv)
    out_store = torch.full((B, Sq, H, D), float("nan"), dtype=dtype, device=DEV)
    out, lse = ops.flash_fwd(q, k, v, out=out_store.transpose(1, 2))
    assert not torch.isnan(out).any(), tag
    for b in range(B):
        ref, ref_lse = O.masked_attention(_np(q[b]), _np(k[b]), _np(v[b]), None, dtype=np.float64)
        err = np.abs(_np(out[b]).astype(np.float64) - ref)
        assert err.max() <= 2e-2 and err.mean() <= 2e-3, (tag, "dense", b, err.max())
        np.testing.assert_allclose(_np(lse[b]), ref_lse, rtol=0, atol=2e-3)
    # block-sparse self-attention on the query tensor's length, mask shared by the batch
    S = Sq
    k2, v2 = make(S), make(S)
    bs = int(rng.choice([64, 128]))
    nb = -(-S // bs)
    m = rng.random((H, nb, nb)) < float(rng.uniform(0.1, 0.8))
    union = bool(rng.integers(0, 2))
    tiles = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), bs, union_rows=union)
    out2_store = torch.full((B, S, H, D), float("nan"), dtype=dtype, device=DEV)
    out2, _ = ops.block_sparse_fwd(q, k2, v2, tiles, out=out2_store.transpose(1, 2))
    tm = O.token_mask_from_tiles(_lists(tiles), H, S, S)
    for b in range(B):
        ref, _ = O.masked_attention(_np(q[b]), _np(k2[b]), _np(v2[b]), tm, dtype=np.float64)
        err = np.abs(_np(out2[b]).astype(np.float64) - ref)
        assert err.max() <= 2e-2 and err.mean() <= 2e-3, (tag, "sparse", b, err.max())


# ---------------------------------------------------------------- quantiser, fp32 M^T S, merge
@pytest.mark.parametrize("i", range(8))
def test_random_quantiser_bit_exact(i):
    """The int8/fp8 quantiser on random shapes, grids, layouts and input offsets: every
    quantised tensor and scale bit-exact to the oracle given the kernel's K mean."""
    rng = np.random.default_rng(23000 + i)
    H = int(rng.integers(1, 4))
    S = int(rng.integers(1, 2000))
    D = int(rng.choice([64, 128]))
    dtype = [torch.bfloat16, torch.float16][int(rng.integers(0, 2))]
    origin = -int(rng.integers(0, 64)) if rng.random() < 0.5 else 0
    bshd = bool(rng.integers(0, 2))
    tag = f"case {i}: H={H} S={S} D={D} {dtype} origin={origin} bshd={bshd}"
    print(tag, flush=True)
    g = torch.Generator().manual_seed(24000 + i)
    shift = [float(rng.normal()) for _ in range(3)]
    if bshd:
        q, k, v = ((torch.randn((1, S, H, D), generator=g) * (1 + j) + shift[j])
                   .to(dtype).to(DEV).transpose(1, 2) for j in range(3))
    else:
        q, k, v = ((torch.randn((1, H, S, D), generator=g) * (1 + j) + shift[j])
                   .to(dtype).to(DEV) for j in range(3))
    qz = ops.quantize_qkv(q, k, v, grid_origin=origin)
    ref = O.quantize_qkv(_np(q[0]), _np(k[0]), _np(v[0]), k_mean=qz.k_mean[0].cpu().numpy(),
                         origin=origin)
    got = dict(q8=qz.q8[0].cpu().numpy(), q_scale=qz.q_scale[0].cpu().numpy(),
               k8=qz.k8[0].cpu().numpy(), k_scale=qz.k_scale[0].cpu().numpy(),
               v8t=qz.v8t[0].cpu().numpy(), v_scale=qz.v_scale[0].cpu().numpy())
    for name in got:
        assert got[name].shape == ref[name].shape and np.array_equal(got[name], ref[name]), \
            (tag, name)
    np.testing.assert_allclose(qz.k_mean[0].cpu().numpy(), _np(k[0]).astype(np.float64).mean(axis=1),
                               rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("i", range(6))
def test_random_mts_fp32_maps(i):
    rng = np.random.default_rng(25000 + i)
    n = int(rng.integers(2, 400))
    bpf = int(rng.integers(1, max(2, n // 2)))
    H = int(rng.integers(1, 4))
    S32 = rng.normal(size=(H, n, n)).astype(np.float32)
    got = md.compute_mts(torch.from_numpy(S32).to(DEV), bpf).cpu().numpy()
    want = np.stack([O.moddit_ref._mts_f64(S32[h].astype(np.float64), bpf) for h in range(H)])
    # worst case of an fp32 sum of m <= n*bpf terms in any order, plus the final rounding:
    # (m + 1) * 2^-24 * (sum of |terms|) per output; the sum of |terms| is M^T |S|
    mag = np.stack([O.moddit_ref._mts_f64(np.abs(S32[h]).astype(np.float64), bpf)
                    for h in range(H)])
    m = n * max(bpf, 1)
    assert np.all(np.abs(got - want) <= (m + 1) * 2.0 ** -24 * mag + 1e-30), (n, bpf, H)


@pytest.mark.parametrize("i", range(6))
def test_random_refresh_merge_exact(i):
    rng = np.random.default_rng(26000 + i)
    H, n = int(rng.integers(1, 5)), int(rng.integers(1, 300))
    pad = int(rng.integers(0, 9))
    prev = rng.random((H, n, n)).astype(np.float16)
    cur = rng.random((H, n, n)).astype(np.float16)
    full = rng.random((H, n + pad, n + pad)) < float(rng.uniform(0.05, 0.95))
    mask = torch.from_numpy(full).to(DEV)[:, :n, :n]  # a strided view when pad > 0
    got = ops.refresh_merge(torch.from_numpy(prev).to(DEV), torch.from_numpy(cur).to(DEV), mask)
    assert np.array_equal(got.cpu().numpy(), O.refresh_merge(prev, cur, full[:, :n, :n])), (H, n, pad)
