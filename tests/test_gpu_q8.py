"""Parity of the int8/fp8 (SageAttention2-style) path with the CPU oracle (GPU only).

- quantisation: bit-exact against the oracle's fp32 restatement (given the kernel's
  per-channel K mean, itself checked against the fp64 mean), on the unshifted and on a
  shifted grid, and deterministic; q . mean_k within fp32 summation error;
- attention: against fp64 attention on the same quantised values with the kernel's tile
  order and lazy row max modelled, elementwise within the bound derived from the
  arithmetic (tests/q8_contract.py: fp32 accumulation, bf16 output, and a re-rounded
  e4m3 weight only where the model's weight sits within fp32's error of a midpoint), and
  against exact attention on the unquantised inputs with the bf16 north-star bound at
  2048 keys (the quantisation error averages over the keys a row attends to; parity with
  the reference's SageAttention kernel itself is unpinned: that dependency is absent);
- LSE: within 2e-4 of the oracle's (fp32 row sums), and of the unsmoothed scores (the
  q . mean_k correction) within 2e-2 of exact attention.
"""
import numpy as np
import pytest
import torch

import mod_dit_amd as md  # noqa: F401  (loads the library)
import oracle as O
from mod_dit_amd import ops
from q8_contract import check_q8_model

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().float().cpu().numpy()


def _randn(shape, seed, dtype, scale=1.0, shift=0.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale + shift).to(dtype).to(DEV)


def _z_np(qz, b=0):
    return dict(q8=qz.q8[b].cpu().numpy(), q_scale=qz.q_scale[b].cpu().numpy(),
                k8=qz.k8[b].cpu().numpy(), k_scale=qz.k_scale[b].cpu().numpy(),
                v8t=qz.v8t[b].cpu().numpy(), v_scale=qz.v_scale[b].cpu().numpy(),
                k_mean=qz.k_mean[b].cpu().numpy(), q_kmean=qz.q_kmean[b].cpu().numpy())


def _check_lse(lse, ref, tag, atol):
    got = _np(lse)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(got), fin), tag
    err = np.abs(got[fin] - ref[fin]) if fin.any() else np.zeros(1)
    print(f"{tag}: LSE max-abs {err.max():.3e}", flush=True)
    assert err.max() <= atol, (tag, err.max())


def _check(out, ref, tag, max_abs, mean_abs):
    err = np.abs(_np(out).astype(np.float64) - ref)
    print(f"{tag}: max-abs {err.max():.3e} mean-abs {err.mean():.3e}", flush=True)
    assert err.max() <= max_abs and err.mean() <= mean_abs, (tag, err.max(), err.mean())


@pytest.mark.parametrize("H,S,D,dtype,strided,origin", [
    (2, 1000, 128, torch.bfloat16, False, 0),
    (3, 512, 64, torch.float16, True, 0),
    (2, 500, 64, torch.bfloat16, False, -14),
])
def test_quantize_matches_oracle(H, S, D, dtype, strided, origin):
    if strided:  # (B,S,H,D) storage viewed as (B,H,S,D)
        q, k, v = (_randn((1, S, H, D), 10 + i, dtype, shift=0.5 * i).transpose(1, 2)
                   for i in range(3))
    else:
        q, k, v = (_randn((1, H, S, D), 10 + i, dtype, shift=0.5 * i) for i in range(3))
    qz = ops.quantize_qkv(q, k, v, grid_origin=origin)
    qz2 = ops.quantize_qkv(q, k, v, grid_origin=origin)
    for name in ("q8", "q_scale", "k8", "k_scale", "v8t", "v_scale", "k_mean", "q_kmean"):
        assert torch.equal(getattr(qz, name), getattr(qz2, name)), name  # deterministic
    kn = _np(k[0]).astype(np.float64)
    np.testing.assert_allclose(qz.k_mean[0].cpu().numpy(), kn.mean(axis=1), rtol=1e-5, atol=1e-6)
    ref = O.quantize_qkv(_np(q[0]), _np(k[0]), _np(v[0]), k_mean=qz.k_mean[0].cpu().numpy(),
                         origin=origin)
    got = _z_np(qz)
    for name in ("q8", "q_scale", "k8", "k_scale", "v8t", "v_scale"):
        assert got[name].shape == ref[name].shape, name
        assert np.array_equal(got[name], ref[name]), name
    # fp32 sum of D products: within D ulps of the sum of magnitudes
    mag = np.einsum("hsd,hd->hs", np.abs(_np(q[0])), np.abs(got["k_mean"]).astype(np.float64))
    assert np.all(np.abs(got["q_kmean"] - ref["q_kmean"]) <= D * 2.0 ** -24 * mag + 1e-30)


@pytest.mark.parametrize("S,D,dtype", [(2048, 128, torch.bfloat16), (2048, 64, torch.float16),
                                       (1000, 128, torch.bfloat16)])
def test_q8_dense_attention(S, D, dtype):
    H = 2
    q, k, v = (_randn((1, H, S, D), 20 + i, dtype) for i in range(3))
    qz = ops.quantize_qkv(q, k, v)
    out, lse = ops.flash_fwd_q8(qz)
    assert out.dtype == dtype and out.shape == q.shape
    ref_q, ref_q_lse = check_q8_model(out[0], _z_np(qz), tag=f"q8 dense S={S} D={D}")
    ref, ref_lse = O.masked_attention(_np(q[0]), _np(k[0]), _np(v[0]), None, dtype=np.float64)
    err = np.abs(_np(out[0]) - ref)
    print(f"q8 dense vs exact S={S} D={D}: max-abs {err.max():.3e} mean-abs {err.mean():.3e}",
          flush=True)
    _check_lse(lse[0], ref_q_lse, f"q8 dense vs quantised oracle S={S} D={D}", 2e-4)
    if S >= 2048:
        _check(out[0], ref, f"q8 dense vs exact S={S} D={D}", 2e-2, 2e-3)
        _check_lse(lse[0], ref_lse, f"q8 dense vs exact S={S} D={D}", 2e-2)
    out2, _ = ops.flash_fwd_q8(qz)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("union", [False, True])
def test_q8_block_sparse_attention(union):
    H, S, D, bs = 2, 2048, 128, 64
    q, k, v = (_randn((1, H, S, D), 30 + i, torch.bfloat16) for i in range(3))
    rng = np.random.default_rng(3)
    m = rng.random((H, S // bs, S // bs)) < 0.4
    m[:, np.arange(S // bs), np.arange(S // bs)] = True
    m[:, 5, :] = False  # a block row with no keys
    tiles = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), bs, union_rows=union)
    qz = ops.quantize_qkv(q, k, v)
    out, lse = ops.block_sparse_fwd_q8(qz, tiles, return_lse=True)
    c = tiles.counts.cpu().numpy()
    e = tiles.entries.cpu().numpy()
    lists = [[[int(x) for x in e[h, t, :c[h, t]]] for t in range(c.shape[1])] for h in range(H)]
    tm = O.token_mask_from_tiles(lists, H, S, S)
    ref_q, ref_lse = check_q8_model(out[0], _z_np(qz), tm, tag=f"q8 sparse union={union}")
    _check_lse(lse[0], ref_lse, f"q8 sparse vs quantised oracle union={union}", 2e-4)
    if not union:  # with union rows, block row 5 shares its 128-row tile with row 4's keys
        assert torch.all(out[0, :, 5 * bs:6 * bs] == 0)
        assert torch.all(torch.isneginf(lse[0, :, 5 * bs:6 * bs]))


def test_q8_shifted_grid_cogvideox_layout():
    # 50 text + 450 video tokens: tiles on the grid that starts 14 tokens before token 0
    H, D, bs, text, video = 2, 64, 64, 50, 450
    S = text + video
    tb, vb, origin = O.cogvideox_grid(text, video, bs)
    q, k, v = (_randn((1, H, S, D), 40 + i, torch.bfloat16) for i in range(3))
    rng = np.random.default_rng(4)
    m = rng.random((H, tb + vb, tb + vb)) < 0.5
    m[:, :, 0] = True
    tiles = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), bs, union_rows=False, grid_origin=origin)
    with pytest.raises(ValueError, match="grid"):
        ops.block_sparse_fwd_q8(ops.quantize_qkv(q, k, v), tiles)  # quantised on another grid
    qz = ops.quantize_qkv(q, k, v, grid_origin=origin)
    out, lse = ops.block_sparse_fwd_q8(qz, tiles, return_lse=True)
    _, lists = O.tiles_from_mask(m, bs, union_rows=False)
    tm = O.token_mask_from_tiles(lists, H, S, S, origin=origin)
    ref_q, ref_lse = check_q8_model(out[0], _z_np(qz), tm, origin=origin, tag="q8 shifted grid")
    _check_lse(lse[0], ref_lse, "q8 shifted grid vs quantised oracle", 2e-4)


def test_q8_query_prefix():
    # queries 0..q_len-1 attend to all keys (the reference's video-query prefix against the
    # full key set); O and LSE hold q_len rows
    H, S, D, bs, q_len = 2, 1000, 64, 64, 640
    q, k, v = (_randn((1, H, S, D), 50 + i, torch.bfloat16) for i in range(3))
    rng = np.random.default_rng(5)
    m = rng.random((H, q_len // bs, (S + bs - 1) // bs)) < 0.4
    m[:, :, 0] = True
    tiles = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), bs, union_rows=True)
    qz = ops.quantize_qkv(q, k, v)
    out, lse = ops.block_sparse_fwd_q8(qz, tiles, return_lse=True, q_len=q_len)
    assert out.shape == (1, H, q_len, D) and lse.shape == (1, H, q_len)
    _, lists = O.tiles_from_mask(m, bs, union_rows=True)
    tm = np.zeros((H, S, S), bool)
    tm[:, :q_len] = O.token_mask_from_tiles(lists, H, q_len, S)
    ref_q, ref_lse = check_q8_model(out[0], _z_np(qz), tm, rows=slice(0, q_len),
                                    tag="q8 query prefix")
    _check_lse(lse[0], ref_lse[:, :q_len], "q8 query prefix vs quantised oracle", 2e-4)
    with pytest.raises(ValueError, match="q_len"):
        ops.block_sparse_fwd_q8(qz, tiles, q_len=S + 1)


def _sparse_mask(H, n, seed, p=0.35):
    rng = np.random.default_rng(seed)
    m = rng.random((H, n, n)) < p
    m[:, np.arange(n), np.arange(n)] = True
    return m


@pytest.mark.parametrize("layout", ["wan", "hunyuan"])
def test_engine_int8_precision(layout):
    """AttentionSparseEngine(precision='int8'): video queries on the quantised kernels (the
    reference engine's block_sparse_sage2_attn_cuda numerics), against the oracle on the
    same quantised tensors; Hunyuan text queries stay bf16 (exact attention, bf16 bound)."""
    import mod_dit_amd as md
    H, D, bs = 2, 64, 64
    if layout == "wan":
        video, text, valid = 2048, 0, 2048
    else:
        video, text, valid = 1536, 256, 1536 + 150
    S = video + text
    q, k, v = (_randn((1, H, S, D), 60 + i, torch.bfloat16) for i in range(3))
    n = S // bs
    m = _sparse_mask(H, n, 6)
    pdm = None
    if layout == "hunyuan":
        m[:, video // bs:, :] = True
        m[:, :, video // bs:] = True
        pdm = torch.zeros(S, S, dtype=torch.bool, device=DEV)
        pdm[:, :valid] = True
    out = md.AttentionSparseEngine(q, k, v, torch.from_numpy(m).to(DEV), pre_defined_mask=pdm,
                                   video_token_num=video, block_size=bs, precision="int8")
    qz = ops.quantize_qkv(q, k, v)  # deterministic: the tensors the engine quantised
    kv_tiles = (valid + 63) // 64 if layout == "hunyuan" else None
    _, lists = O.tiles_from_mask(m[:, :video // bs], bs, True, kv_tiles=kv_tiles)
    tm = np.zeros((H, S, S), bool)
    tm[:, :video] = O.token_mask_from_tiles(lists, H, video, S)
    check_q8_model(out[0, :, :video], _z_np(qz), tm, rows=slice(0, video),
                   tag=f"engine int8 {layout} video rows")
    if text:
        ref, _ = O.masked_attention(_np(q[0]), _np(k[0, :, :valid]), _np(v[0, :, :valid]), None,
                                    dtype=np.float64)
        _check(out[0, :, video:], ref[:, video:], f"engine int8 {layout} text rows", 2e-2, 2e-3)
    with pytest.raises(ValueError, match="precision"):
        md.AttentionSparseEngine(q, k, v, torch.from_numpy(m).to(DEV), precision="fp4")


@pytest.mark.parametrize("layout", ["wan", "hunyuan"])
def test_use_dense_int8_precision(layout):
    """SparseAttentionWithMap(use_dense=True) under precision='int8': the reference builds an
    all-True mask and its engine takes the dense branch, sageattn over the valid keys
    (MoD/mod/attn_mask.py:598-609,268-276), so the video queries run the quantised
    kernels with K smoothed by the mean of the valid keys only; Hunyuan text queries stay
    bf16 (its flashinfer call). Under precision='bf16' the call is the bf16 dense kernel."""
    import mod_dit_amd as md
    H, D, bs = 2, 128, 64
    if layout == "wan":
        video, text, valid = 1920, 0, 1920
    else:
        video, text, valid = 1536, 256, 1536 + 150
    S = video + text
    q, k, v = (_randn((1, H, S, D), 80 + i, torch.bfloat16) for i in range(3))
    pdm = None
    if layout == "hunyuan":
        pdm = torch.zeros(S, S, dtype=torch.bool, device=DEV)
        pdm[:, :valid] = True
    outs = {}
    for prec in ("int8", "bf16"):
        st = md.create_adaptive_mask_state(layout, H, video, text, 384, video // 384,
                                           warmup_steps=4, block_size=bs, precision=prec)
        outs[prec], info = md.SparseAttentionWithMap(q, k, v, st, None, pre_defined_mask=pdm,
                                                     current_step=0, use_dense=True)
        assert info == {"mode": "warmup", "mask": None}
    qz = ops.quantize_qkv(q[:, :, :valid], k[:, :, :valid], v[:, :, :valid])
    check_q8_model(outs["int8"][0, :, :video], _z_np(qz), rows=slice(0, video),
                   tag=f"use_dense int8 {layout} video rows")
    ref, _ = O.masked_attention(_np(q[0]), _np(k[0, :, :valid]), _np(v[0, :, :valid]), None,
                                dtype=np.float64)
    _check(outs["bf16"][0], ref, f"use_dense bf16 {layout}", 2e-2, 2e-3)
    if text:
        assert torch.equal(outs["int8"][0, :, video:], outs["bf16"][0, :, video:])
    # the quantised rows differ from the bf16 ones: the int8 path really ran
    assert not torch.equal(outs["int8"][0, :, :video], outs["bf16"][0, :, :video])


def test_schedule_int8_precision_cogvideox_shifted_grid():
    """create_adaptive_mask_state(precision='int8'): sparse steps of an unaligned CogVideoX
    layout (grid starting 14 tokens before the text) run the quantised kernels on the
    shifted grid; map steps stay bf16."""
    import mod_dit_amd as md
    H, D, bs = 2, 64, 64
    text, F, tpf = 50, 3, 150
    video = F * tpf
    S = text + video
    W, T = 4, 3
    tb, vb, origin = O.cogvideox_grid(text, video, bs)
    st = md.create_adaptive_mask_state("cogvideox", H, video, text, tpf, F, warmup_steps=W,
                                       top_k=6, predict_T=T, threshold=1e-3, block_size=bs,
                                       tile_rows="union", precision="int8")
    checked = 0
    for step in range(W + 2):
        g = torch.Generator().manual_seed(70 + step)
        q, k, v = ((torch.randn(1, H, S, D, generator=g)).to(torch.bfloat16).to(DEV)
                   for _ in range(3))
        phase = O.step_phase(step, W, T)
        out, _ = md.SparseAttentionWithMap(q, k, v, st, None, current_step=step,
                                           use_dense=step < W - 2)
        if phase != "sparse":
            continue
        mask = st["mask"].cpu().numpy()
        _, lists = O.tiles_from_mask(mask, bs, True)
        tm = O.token_mask_from_tiles(lists, H, S, S, origin=origin)
        qz = ops.quantize_qkv(q, k, v, grid_origin=origin)
        check_q8_model(out[0], _z_np(qz), tm, origin=origin,
                       tag=f"cogvideox int8 sparse step {step}")
        checked += 1
    assert checked == 2
    with pytest.raises(ValueError, match="precision"):
        md.create_adaptive_mask_state("wan", 2, 1024, 0, 512, 2, precision="fp8")


def test_short_tile_lists_bf16_and_int8():
    """Query tiles with 0..5 active key tiles: every prologue / prefetch / ring-wait branch
    of both attention kernels (the int8/fp8 ring keeps K three tiles ahead and V two, the
    bf16 ring one), with random row bits, against the oracle (bf16: fp64 attention, the
    north-star bound; int8/fp8: the quantised model, within its derived bound); rows without keys
    give zeros and an LSE of -inf."""
    H, S, D, bs = 2, 1536, 128, 64
    nb = S // bs
    q, k, v = (_randn((1, H, S, D), 60 + i, torch.bfloat16) for i in range(3))
    rng = np.random.default_rng(17)
    m = np.zeros((H, nb, nb), dtype=bool)
    want = np.zeros((H, nb // 2), dtype=np.int32)
    for h in range(H):
        for t in range(nb // 2):
            cnt = (t + 3 * h) % 6
            want[h, t] = cnt
            for kt in rng.choice(nb, size=cnt, replace=False):
                bits = int(rng.integers(1, 4))
                m[h, 2 * t, kt] = bool(bits & 1)
                m[h, 2 * t + 1, kt] = bool(bits & 2)
    tiles = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), bs, union_rows=False)
    assert np.array_equal(tiles.counts.cpu().numpy(), want)
    c = tiles.counts.cpu().numpy()
    e = tiles.entries.cpu().numpy()
    lists = [[[int(x) for x in e[h, t, :c[h, t]]] for t in range(c.shape[1])] for h in range(H)]
    tm = O.token_mask_from_tiles(lists, H, S, S)
    empty = ~tm.any(axis=-1)  # (H, S) rows without keys

    out, lse = ops.block_sparse_fwd(q, k, v, tiles, return_lse=True)
    ref, ref_lse = O.masked_attention(_np(q[0]), _np(k[0]), _np(v[0]), tm, dtype=np.float64)
    _check(out[0], ref, "bf16 short lists", 2e-2, 2e-3)
    _check_lse(lse[0], ref_lse, "bf16 short lists", 2e-3)
    assert torch.all(out[0][torch.from_numpy(empty).to(DEV)] == 0)

    qz = ops.quantize_qkv(q, k, v)
    out8, lse8 = ops.block_sparse_fwd_q8(qz, tiles, return_lse=True)
    ref8, ref8_lse = check_q8_model(out8[0], _z_np(qz), tm, tag="int8/fp8 short lists")
    _check_lse(lse8[0], ref8_lse, "int8/fp8 short lists", 2e-4)
    assert torch.all(out8[0][torch.from_numpy(empty).to(DEV)] == 0)
