"""Parity of every HIP kernel with the CPU oracle (GPU only).

Tolerances: integer/byte/index outputs are compared bit-exactly; attention outputs use
the north-star bound (max-abs <= 2e-2, mean-abs <= 2e-3 against fp32/fp64 attention on
the same bf16/fp16-rounded inputs and the same effective mask); map counts use the
reference test bounds (<= 2.1 counts per block against the same-LSE replay,
tests/test_flash_sparsity.py:100-101, and <= 8.1 against the fp32 probability map,
:138-139).
"""
import math

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


def _randn(shape, seed, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(DEV)


def _check_attn(out, ref, tag=""):
    err = np.abs(_np(out).astype(np.float64) - ref)
    print(f"{tag} max-abs {err.max():.3e} mean-abs {err.mean():.3e}", flush=True)
    assert err.max() <= 2e-2, tag
    assert err.mean() <= 2e-3, tag


# ====================================================================== dense attention
@pytest.mark.parametrize("H,S,D,dtype", [
    (2, 4096, 64, torch.bfloat16),    # the small plumbing shape (B=1, H=2, N=4096, d=64)
    (2, 1000, 128, torch.bfloat16),   # ragged tail (1000 = 7*128 + 104)
    (1, 640, 128, torch.float16),
    (3, 200, 64, torch.float16),
])
def test_flash_fwd_matches_fp64(H, S, D, dtype):
    q, k, v = (_randn((1, H, S, D), 100 + i, dtype) for i in range(3))
    out, lse = ops.flash_fwd(q, k, v)
    torch.cuda.synchronize()
    ref, ref_lse = O.masked_attention(_np(q[0]), _np(k[0]), _np(v[0]), None, dtype=np.float64)
    _check_attn(out[0], ref, f"dense H={H} S={S} D={D} {dtype}")
    np.testing.assert_allclose(_np(lse[0]), ref_lse, rtol=0, atol=2e-3)


def test_flash_fwd_strided_view_and_cross_lengths():
    B, H, S, D = 1, 2, 384, 128
    store = _randn((B, S, H, D), 7, torch.bfloat16)  # (B,S,H,D) storage
    q = store.transpose(1, 2)                          # (B,H,S,D) view, non-contiguous
    k = _randn((B, H, 700, D), 8, torch.bfloat16)
    v = _randn((B, H, 700, D), 9, torch.bfloat16)
    out, lse = ops.flash_fwd(q, k, v)
    ref, _ = O.masked_attention(_np(q[0]), _np(k[0]), _np(v[0]), None, dtype=np.float64)
    _check_attn(out[0], ref, "strided q, Skv=700")
    out2, _ = ops.flash_fwd(q.contiguous(), k, v)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("H,S,D,dtype", [
    (4, 8192, 128, torch.bfloat16),
    (6, 4544, 64, torch.bfloat16),
    (2, 3001, 128, torch.float16),
])
def test_flash_fwd_agrees_with_torch_sdpa_flash(H, S, D, dtype):
    """An independent GPU reference: torch's scaled_dot_product_attention restricted to its
    flash backend (AOTriton on ROCm) on the same inputs, to the north-star bound. Only the
    flash backend is allowed, so torch's math path never runs; the test skips when torch
    has no flash backend for this GPU."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    q, k, v = (_randn((1, H, S, D), 300 + i, dtype) for i in range(3))
    out, _ = ops.flash_fwd(q, k, v)
    try:
        with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
            ref = torch.nn.functional.scaled_dot_product_attention(q, k, v)
    except RuntimeError as e:  # no flash kernel for this dtype/shape/GPU
        pytest.skip(f"torch SDPA flash backend unavailable: {e}")
    torch.cuda.synchronize()
    err = (out.float() - ref.float()).abs()
    print(f"vs SDPA flash H={H} S={S} D={D} {dtype}: max-abs {err.max().item():.3e} "
          f"mean-abs {err.mean().item():.3e}", flush=True)
    assert err.max().item() <= 2e-2
    assert err.mean().item() <= 2e-3


# ====================================================================== tiles + sparse
def _random_block_mask(H, nb, density, seed, diag=True):
    rng = np.random.default_rng(seed)
    m = rng.random((H, nb, nb)) < density
    if diag:
        m[:, np.arange(nb), np.arange(nb)] = True
    return m


@pytest.mark.parametrize("model_type", ["wan", "hunyuan"])
@pytest.mark.parametrize("union", [False, True])
def test_mask_from_lines_beyond_one_column_pass(model_type, union):
    """nb > 2048 (256 threads x 8 columns): the kernel leaves its batched one-pass path and
    walks the columns in passes; the second pass here holds 53-56 columns, a partial
    thread and (hunyuan) the text columns."""
    rng = np.random.default_rng(1234 + union)
    H, n, bs, bpf, k = 3, 2101, 64, 30, 80
    tb = 3 if model_type == "hunyuan" else 0
    nb = n + tb
    sel = rng.integers(0, 3 * n - 1, size=(H, k)).astype(np.int32)
    modes = np.array([0, 1, 2], np.uint8)
    st = {"block_size": bs, "text_token_num": tb * bs, "video_token_num": n * bs,
          "model_type": model_type, "tile_rows": "union" if union else "exact"}
    mask, tiles = md.attn_mask._generate_mask_and_tiles(
        st, H, nb * bs, bpf, torch.from_numpy(sel).to(DEV),
        torch.from_numpy(modes).to(DEV), torch.device(DEV))
    ref = O.generate_mask_from_lines(sel, list(modes), seq_len=nb * bs, block_size=bs,
                                     video_tokens=n * bs, text_tokens=tb * bs, bpf=bpf,
                                     model_type=model_type)
    got = mask.cpu().numpy()
    assert got.shape == ref.shape and np.array_equal(got, ref)
    c, lists = _tiles_np(tiles)
    rc, rlists = O.tiles_from_mask(ref, bs, union)
    assert np.array_equal(c, rc) and lists == rlists


def _tiles_np(t: ops.TileList):
    c = t.counts.cpu().numpy()
    e = t.entries.cpu().numpy()
    return c, [[list(e[h, i, :c[h, i]]) for i in range(c.shape[1])] for h in range(c.shape[0])]


@pytest.mark.parametrize("union", [False, True])
@pytest.mark.parametrize("nb,bs", [(64, 64), (13, 64), (9, 128), (2113, 64)])
def test_mask_to_tiles_bit_exact(nb, bs, union):
    """nb=2113 walks the mask's columns in two passes (the second holds 65)."""
    m = _random_block_mask(3, nb, 0.4, nb + bs)
    tiles = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), bs, union_rows=union)
    c, lists = _tiles_np(tiles)
    rc, rlists = O.tiles_from_mask(m, bs, union)
    assert np.array_equal(c, rc)
    assert lists == rlists


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("union", [False, True])
def test_block_sparse_config1_matches_masked_fp64(union, dtype):
    # small plumbing shape: B=1, H=2, N=4096, d=64, 64x64 blocks, 50% random mask, diagonal
    # on; fp16 is the dtype the reference runs CogVideoX in (inference/cogvideo_test.py:48)
    H, S, D, bs = 2, 4096, 64, 64
    q, k, v = (_randn((1, H, S, D), 200 + i, dtype) for i in range(3))
    m = _random_block_mask(H, S // bs, 0.5, 5)
    tiles = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), bs, union_rows=union)
    out, lse = ops.block_sparse_fwd(q, k, v, tiles, return_lse=True)
    _, lists = _tiles_np(tiles)
    tm = O.token_mask_from_tiles(lists, H, S, S)
    if not union:
        assert np.array_equal(tm, O.token_mask_from_blocks(m, bs))
    ref, ref_lse = O.masked_attention(_np(q[0]), _np(k[0]), _np(v[0]), tm, dtype=np.float64)
    _check_attn(out[0], ref, f"sparse config1 union={union} {dtype}")
    np.testing.assert_allclose(_np(lse[0]), ref_lse, rtol=0, atol=2e-3)


def test_block_sparse_all_true_equals_dense_and_empty_rows_are_zero():
    H, S, D, bs = 2, 512, 128, 64
    q, k, v = (_randn((1, H, S, D), 300 + i, torch.bfloat16) for i in range(3))
    nb = S // bs
    full = torch.ones((H, nb, nb), dtype=torch.bool, device=DEV)
    t_full = ops.mask_to_tiles(full, bs, union_rows=False)
    o_sparse, _ = ops.block_sparse_fwd(q, k, v, t_full)
    o_dense, _ = ops.flash_fwd(q, k, v, return_lse=False)
    assert torch.equal(o_sparse, o_dense)
    m = full.clone()
    m[:, 3, :] = False  # rows 192..255 have no key block
    t = ops.mask_to_tiles(m, bs, union_rows=False)
    o, lse = ops.block_sparse_fwd(q, k, v, t, return_lse=True)
    assert torch.all(o[:, :, 192:256] == 0)
    assert torch.all(torch.isneginf(lse[:, :, 192:256]))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_block_sparse_bs128_mask(dtype):
    H, S, D, bs = 2, 1024, 128, 128
    q, k, v = (_randn((1, H, S, D), 400 + i, dtype) for i in range(3))
    m = _random_block_mask(H, S // bs, 0.3, 11)
    tiles = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), bs)
    out, _ = ops.block_sparse_fwd(q, k, v, tiles)
    ref, _ = O.masked_attention(_np(q[0]), _np(k[0]), _np(v[0]), O.token_mask_from_blocks(m, bs),
                                dtype=np.float64)
    _check_attn(out[0], ref, f"sparse bs128 {dtype}")


@pytest.mark.parametrize("S", [1041, 1088, 1089])
def test_block_sparse_bs128_tile_past_the_sequence_end(S):
    """A 128-token block mask on a sequence that ends in the first half of its last block
    (S mod 128 in 1..64) lists a 64-key tile wholly past the end. That entry holds no keys:
    outputs equal those of the lists without it (bit for bit) and fp64 attention.
    Regression: the kernels clamped the tile index and recomputed the last tile."""
    H, D, bs = 2, 128, 128
    nb = -(-S // bs)
    q, k, v = (_randn((1, H, S, D), 640 + i, torch.bfloat16) for i in range(3))
    m = _random_block_mask(H, nb, 0.5, 17)
    m[:, :, nb - 1] = True  # every query tile lists the last block's two key tiles
    full = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), bs, union_rows=False)
    clipped = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), bs, union_rows=False,
                                kv_tiles=-(-S // 64))
    past = S % 128 and S % 128 <= 64
    assert bool((full.counts > clipped.counts).any()) == bool(past)
    o_full, l_full = ops.block_sparse_fwd(q, k, v, full, return_lse=True)
    o_clip, l_clip = ops.block_sparse_fwd(q, k, v, clipped, return_lse=True)
    assert torch.equal(o_full, o_clip) and torch.equal(l_full, l_clip)
    tm = O.token_mask_from_blocks(m, bs)[:, :S, :S]
    ref, _ = O.masked_attention(_np(q[0]), _np(k[0]), _np(v[0]), tm, dtype=np.float64)
    _check_attn(o_full[0], ref, f"bs128 S={S}")
    qz = ops.quantize_qkv(q, k, v)
    o8_full, _ = ops.block_sparse_fwd_q8(qz, full)
    o8_clip, _ = ops.block_sparse_fwd_q8(qz, clipped)
    assert torch.equal(o8_full, o8_clip)


@pytest.mark.parametrize("text,video,D,union,dtype", [
    (50, 450, 64, False, torch.bfloat16), (50, 450, 128, True, torch.bfloat16),
    (226, 1350, 64, False, torch.bfloat16), (100, 200, 128, False, torch.bfloat16),
    (226, 1350, 64, False, torch.float16), (50, 450, 128, True, torch.float16),
])
def test_block_sparse_shifted_grid_matches_masked_fp64(text, video, D, union, dtype):
    # text-first sequence with text not block-aligned: the tile grid starts
    # origin = text - 64*ceil(text/64) tokens before token 0 (this build's padding rule)
    H, bs = 2, 64
    S = text + video
    tb, vb, origin = O.cogvideox_grid(text, video, bs)
    q, k, v = (_randn((1, H, S, D), 600 + i, dtype) for i in range(3))
    m = _random_block_mask(H, tb + vb, 0.35, 21)
    m[:, 1, :] = False  # a grid row whose queries attend to nothing
    tiles = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), bs, union_rows=union, grid_origin=origin)
    assert tiles.n_qtiles == -(-(S - origin) // 128)
    out, lse = ops.block_sparse_fwd(q, k, v, tiles, return_lse=True)
    _, lists = _tiles_np(tiles)
    tm = O.token_mask_from_tiles(lists, H, S, S, origin=origin)
    ref, ref_lse = O.masked_attention(_np(q[0]), _np(k[0]), _np(v[0]), tm, dtype=np.float64)
    _check_attn(out[0], ref, f"shifted grid text={text} video={video} D={D} union={union} {dtype}")
    np.testing.assert_allclose(_np(lse[0]), ref_lse, rtol=0, atol=2e-3)


def test_attention_kernels_are_deterministic():
    """Repeated calls give identical bits (regression: the tile DMA is inline asm, so the
    wait states after m0 / descriptor writes are the asm's job; a missing one showed as
    run-to-run differences)."""
    H, S, D, bs = 8, 8192, 128, 64
    q, k, v = (_randn((1, H, S, D), 700 + i, torch.bfloat16) for i in range(3))
    m = _random_block_mask(H, S // bs, 0.2, 31)
    tiles = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), bs, union_rows=False)
    runs = [(ops.flash_fwd(q, k, v), ops.block_sparse_fwd(q, k, v, tiles)) for _ in range(3)]
    for (d, sp) in runs[1:]:
        assert torch.equal(d[0], runs[0][0][0]) and torch.equal(d[1], runs[0][0][1])
        assert torch.equal(sp[0], runs[0][1][0])


@pytest.mark.parametrize("H,S,D", [
    (5, 16000, 64),   # 4 MB of K/V per head: one contiguous eighth of 625 tiles per XCD
    (3, 33024, 128),  # 8.5-17 MB per head: 32-tile runs dealt to the XCDs, 774 tiles =
                      # three whole rounds of 256 + 6 in the dispatcher's order
])
def test_multi_round_grid_writes_every_query_tile(H, S, D):
    """The workgroup -> tile order (contiguous eighths, or 32-tile runs dealt to the 8
    XCDs, chosen by the bytes of one head's key sweep) must be a permutation: every
    output row of the dense, block-sparse, int8/fp8 and replay-map kernels is written
    (outputs start as NaN and none may remain), and one row per query tile matches fp64
    attention."""
    bs = 64
    q, k, v = (_randn((1, H, S, D), 750 + i, torch.bfloat16) for i in range(3))
    m = _random_block_mask(H, S // bs, 0.3, 37)
    tiles = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), bs, union_rows=False)
    nan_out = lambda: torch.full_like(q, float("nan"))
    dense = ops.flash_fwd(q, k, v, return_lse=False, out=nan_out())[0]
    sparse = ops.block_sparse_fwd(q, k, v, tiles, out=nan_out())[0]
    qz = ops.quantize_qkv(q, k, v)
    dense8 = ops.flash_fwd_q8(qz, return_lse=False, out=nan_out())[0]
    sparse8 = ops.block_sparse_fwd_q8(qz, tiles, out=nan_out())[0]
    for name, o in (("dense", dense), ("sparse", sparse), ("dense q8", dense8),
                    ("sparse q8", sparse8)):
        assert not torch.isnan(o).any(), f"{name}: rows left unwritten"
    # a query tile computed in another tile's place would differ from the bf16 result
    assert (dense8.float() - dense.float()).abs().mean().item() <= 2e-3
    assert (sparse8.float() - sparse.float()).abs().mean().item() <= 2e-3

    t = np.arange(S // 128)
    rows = t * 128 + (t * 53) % 128  # one row per query tile, at varying positions
    qn, kn, vn = _np(q[0]), _np(k[0]), _np(v[0])
    ref_d, _ = O.masked_attention(qn[:, rows], kn, vn, None, dtype=np.float64)
    _check_attn(dense[0][:, rows], ref_d, "multi-round dense")
    tm = np.repeat(m[:, rows // bs, :], bs, axis=2)  # block mask at the sampled rows
    ref_s, _ = O.masked_attention(qn[:, rows], kn, vn, tm, dtype=np.float64)
    _check_attn(sparse[0][:, rows], ref_s, "multi-round block-sparse")

    # replay map through the C-ABI into a NaN-filled map
    _, lse = ops.flash_fwd(q, k, k)
    n = S // bs
    smap = torch.full((1, H, n, n), float("nan"), device=DEV, dtype=torch.float16)
    st = md._lib.strides3(*q.stride()[:3])
    rc = md._lib.load().moddit_sparsity_map(
        q.data_ptr(), k.data_ptr(), lse.data_ptr(), smap.data_ptr(), 1, H, S, D, st, st,
        D ** -0.5, math.log(1e-3), 0, 0, n, bs, md._lib.BF16,
        torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    assert not torch.isnan(smap).any(), "replay map: blocks left unwritten"
    assert torch.equal(smap, ops.sparsity_map(q, k, lse, softmax_scale=D ** -0.5,
                                              log_threshold=math.log(1e-3), q_video_offset=0,
                                              k_video_offset=0, video_blocks=n, block_size=bs))


# ====================================================================== sparsity map
def _layout(model_type, bs):
    # tests/test_flash_sparsity.py:22-25
    if model_type == "wan":
        return bs * 2, bs * 2, 0
    return bs * 3, bs * 2, bs


@pytest.mark.parametrize("model_type", ["hunyuan", "cogvideox", "wan"])
@pytest.mark.parametrize("bs", [64, 128])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_sparsity_map_dyadic_bit_exact(model_type, bs, D, dtype):
    S, vt, tt = _layout(model_type, bs)
    rng = np.random.default_rng(bs + D)
    qn = rng.integers(-4, 5, size=(2, 2, S, D)).astype(np.float32) / 8
    kn = rng.integers(-4, 5, size=(2, 2, S, D)).astype(np.float32) / 8
    q = torch.from_numpy(qn).to(dtype).to(DEV)
    k = torch.from_numpy(kn).to(dtype).to(DEV)
    scale = D ** -0.5
    s = np.einsum("bhqd,bhkd->bhqk", qn.astype(np.float64), kn.astype(np.float64)) * scale
    lse = np.log(np.exp(s).sum(-1)).astype(np.float32)
    vb, qo, ko = O.video_layout(model_type, S, vt, tt, bs)
    ln_thr = math.log(1e-3)
    got = md.cuda_sparsity_map(q, k, torch.from_numpy(lse).to(DEV), softmax_scale=scale,
                               log_threshold=ln_thr, q_video_offset=qo, k_video_offset=ko,
                               video_blocks=vb, block_size=bs)
    assert got.dtype == torch.float16 and got.shape == (2, 2, vb, vb)
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    for b in range(2):
        ref = O.replay_map(qn[b], kn[b], lse[b], scale=scale, log_threshold=ln_thr, q_off=qo,
                           k_off=ko, video_blocks=vb, block_size=bs, dtype=dt)
        assert np.array_equal(got[b].cpu().numpy(), ref), (model_type, bs, D, dtype, b)


@pytest.mark.parametrize("text,video,bs,D,dtype", [
    (40, 150, 64, 64, torch.bfloat16),    # 3 blocks, the last with 22 tokens
    (40, 150, 64, 128, torch.float16),
    (30, 200, 128, 128, torch.bfloat16),  # 2 blocks, the last with 72 tokens
    (30, 130, 128, 64, torch.bfloat16),   # the last 64-key tile lies wholly past the end
])
def test_sparsity_map_partial_last_block_dyadic_bit_exact(text, video, bs, D, dtype):
    S = text + video
    rng = np.random.default_rng(S + D)
    qn = rng.integers(-4, 5, size=(1, 2, S, D)).astype(np.float32) / 8
    kn = rng.integers(-4, 5, size=(1, 2, S, D)).astype(np.float32) / 8
    q = torch.from_numpy(qn).to(dtype).to(DEV)
    k = torch.from_numpy(kn).to(dtype).to(DEV)
    scale = D ** -0.5
    s = np.einsum("bhqd,bhkd->bhqk", qn.astype(np.float64), kn.astype(np.float64)) * scale
    lse = np.log(np.exp(s).sum(-1)).astype(np.float32)
    vb, qo, ko = O.video_layout("cogvideox", S, video, text, bs)
    assert qo + (vb - 1) * bs < S < qo + vb * bs
    ln_thr = math.log(1e-2)
    got = md.cuda_sparsity_map(q, k, torch.from_numpy(lse).to(DEV), softmax_scale=scale,
                               log_threshold=ln_thr, q_video_offset=qo, k_video_offset=ko,
                               video_blocks=vb, block_size=bs)
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    ref = O.replay_map(qn[0], kn[0], lse[0], scale=scale, log_threshold=ln_thr, q_off=qo,
                       k_off=ko, video_blocks=vb, block_size=bs, dtype=dt)
    assert np.array_equal(got[0].cpu().numpy(), ref), (text, video, bs, D, dtype)


@pytest.mark.parametrize("model_type,video,text,bs,D,dtype", [
    ("wan", 1024, 0, 64, 128, torch.bfloat16),
    ("hunyuan", 1024, 256, 128, 64, torch.float16),
    ("cogvideox", 450, 50, 64, 64, torch.bfloat16),    # partial last block, shifted grid
    ("cogvideox", 400, 130, 128, 128, torch.bfloat16),  # 128-blocks, grid origin -126
])
def test_flash_fwd_map_fused_pass(model_type, video, text, bs, D, dtype):
    """Dense pass + map in one kernel: the map is bit-exact to the replay of the kernel's
    own LSE (oracle and the separate replay kernel), O/LSE match the dense kernel.

    Q and K are multiples of 1/4 in [-2, 2], so every score is exact in fp32 and the
    probabilities span the threshold: the map holds dozens of distinct counts per head,
    and a key tile read from the wrong ring stage changes them."""
    S = video + text
    rng = np.random.default_rng(S + bs + D)
    qn = rng.integers(-8, 9, size=(1, 2, S, D)).astype(np.float32) / 4
    kn = rng.integers(-8, 9, size=(1, 2, S, D)).astype(np.float32) / 4
    q = torch.from_numpy(qn).to(dtype).to(DEV)
    k = torch.from_numpy(kn).to(dtype).to(DEV)
    v = _randn((1, 2, S, D), 900, dtype)
    scale = D ** -0.5
    vb, qo, _ = O.video_layout(model_type, S, video, text, bs)
    ln_thr = math.log(1e-3)
    out, lse, smap = ops.flash_fwd_map(q, k, v, softmax_scale=scale, log_threshold=ln_thr,
                                       video_offset=qo, video_blocks=vb, block_size=bs)
    assert smap.shape == (1, 2, vb, vb) and smap.dtype == torch.float16
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    ref = O.replay_map(qn[0], kn[0], _np(lse[0]), scale=scale, log_threshold=ln_thr, q_off=qo,
                       k_off=qo, video_blocks=vb, block_size=bs, dtype=dt)
    assert len(np.unique(ref)) >= 16  # an informative map, not a constant one
    assert np.array_equal(smap[0].cpu().numpy(), ref)
    sep = md.cuda_sparsity_map(q, k, lse, softmax_scale=scale, log_threshold=ln_thr,
                               q_video_offset=qo, k_video_offset=qo, video_blocks=vb, block_size=bs)
    assert torch.equal(sep, smap)
    # the dense pass is the dense kernel's algorithm in its range-checked instantiation
    # (FMA contraction may differ, so P can round differently): close to it, and
    # deterministic across calls
    o2, lse2 = ops.flash_fwd(q, k, v)
    assert ((out.float() - o2.float()).abs() <= 4e-3 + o2.float().abs() * 2.0 ** -7).all()
    if qo % 128 == 0:
        assert (lse - lse2).abs().max().item() <= 1e-5
    out3, lse3, smap3 = ops.flash_fwd_map(q, k, v, softmax_scale=scale, log_threshold=ln_thr,
                                          video_offset=qo, video_blocks=vb, block_size=bs)
    assert torch.equal(out3, out) and torch.equal(lse3, lse) and torch.equal(smap3, smap)
    ref_o, ref_lse = O.masked_attention(qn[0], kn[0], _np(v[0]), None, dtype=np.float64)
    _check_attn(out[0], ref_o, f"fused dense {model_type} bs={bs}")
    np.testing.assert_allclose(_np(lse[0]), ref_lse, rtol=0, atol=2e-3)


@pytest.mark.parametrize("bs", [64, 128])
@pytest.mark.parametrize("D", [64, 128])
def test_sparsity_map_randn_within_reference_count_bound(bs, D):
    # the reference's CUDA-vs-Triton bound (<= 2.1 counts) against the same-LSE replay
    torch.manual_seed(7)
    S = bs * 4
    q = torch.randn(2, 2, S, D).to(torch.bfloat16)
    k = torch.randn(2, 2, S, D).to(torch.bfloat16)
    scale = D ** -0.5
    sq = (q.float() * scale).to(torch.bfloat16).float()
    lse = torch.logsumexp(sq @ k.float().transpose(-1, -2), dim=-1)
    got = md.cuda_sparsity_map(q.to(DEV), k.to(DEV), lse.to(DEV), softmax_scale=scale,
                               log_threshold=math.log(1e-3), q_video_offset=0, k_video_offset=0,
                               video_blocks=S // bs, block_size=bs)
    for b in range(2):
        ref = O.replay_map(q[b].float().numpy(), k[b].float().numpy(), lse[b].numpy(),
                           scale=scale, log_threshold=math.log(1e-3), q_off=0, k_off=0,
                           video_blocks=S // bs, block_size=bs)
        err = np.abs(got[b].cpu().float().numpy() - ref.astype(np.float32)) * bs * bs
        assert err.max() <= 2.1
    g = got.float()
    assert torch.all((g >= 0) & (g <= 1))


@pytest.mark.parametrize("model_type", ["hunyuan", "cogvideox", "wan"])
@pytest.mark.parametrize("bs", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_public_api_matches_probability_reference(model_type, bs, dtype):
    # tests/test_flash_sparsity.py:107-139
    torch.manual_seed(11)
    S, vt, tt = _layout(model_type, bs)
    q = torch.randn(1, 2, S, 64).to(dtype)
    k = torch.randn_like(q)
    v = torch.randn_like(q)
    out, sp = md.flash_attn_with_sparsity_map(q.to(DEV), k.to(DEV), v.to(DEV), 1e-3, bs,
                                              model_type=model_type,
                                              video_token_num=vt if model_type != "wan" else 0,
                                              text_token_num=tt)
    assert out.shape == q.shape
    _, qo, ko = O.video_layout(model_type, S, vt, tt, bs)
    ref = O.probability_map(q[0].float().numpy(), k[0].float().numpy(), 1e-3, bs, qo, ko, vt)
    err = np.abs(sp[0].cpu().float().numpy() - ref) * bs * bs
    assert err.max() <= 8.1
    ref_o, _ = O.masked_attention(q[0].float().numpy(), k[0].float().numpy(), v[0].float().numpy(),
                                  None, dtype=np.float64)
    _check_attn(out[0], ref_o, "map pass output")


def test_non_positive_threshold_produces_zero_map():
    q = torch.randn(1, 1, 128, 64).to(torch.float16).to(DEV)
    out, sp = md.flash_attn_with_sparsity_map(q, q, q, 0.0, 64, model_type="wan")
    assert out.shape == q.shape
    assert torch.count_nonzero(sp).item() == 0


def test_kernels_use_current_stream():
    q = torch.randn(1, 1, 128, 64).to(torch.float16).to(DEV)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        out, sp = md.flash_attn_with_sparsity_map(q, q, q, 1e-3, 64, model_type="wan")
        marker = sp.float().sum() + out.float().sum()
    stream.synchronize()
    assert torch.isfinite(marker)


# ====================================================================== M^T S / solve
@pytest.mark.parametrize("n,bpf", [(64, 16), (100, 7), (1800, 60)])
def test_mts_bit_exact_on_map_domain(n, bpf):
    H = 2 if n > 500 else 3
    rng = np.random.default_rng(n)
    S = (rng.integers(0, 4097, size=(H, n, n)) / 4096.0).astype(np.float16)
    got = md.compute_mts(torch.from_numpy(S).to(DEV), bpf).cpu().numpy()
    assert np.array_equal(got, O.mts_exact(S, bpf))
    if n <= 100:
        loop = O.mts_loop(S, bpf)  # the reference's fp32 order: diag/col sums are exact
        assert np.array_equal(got[:, :-1], loop[:, :-1])


@pytest.mark.parametrize("n,bpf,H", [(37, 5, 2), (120, 9, 2), (2112, 64, 1)])
def test_mts_arbitrary_fp16_inputs(n, bpf, H):
    """Any finite fp16 (both signs, subnormals, up to 65504): exact sums rounded once.
    n=37: the scalar-load path; n=120: 16-byte loads; n=2112: 5 x 9 tiles of 512 rows x
    256 columns per head, the last row and column tiles partial (64 of 512 rows, 64 of 256
    columns)."""
    rng = np.random.default_rng(n)
    bits = rng.integers(0, 0x7C00, size=(H, n, n)).astype(np.uint16)
    bits |= (rng.integers(0, 2, size=bits.shape) << 15).astype(np.uint16)
    S = bits.view(np.float16)
    t = torch.from_numpy(S.copy()).to(DEV)
    got = md.compute_mts(t, bpf).cpu().numpy()
    assert np.array_equal(got, O.mts_exact(S, bpf))
    assert np.array_equal(md.compute_mts(t, bpf).cpu().numpy(), got)  # deterministic


def test_mts_non_finite_fp16_inputs_follow_float_semantics():
    """An output whose cells hold inf/NaN is the float sum of those values (NaN if a NaN
    or both infinities occur); the other outputs stay exact."""
    rng = np.random.default_rng(11)
    n, bpf = 48, 8
    S = (rng.integers(0, 4097, size=(1, n, n)) / 4096.0).astype(np.float16)
    S[0, 3, 5] = np.inf      # column 5, diagonal 2
    S[0, 7, 9] = -np.inf     # column 9, diagonal 2 as well -> NaN there
    S[0, 10, 10] = np.inf    # column 10, main diagonal, frame block 1
    S[0, 20, 40] = np.nan    # column 40, diagonal 20
    got = md.compute_mts(torch.from_numpy(S).to(DEV), bpf).cpu().numpy()[0]
    finite = np.where(np.isfinite(S), S, np.float16(0))
    want = O.mts_exact(finite, bpf)[0]
    nd = 2 * n - 1
    special = np.zeros(3 * n)
    for (r, c) in zip(*np.nonzero(~np.isfinite(S[0]))):
        v = float(S[0, r, c])
        idx = [nd + c, c - r + n - 1]
        if r // bpf == c // bpf:
            idx.append(3 * n - 1)
        for i in idx:
            special[i] = v if special[i] == 0 else special[i] + v
    want = np.where((special != 0) | np.isnan(special), special, want).astype(np.float32)
    np.testing.assert_array_equal(got, want)
    assert np.isnan(got[nd + 40]) and np.isnan(got[2 + n - 1])  # NaN cell; inf + -inf


def test_mts_fp32_inputs():
    rng = np.random.default_rng(3)
    n, bpf = 37, 5
    S32 = rng.normal(size=(2, n, n)).astype(np.float32)
    got32 = md.compute_mts(torch.from_numpy(S32).to(DEV), bpf).cpu().numpy()
    want = np.stack([O.moddit_ref._mts_f64(S32[h].astype(np.float64), bpf) for h in range(2)])
    np.testing.assert_allclose(got32, want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("n,bpf", [(64, 16), (270, 21), (1080, 60), (1800, 60)])
def test_solve_lstsq_matches_fp64_ridge(n, bpf):
    """The fit (M^T S kernel + the three fp64 Schur-complement kernels) against the fp64
    ridge solution of the full 3n x 3n system, up to the Wan-like (n=1080) and headline
    (n=1800) shapes: agreement to fp32 rounding of X, and the same selected lines as
    the oracle's selection on the fp64 fit."""
    rng = np.random.default_rng(n)
    H = 3
    S = (rng.integers(0, 4097, size=(H, n, n)) / 4096.0).astype(np.float16)
    st = md.create_adaptive_mask_state("wan", H, n * 64, 0, bpf * 64, n // bpf, block_size=64)
    feats = md.solve_lstsq(st, torch.from_numpy(S).to(DEV), step=st["warmup_steps"], blocks_per_frame=bpf,
                           regularization=1.0)
    X = O.ridge_solve(S.astype(np.float64), bpf, 1.0)
    got = feats["_x"].cpu().numpy().astype(np.float64)
    scale = np.abs(X).max()
    err = np.abs(got - X).max() / scale
    print(f"fit n={n}: max err / max|X| = {err:.3e}", flush=True)
    assert err <= 2e-6
    f = O.features_from_x(got.astype(np.float32), n)
    assert np.array_equal(feats["c"].cpu().numpy(), f["c"])
    zero_hist = np.zeros_like(X, dtype=np.float32)
    k = n // 3
    sel_gpu = O.choose_topk_lines(got.astype(np.float32), zero_hist, n, 10, k)
    sel_f64 = O.choose_topk_lines(X.astype(np.float32), zero_hist, n, 10, k)
    agree = np.mean([len(set(a) & set(b)) / k for a, b in zip(sel_gpu, sel_f64)])
    print(f"fit n={n}: selected-line agreement with the fp64 fit {agree:.5f}", flush=True)
    assert agree >= 0.999
    zero = md.solve_lstsq(st, torch.from_numpy(S).to(DEV), step=st["warmup_steps"] - 2, blocks_per_frame=bpf)
    assert torch.count_nonzero(zero["_x"]).item() == 0


# ====================================================================== select / modes
@pytest.mark.parametrize("n,k", [(8, 5), (64, 40), (1800, 400), (10, 1000)])
def test_select_lines_bit_exact(n, k):
    rng = np.random.default_rng(n + k)
    H = 4
    xc = rng.normal(size=(H, 3 * n)).astype(np.float32)
    xl = rng.normal(size=(H, 3 * n)).astype(np.float32)
    # inject exact ties, signed zeros and NaN
    xc[0, :6] = 0.5
    xl[0, :6] = 0.5
    xc[1, 3], xl[1, 3] = np.nan, 0.0
    xc[2, 2 * n - 1:2 * n + 3] = 0.0
    xl[2, 2 * n - 1:2 * n + 3] = -0.0
    got = ops.select_lines(torch.from_numpy(xc).to(DEV), torch.from_numpy(xl).to(DEV), n, 10, k)
    ref = O.choose_topk_lines(xc, xl, n, 10, k)
    assert np.array_equal(got.cpu().numpy(), ref)


def test_check_bd():
    x = torch.zeros(4, 9, device=DEV)
    x[:, -1] = torch.tensor([0.5, 1.0, 1.5, -3.0], device=DEV)
    mode = torch.tensor([0, 0, 0, 2], dtype=torch.uint8, device=DEV)
    ops.check_bd(x, mode, 1.0)
    assert mode.tolist() == [1, 1, 0, 2]


# ====================================================================== mask from lines
@pytest.mark.parametrize("model_type", ["wan", "hunyuan", "cogvideox", "other"])
@pytest.mark.parametrize("bs", [64, 128])
@pytest.mark.parametrize("union", [False, True])
@pytest.mark.parametrize("n,bpf,k", [(23, 4, 7), (301, 12, 60)])
def test_mask_from_lines_bit_exact(model_type, bs, union, n, bpf, k):
    """n=301: most threads own 8 consecutive video columns and read their diagonal bytes
    as one 8-byte window, at every alignment; threads at the text boundary and the last,
    partial thread take the per-column path."""
    rng = np.random.default_rng(hash((model_type, bs, union, n)) % 2**32)
    H = 5
    tb = 3 if model_type in ("hunyuan", "cogvideox") else 0
    nb = n + tb
    sel = rng.integers(0, 3 * n - 1, size=(H, k)).astype(np.int32)
    modes = np.array([0, 1, 2, 0, 1], np.uint8)
    st = {"block_size": bs, "text_token_num": tb * bs, "video_token_num": n * bs,
          "model_type": model_type, "tile_rows": "union" if union else "exact"}
    mask, tiles = md.attn_mask._generate_mask_and_tiles(
        st, H, nb * bs, bpf, torch.from_numpy(sel).to(DEV),
        torch.from_numpy(modes).to(DEV), torch.device(DEV))
    ref = O.generate_mask_from_lines(sel, list(modes), seq_len=nb * bs, block_size=bs,
                                     video_tokens=n * bs, text_tokens=tb * bs, bpf=bpf,
                                     model_type=model_type)
    got = mask.cpu().numpy()
    assert got.shape == ref.shape and np.array_equal(got, ref)
    c, lists = _tiles_np(tiles)
    rc, rlists = O.tiles_from_mask(ref, bs, union)
    assert np.array_equal(c, rc) and lists == rlists


def test_refresh_merge_exact():
    rng = np.random.default_rng(9)
    H, n = 3, 50
    prev = rng.random((H, n, n)).astype(np.float16)
    cur = rng.random((H, n, n)).astype(np.float16)
    full = rng.random((H, n + 4, n + 4)) < 0.5
    mask = torch.from_numpy(full).to(DEV)[:, :n, :n]  # strided view like the hunyuan slice
    got = ops.refresh_merge(torch.from_numpy(prev).to(DEV), torch.from_numpy(cur).to(DEV), mask)
    assert np.array_equal(got.cpu().numpy(), O.refresh_merge(prev, cur, full[:, :n, :n]))


@pytest.mark.parametrize("S", [0, 1, 17, 63, 64, 65, 127, 129])
def test_tiny_and_ragged_sequences(S):
    """Sequences shorter than one 64-key tile or one 128-row query tile, and one token past
    a tile boundary: dense, block-sparse (every block active) and int8/fp8 dense attention
    against the oracle; an empty sequence gives empty outputs."""
    H, D, bs = 2, 128, 64
    q, k, v = (_randn((1, H, S, D), 910 + i, torch.bfloat16) for i in range(3))
    out, lse = ops.flash_fwd(q, k, v)
    nb = max(1, -(-S // bs))
    tiles = ops.mask_to_tiles(torch.ones((H, nb, nb), dtype=torch.bool, device=DEV), bs,
                              union_rows=False)
    sp, sp_lse = ops.block_sparse_fwd(q, k, v, tiles, return_lse=True)
    qz = ops.quantize_qkv(q, k, v)
    o8, l8 = ops.flash_fwd_q8(qz)
    for t_, shape in ((out, (1, H, S, D)), (lse, (1, H, S)), (sp, (1, H, S, D)),
                      (o8, (1, H, S, D)), (l8, (1, H, S))):
        assert tuple(t_.shape) == shape
    if S == 0:
        return
    qn, kn, vn = _np(q[0]), _np(k[0]), _np(v[0])
    ref, ref_lse = O.masked_attention(qn, kn, vn, None, dtype=np.float64)
    _check_attn(out[0], ref, f"dense S={S}")
    _check_attn(sp[0], ref, f"block-sparse S={S}")
    np.testing.assert_allclose(_np(lse[0]), ref_lse, rtol=0, atol=2e-3)
    np.testing.assert_allclose(_np(sp_lse[0]), ref_lse, rtol=0, atol=2e-3)
    z = {name: getattr(qz, name)[0].cpu().numpy()
         for name in ("q8", "q_scale", "k8", "k_scale", "v8t", "v_scale", "k_mean", "q_kmean")}
    ref8, ref8_lse = check_q8_model(o8[0], z, tag=f"int8/fp8 dense S={S}")
    np.testing.assert_allclose(_np(l8[0]), ref8_lse, rtol=0, atol=2e-4)


def test_diagonal_block_mask_is_per_block_attention():
    """A mask holding only the diagonal 64x64 blocks equals attention inside each block on
    its own (computed block by block with the oracle), for the bf16 kernel in exact and
    union rows; union rows add the partner block of each 128-row tile."""
    H, S, D, bs = 2, 640, 128, 64
    nb = S // bs
    q, k, v = (_randn((1, H, S, D), 950 + i, torch.bfloat16) for i in range(3))
    m = np.zeros((H, nb, nb), dtype=bool)
    m[:, np.arange(nb), np.arange(nb)] = True
    qn, kn, vn = _np(q[0]), _np(k[0]), _np(v[0])
    for union in (False, True):
        tiles = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), bs, union_rows=union)
        out, _ = ops.block_sparse_fwd(q, k, v, tiles)
        span = 2 * bs if union else bs  # keys a row sees: its block, or its 128-row tile
        ref = np.zeros((H, S, D))
        for b0 in range(0, S, span):
            sl = slice(b0, b0 + span)
            ref[:, sl], _ = O.masked_attention(qn[:, sl], kn[:, sl], vn[:, sl], None,
                                               dtype=np.float64)
        _check_attn(out[0], ref, f"diagonal mask union={union}")
