"""Seeded random configurations through the attention kernels and the mask builder (GPU).

Each case draws heads, sequence length (aligned or ragged), head size, dtype, block size,
tile rows, mask density and, for text-first layouts, a shifted block grid. It checks:

- dense and block-sparse attention against fp64 attention under the executed mask, to
  the north-star bound (max-abs <= 2e-2, mean-abs <= 2e-3) and an LSE bound of 2e-3;
- the int8/fp8 block-sparse kernel against the oracle's model of its arithmetic (the
  bounds of tests/test_gpu_q8.py: 4e-3 max-abs, 3e-4 mean-abs, 2e-4 on the LSE);
- masks and tile lists generated from selected lines, bit-exactly.

The draws are fixed by the case index, so a failure names a reproducible configuration.
"""
import numpy as np
import pytest
import torch

import mod_dit_amd as md
import oracle as O
from mod_dit_amd import ops

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
    ref, ref_lse = O.attention_q8(zn, tm, origin=c["origin"])
    err = np.abs(_np(out[0]).astype(np.float64) - ref)
    print(f"  q8 max-abs {err.max():.3e} mean-abs {err.mean():.3e}", flush=True)
    assert err.max() <= 4e-3 and err.mean() <= 3e-4, (tag, err.max(), err.mean())
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
