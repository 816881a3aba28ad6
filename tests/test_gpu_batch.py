"""Batch > 1 through every attention-path kernel (GPU only).

Every kernel indexes (b, h) as b*H + h; block masks and tile lists are per head and
shared by the batch (MoD/mod/attn_mask.py:296-317 passes one (H, n, n) mask for the
whole batch). Each batch element is checked against the oracle on its own, with the
tolerances of the single-batch tests: attention max-abs <= 2e-2 / mean-abs <= 2e-3 vs
fp64; replay map counts <= 2.1 vs the same-LSE replay; quantiser bit-exact; int8/fp8
attention within the derived bound of the oracle's model of its arithmetic
(tests/q8_contract.py). Inputs are
(B,S,H,D) storage viewed as (B,H,S,D) (the processors' layout) with a ragged length.
"""
import math

import numpy as np
import pytest
import torch

import mod_dit_amd as md  # noqa: F401  (loads the library)
import oracle as O
from mod_dit_amd import ops
from q8_contract import check_q8_model

pytestmark = pytest.mark.gpu
DEV = "cuda"
B, H, S, D, BS = 2, 2, 1000, 64, 64


def _np(t):
    return t.detach().float().cpu().numpy()


def _inputs(seed, scaled=True):
    g = torch.Generator().manual_seed(seed)
    out = []
    for i in range(3):
        x = torch.randn((B, S, H, D), generator=g) * ((1.0 + 0.5 * i) if scaled else 1.0)
        out.append(x.to(torch.bfloat16).to(DEV).transpose(1, 2))  # (B,H,S,D) view
    return out


def _check(out, ref, tag, max_abs, mean_abs):
    err = np.abs(_np(out).astype(np.float64) - ref)
    print(f"{tag}: max-abs {err.max():.3e} mean-abs {err.mean():.3e}", flush=True)
    assert err.max() <= max_abs and err.mean() <= mean_abs, (tag, err.max(), err.mean())


def _mask():
    n = (S + BS - 1) // BS
    rng = np.random.default_rng(11)
    m = rng.random((H, n, n)) < 0.35
    m[:, np.arange(n), np.arange(n)] = True
    m[:, 3, :] = False  # a block row without keys
    return m


def test_batch_dense_and_block_sparse():
    q, k, v = _inputs(1)
    out, lse = ops.flash_fwd(q, k, v)
    assert out.shape == (B, H, S, D) and lse.shape == (B, H, S)
    m = _mask()
    tiles = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), BS, union_rows=False)
    # strided output: (B,S,H,D) storage
    sp_store = torch.empty((B, S, H, D), device=DEV, dtype=torch.bfloat16)
    _, sp_lse = ops.block_sparse_fwd(q, k, v, tiles, return_lse=True, out=sp_store.transpose(1, 2))
    _, lists = O.tiles_from_mask(m, BS, union_rows=False)
    tm = O.token_mask_from_tiles(lists, H, S, S)
    for b in range(B):
        qn, kn, vn = _np(q[b]), _np(k[b]), _np(v[b])
        ref, ref_lse = O.masked_attention(qn, kn, vn, None, dtype=np.float64)
        _check(out[b], ref, f"batch {b} dense", 2e-2, 2e-3)
        np.testing.assert_allclose(_np(lse[b]), ref_lse, rtol=0, atol=2e-3)
        ref_s, ref_sl = O.masked_attention(qn, kn, vn, tm, dtype=np.float64)
        _check(sp_store.transpose(1, 2)[b], ref_s, f"batch {b} block-sparse", 2e-2, 2e-3)
        fin = np.isfinite(ref_sl)
        assert np.array_equal(np.isfinite(_np(sp_lse[b])), fin)
        np.testing.assert_allclose(_np(sp_lse[b])[fin], ref_sl[fin], rtol=0, atol=2e-3)
    # the batch elements differ, so a (b, h) mix-up cannot pass both
    assert not torch.equal(out[0], out[1])


def test_batch_replay_map():
    q, k, _ = _inputs(2)
    _, lse = ops.flash_fwd(q, k, k)
    thr = 1e-3
    n = S // BS  # whole video blocks only
    smap = ops.sparsity_map(q, k, lse, softmax_scale=D ** -0.5, log_threshold=math.log(thr),
                            q_video_offset=0, k_video_offset=0, video_blocks=n, block_size=BS)
    assert smap.shape == (B, H, n, n)
    for b in range(B):
        rep = O.replay_map(_np(q[b]), _np(k[b]), _np(lse[b]), scale=D ** -0.5,
                           log_threshold=math.log(thr), q_off=0, k_off=0, video_blocks=n,
                           block_size=BS)
        err = np.abs(_np(smap[b]) - rep.astype(np.float32)) * BS * BS
        print(f"batch {b} replay map: max count diff {err.max():.2f}", flush=True)
        assert err.max() <= 2.1


def _z_np(qz, b):
    return dict(q8=qz.q8[b].cpu().numpy(), q_scale=qz.q_scale[b].cpu().numpy(),
                k8=qz.k8[b].cpu().numpy(), k_scale=qz.k_scale[b].cpu().numpy(),
                v8t=qz.v8t[b].cpu().numpy(), v_scale=qz.v_scale[b].cpu().numpy(),
                k_mean=qz.k_mean[b].cpu().numpy(), q_kmean=qz.q_kmean[b].cpu().numpy())


def test_batch_quantised_path():
    # unit-scale inputs: the int8/fp8 bounds include the bf16 rounding of outputs ~ N(0, 1/S)
    q, k, v = _inputs(3, scaled=False)
    qz = ops.quantize_qkv(q, k, v)
    dense, dense_lse = ops.flash_fwd_q8(qz)
    m = _mask()
    tiles = ops.mask_to_tiles(torch.from_numpy(m).to(DEV), BS, union_rows=True)
    sp_store = torch.empty((B, S, H, D), device=DEV, dtype=torch.bfloat16)
    _, sp_lse = ops.block_sparse_fwd_q8(qz, tiles, return_lse=True, out=sp_store.transpose(1, 2))
    _, lists = O.tiles_from_mask(m, BS, union_rows=True)
    tm = O.token_mask_from_tiles(lists, H, S, S)
    for b in range(B):
        ref = O.quantize_qkv(_np(q[b]), _np(k[b]), _np(v[b]), k_mean=qz.k_mean[b].cpu().numpy())
        z = _z_np(qz, b)
        for name in ("q8", "q_scale", "k8", "k_scale", "v8t", "v_scale"):
            assert np.array_equal(z[name], ref[name]), (b, name)
        ref_d, ref_dl = check_q8_model(dense[b], z, tag=f"batch {b} int8 dense")
        np.testing.assert_allclose(_np(dense_lse[b]), ref_dl, rtol=0, atol=2e-4)
        ref_s, ref_sl = check_q8_model(sp_store.transpose(1, 2)[b], z, tm,
                                       tag=f"batch {b} int8 block-sparse")
        fin = np.isfinite(ref_sl)
        assert np.array_equal(np.isfinite(_np(sp_lse[b])), fin)
        np.testing.assert_allclose(_np(sp_lse[b])[fin], ref_sl[fin], rtol=0, atol=2e-4)
