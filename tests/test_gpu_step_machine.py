"""End-to-end schedule of SparseAttentionWithMap against the oracle (GPU only).

Runs a short MOD-DiT schedule (W=4, T=3) on a wan-layout layer and checks, stage by
stage and given identical inputs to each stage: the map against the replay oracle
(reference count bound), the fit against the fp64 ridge solve, modes, the selected
lines and the mask bit-exactly, the refresh merge bit-exactly, and every attention
output against fp64 attention under the mask the kernels executed.
"""
import math

import numpy as np
import pytest
import torch

import mod_dit_amd as md
import oracle as O
from mod_dit_amd import ops
from q8_contract import check_q8_exact, check_q8_model

pytestmark = pytest.mark.gpu
DEV = "cuda"


class _Log:
    def __init__(self):
        self.lines = []

    def isEnabledFor(self, level):
        return True

    def info(self, msg):
        self.lines.append(msg)


def _np(t):
    return t.detach().float().cpu().numpy()


def _check_attn(out, ref, tag, sparse=False):
    """North-star bound (max-abs 2e-2, mean-abs 2e-3). Sparse rows attend to few keys, so
    outputs can reach |o| ~ 4, where the bf16 output quantum alone is 2^-7: there the
    elementwise bound also admits half a bf16 ulp of |ref| (2^-9 |ref|). How many
    elements use that slack is printed, and they must be rare (<= 0.1 %) and large
    (|ref| >= 1, where half an ulp is >= 2^-9)."""
    err = np.abs(_np(out).astype(np.float64) - ref)
    bound = 2e-2 + (2.0 ** -9) * np.abs(ref) if sparse else 2e-2
    slack = err > 2e-2
    n_slack = int(slack.sum())
    print(f"{tag}: max-abs {err.max():.3e} mean-abs {err.mean():.3e} "
          f"beyond 2e-2: {n_slack} of {err.size}", flush=True)
    assert np.all(err <= bound) and err.mean() <= 2e-3, (tag, err.max(), err.mean())
    assert n_slack <= 1e-3 * err.size, (tag, n_slack)
    assert np.all(np.abs(ref[slack]) >= 1.0), (tag, "slack used at |ref| < 1")


def _structured_qkv(H, F, tpf, D, seed):
    g = torch.Generator().manual_seed(seed)
    N = F * tpf
    pos = torch.arange(N) % tpf
    emb = torch.randn(tpf, D, generator=g) * 1.5
    q = torch.randn(1, H, N, D, generator=g) + emb[pos]
    k = torch.randn(1, H, N, D, generator=g) + emb[pos]
    v = torch.randn(1, H, N, D, generator=g)
    return (t.to(torch.bfloat16).to(DEV) for t in (q, k, v))


@pytest.mark.parametrize("tile_rows", ["exact", "union"])
def test_schedule_matches_oracle_stage_by_stage(tile_rows):
    H, F, tpf, D, bs = 2, 4, 512, 64, 64
    W, T, top_k, thr = 4, 3, 40, 1e-3
    N = F * tpf
    n, bpf = N // bs, tpf // bs
    st = md.create_adaptive_mask_state("wan", H, N, 0, tpf, F, warmup_steps=W, top_k=top_k,
                                       predict_T=T, threshold=thr, block_size=bs,
                                       tile_rows=tile_rows)
    log = _Log()
    history_x = []
    for step in range(W + 2 * T + 2):
        q, k, v = _structured_qkv(H, F, tpf, D, seed=step)
        qn, kn, vn = (_np(t[0]) for t in (q, k, v))
        phase = O.step_phase(step, W, T)
        use_dense = step < W - 2  # the processors' gate
        prev_mask = st.get("mask")
        prev_maps = st.get("prev_full_maps")
        out, info = md.SparseAttentionWithMap(q, k, v, st, log, current_step=step, layer_idx=0,
                                              use_dense=use_dense)
        assert out.shape == q.shape
        if phase == "dense":
            ref, _ = O.masked_attention(qn, kn, vn, None, dtype=np.float64)
            _check_attn(out[0], ref, f"dense step {step}")
            assert info == {"mode": "warmup", "mask": None}
            continue
        if phase in ("map_fit", "map_fit_predict", "refresh"):
            # output of a map step is the dense pass
            ref, ref_lse = O.masked_attention(qn, kn, vn, None, dtype=np.float64)
            _check_attn(out[0], ref, f"map-step output {step}")
            # features: the fit of the map this step produced (or merged)
            feats = st["features_history"][-1]
            X = feats["_x"].cpu().numpy().astype(np.float64)
            S_fit = st["prev_full_maps"].cpu().numpy()
            if step == W - 2:
                assert np.all(X == 0)  # zero features at W-2
            else:
                Xr = O.ridge_solve(S_fit.astype(np.float64), bpf, 1.0)
                assert np.abs(X - Xr).max() <= 2e-6 * max(np.abs(Xr).max(), 1e-6)
            if phase == "refresh":
                # prev = where(mask, current map, prev) over the video blocks
                smap = md.flash_attn_with_sparsity_map(q, k, v, thr, bs, model_type="wan")[1][0]
                merged = O.refresh_merge(prev_maps.cpu().numpy(), smap.cpu().numpy(),
                                         prev_mask.cpu().numpy())
                assert np.array_equal(S_fit, merged)
            else:
                # the map is the replay of this step's inputs (reference count bound)
                _, lse = ops.flash_fwd(q, k, v)
                rep = O.replay_map(qn, kn, _np(lse[0]), scale=D ** -0.5,
                                   log_threshold=math.log(thr), q_off=0, k_off=0,
                                   video_blocks=n, block_size=bs)
                err = np.abs(S_fit.astype(np.float32) - rep.astype(np.float32)) * bs * bs
                assert err.max() <= 2.1
        if phase in ("map_fit_predict", "refresh"):
            hist = st["features_history"]
            assert len(hist) == 2
            xc, xl = (f["_x"].cpu().numpy() for f in hist[-1:] + hist[-2:-1])
            if phase == "map_fit_predict":
                modes = [O.MODE_BLOCK_DIAGONAL if x <= 1.0 else O.MODE_SPARSE for x in xc[:, -1]]
                assert list(st["mode"]) == ["block_diagonal" if m else "sparse" for m in modes]
                assert any("Mask Sparsity" in l for l in log.lines)
            modes = [O.MODE_BLOCK_DIAGONAL if m == "block_diagonal" else O.MODE_SPARSE
                     for m in st["mode"]]
            sel = O.choose_topk_lines(xc, xl, n, T, top_k)
            mask_ref = O.generate_mask_from_lines(sel, modes, seq_len=N, block_size=bs,
                                                  video_tokens=N, text_tokens=0, bpf=bpf,
                                                  model_type="wan")
            assert np.array_equal(st["mask"].cpu().numpy(), mask_ref)
            history_x.append(xc)
        if phase == "sparse":
            mask = st["mask"].cpu().numpy()
            counts, lists = O.tiles_from_mask(mask, bs, tile_rows == "union")
            tm = O.token_mask_from_tiles(lists, H, N, N)
            ref, _ = O.masked_attention(qn, kn, vn, tm, dtype=np.float64)
            _check_attn(out[0], ref, f"sparse step {step}", sparse=True)
            assert info["mask"] is st["mask"]
    assert len(history_x) == 3  # predict at W-1 and refreshes at W+T-1, W+2T-1


@pytest.mark.parametrize("tile_rows", ["exact", "union"])
@pytest.mark.parametrize("bs", [64, 128])
def test_hunyuan_text_tail_with_padding_mask(tile_rows, bs):
    """Hunyuan layout: video first, then text of which only `valid_text` tokens are real.

    Dense steps attend to the valid keys; sparse steps run video queries block-sparse over
    the key tiles below ceil(valid/64) (MoD/mod/attn_mask.py:310-317) and text queries
    densely over the valid keys (:319-330).
    """
    H, F, tpf, D = 2, 3, 512, 64
    video, text, valid_text = F * tpf, 256, 150
    S = video + text
    W, T, top_k, thr = 4, 3, 30, 1e-3
    st = md.create_adaptive_mask_state("hunyuan", H, video, text, tpf, F, warmup_steps=W,
                                       top_k=top_k, predict_T=T, threshold=thr, block_size=bs,
                                       tile_rows=tile_rows)
    valid = video + valid_text
    pdm = torch.zeros(S, S, dtype=torch.bool, device=DEV)
    pdm[:, :valid] = True
    for step in range(W + T):
        q, k, v = _structured_qkv(H, 1, S, D, seed=100 + step)
        qn, kn, vn = (_np(t[0]) for t in (q, k, v))
        phase = O.step_phase(step, W, T)
        out, _ = md.SparseAttentionWithMap(q, k, v, st, None, pre_defined_mask=pdm,
                                           current_step=step, use_dense=step < W - 2)
        if phase == "dense":
            tm = np.zeros((H, S, S), bool)
            tm[:, :, :valid] = True
            ref, _ = O.masked_attention(qn, kn, vn, tm, dtype=np.float64)
            _check_attn(out[0], ref, f"hunyuan dense {step}")
        elif phase == "sparse":
            mask = st["mask"].cpu().numpy()
            nbv = video // bs
            assert mask.shape == (H, S // bs, S // bs) and mask[:, nbv:, :].all() and mask[:, :, nbv:].all()
            kv_tiles = (valid + 63) // 64
            _, lists = O.tiles_from_mask(mask[:, :nbv, :], bs, tile_rows == "union", kv_tiles=kv_tiles)
            tm = np.zeros((H, S, S), bool)
            tm[:, :video, :] = O.token_mask_from_tiles(lists, H, video, S)
            tm[:, video:, :valid] = True
            ref, _ = O.masked_attention(qn, kn, vn, tm, dtype=np.float64)
            _check_attn(out[0], ref, f"hunyuan sparse {step}", sparse=True)
        else:
            # map steps: dense pass without the padding mask (MoD/mod/attn_mask.py:633)
            ref, _ = O.masked_attention(qn, kn, vn, None, dtype=np.float64)
            _check_attn(out[0], ref, f"hunyuan map step {step}")


@pytest.mark.parametrize("tile_rows", ["exact", "union"])
def test_cogvideox_unaligned_text_and_video(tile_rows):
    """CogVideoX layout with 50 text + 450 video tokens at block 64: neither is
    block-aligned (the reference rejects this, MoD/mod/triton_flash_sparsity.py:157-160).
    This build's grid starts 14 virtual tokens before the text so that text fills one
    block and video starts on a block boundary; the video's last block is partial.
    """
    H, D, bs = 2, 64, 64
    text, F, tpf = 50, 3, 150
    video = F * tpf
    S = text + video
    W, T, top_k, thr = 4, 3, 6, 1e-3
    tb, vb, origin = O.cogvideox_grid(text, video, bs)
    assert (tb, vb, origin) == (1, 8, -14)
    st = md.create_adaptive_mask_state("cogvideox", H, video, text, tpf, F, warmup_steps=W,
                                       top_k=top_k, predict_T=T, threshold=thr, block_size=bs,
                                       tile_rows=tile_rows)
    for step in range(W + 2 * T):
        q, k, v = _structured_qkv(H, 1, S, D, seed=300 + step)
        qn, kn, vn = (_np(t[0]) for t in (q, k, v))
        phase = O.step_phase(step, W, T)
        out, _ = md.SparseAttentionWithMap(q, k, v, st, None, current_step=step,
                                           use_dense=step < W - 2)
        if phase != "sparse":
            ref, _ = O.masked_attention(qn, kn, vn, None, dtype=np.float64)
            _check_attn(out[0], ref, f"cogvideox {phase} {step}")
            if phase == "map_fit":
                # the map covers the partial last video block (reference count bound)
                _, lse = ops.flash_fwd(q, k, v)
                rep = O.replay_map(qn, kn, _np(lse[0]), scale=D ** -0.5, log_threshold=math.log(thr),
                                   q_off=text, k_off=text, video_blocks=vb, block_size=bs)
                got = st["prev_full_maps"].cpu().numpy().astype(np.float32)
                assert got.shape == (H, vb, vb)
                assert (np.abs(got - rep.astype(np.float32)) * bs * bs).max() <= 2.1
            continue
        mask = st["mask"].cpu().numpy()
        assert mask.shape == (H, tb + vb, tb + vb)
        assert mask[:, :tb, :].all() and mask[:, :, :tb].all()
        _, lists = O.tiles_from_mask(mask, bs, tile_rows == "union")
        tm = O.token_mask_from_tiles(lists, H, S, S, origin=origin)
        assert tm[:, :text, :].all() and tm[:, :, :text].all()  # text rows/cols are dense
        ref, _ = O.masked_attention(qn, kn, vn, tm, dtype=np.float64)
        _check_attn(out[0], ref, f"cogvideox sparse {step}", sparse=True)


def test_configs1_cogvideox_full_shape():
    """CogVideoX-sized layer: H=48, d=64, 226 text + 13 x 1350 video tokens, bf16
    Q/K/V ~ N(0,1)/sqrt(d), block 64, ~75% mask sparsity. The schedule runs at full shape;
    outputs are checked against fp64 attention under the executed mask for two heads on
    a row subset that covers the text, the first video block and the partial last one."""
    H, D, bs = 48, 64, 64
    text, F, tpf = 226, 13, 1350
    video = F * tpf
    S = text + video
    W, T, thr = 4, 3, 1e-4
    tb, vb, origin = O.cogvideox_grid(text, video, bs)
    top_k = round(0.25 * vb)
    st = md.create_adaptive_mask_state("cogvideox", H, video, text, tpf, F, warmup_steps=W,
                                       top_k=top_k, predict_T=T, threshold=thr, block_size=bs,
                                       tile_rows="exact")
    g = torch.Generator().manual_seed(2024)
    rows = np.r_[0:300, S - 200:S]
    heads = [0, 47]
    for step in range(W + 1):
        q, k, v = ((torch.randn(1, H, S, D, generator=g) * D ** -0.5).to(torch.bfloat16).to(DEV)
                   for _ in range(3))
        phase = O.step_phase(step, W, T)
        out, _ = md.SparseAttentionWithMap(q, k, v, st, None, current_step=step,
                                           use_dense=step < W - 2)
        if phase != "sparse":
            continue
        mask = st["mask"].cpu().numpy()
        assert mask.shape == (H, tb + vb, tb + vb)
        sparsity = 1.0 - mask[:, tb:, tb:].mean()
        assert 0.6 < sparsity < 0.9, sparsity
        _, lists = O.tiles_from_mask(mask[heads], bs, union_rows=False)
        tm = O.token_mask_from_tiles(lists, len(heads), S, S, origin=origin)[:, rows]
        qn = _np(q[0, heads])[:, rows]
        kn, vn = _np(k[0, heads]), _np(v[0, heads])
        ref, _ = O.masked_attention(qn, kn, vn, tm, dtype=np.float64)
        _check_attn(out[0, heads][:, rows], ref, "cogvideox full-shape sparse", sparse=True)


def test_configs1_cogvideox_full_shape_int8():
    """The int8 Q.K^T / fp8 P.V engine (precision='int8', MoD/mod/attn_mask.py:306) on
    the CogVideoX-sized layer of test_configs1_cogvideox_full_shape: head_dim 64, text
    first, the grid shifted to the text blocks. Rows covering the text, the first video
    block and the partial last one, for the first and last head, against exact fp64
    attention on the unquantised inputs under the executed mask, elementwise within the
    bound derived from the rounding model of that arithmetic (oracle.q8_exact_error_bound,
    the same contract as the d=128 layers)."""
    H, D, bs = 48, 64, 64
    text, F, tpf = 226, 13, 1350
    video = F * tpf
    S = text + video
    W, T, thr = 4, 3, 1e-4
    tb, vb, origin = O.cogvideox_grid(text, video, bs)
    top_k = round(0.25 * vb)
    st = md.create_adaptive_mask_state("cogvideox", H, video, text, tpf, F, warmup_steps=W,
                                       top_k=top_k, predict_T=T, threshold=thr, block_size=bs,
                                       tile_rows="exact", precision="int8")
    g = torch.Generator().manual_seed(2024)
    rows = np.r_[0:300, S - 200:S]
    checked = 0
    for step in range(W + 1):
        q, k, v = ((torch.randn(1, H, S, D, generator=g) * D ** -0.5).to(torch.bfloat16).to(DEV)
                   for _ in range(3))
        out, _ = md.SparseAttentionWithMap(q, k, v, st, None, current_step=step,
                                           use_dense=step < W - 2)
        if O.step_phase(step, W, T) != "sparse":
            continue
        torch.cuda.synchronize()
        tiles = st["_tiles"]
        assert tiles.origin == origin
        qz = ops.quantize_qkv(q, k, v, grid_origin=tiles.origin)  # what the engine quantised
        counts, entries = tiles.counts.cpu().numpy(), tiles.entries.cpu().numpy()
        for h in (0, H - 1):
            qh, kh, vh = (_np(t[0, h]).astype(np.float64) for t in (q, k, v))
            tm = O.token_mask_rows_from_tiles(counts[h], entries[h], rows, S, origin=origin)
            err, bound, E = check_q8_exact(_np(out[0, h])[rows], qh, kh, vh, qz, 0, h, rows, tm,
                                           tag=f"cogvideox int8 head {h}")
            print(f"cogvideox int8 head {h}: max-abs {err.max():.3e} mean-abs {err.mean():.3e}; "
                  f"worst element at {(err / bound).max():.3f} of its bound; E median "
                  f"{np.median(E):.3f}", flush=True)
            checked += 1
    assert checked == 2


def test_use_dense_and_error_paths():
    H, S, D = 1, 256, 64
    q, k, v = (torch.randn(1, H, S, D).to(torch.bfloat16).to(DEV) for _ in range(3))
    st = md.create_adaptive_mask_state("wan", H, S, 0, 128, 2, warmup_steps=6, block_size=64)
    out, info = md.SparseAttentionWithMap(q, k, v, st, None, current_step=0, use_dense=True)
    ref, _ = O.masked_attention(_np(q[0]), _np(k[0]), _np(v[0]), None, dtype=np.float64)
    _check_attn(out[0], ref, "use_dense")
    with pytest.raises(RuntimeError, match="use_dense"):
        md.SparseAttentionWithMap(q, k, v, st, None, current_step=0)
    with pytest.raises(RuntimeError, match="no mask"):
        md.SparseAttentionWithMap(q, k, v, st, None, current_step=7)
    st2 = md.create_adaptive_mask_state("wan", H, S, 0, 128, 2, sparse_type="radial")
    with pytest.raises(NotImplementedError):
        md.SparseAttentionWithMap(q, k, v, st2, None, current_step=20)


@pytest.mark.parametrize("precision", ["bf16", "int8"])
def test_cogvideox_128_blocks_grid_starting_beyond_64_tokens(precision):
    """Text-first layout with 128-token blocks and 130 text tokens: the padded grid starts
    126 tokens before token 0, beyond the (-64, 0] the kernels' 64-tile grids take. The
    engine runs the equivalent 64-tile grid (origin -62, first tile row and column all
    padding). Sparse steps must match attention under the 128-block mask on the -126 grid.
    Regression: the sparse steps raised on the grid origin."""
    H, D, bs, text, F, tpf = 2, 64, 128, 130, 3, 300
    video = F * tpf
    S = text + video
    W, T = 4, 3
    tb, vb, origin = O.cogvideox_grid(text, video, bs)
    assert origin == -126
    st = md.create_adaptive_mask_state("cogvideox", H, video, text, tpf, F, warmup_steps=W,
                                       top_k=8, predict_T=T, threshold=1e-3, block_size=bs,
                                       tile_rows="exact", precision=precision)
    checked = 0
    for step in range(W - 2, W + 2):
        g = torch.Generator().manual_seed(90 + step)
        q, k, v = (torch.randn(1, H, S, D, generator=g).to(torch.bfloat16).to(DEV)
                   for _ in range(3))
        out, _ = md.SparseAttentionWithMap(q, k, v, st, None, current_step=step)
        if O.step_phase(step, W, T) != "sparse":
            continue
        mask = st["mask"].cpu().numpy()
        assert mask.shape == (H, tb + vb, tb + vb)
        _, lists = O.tiles_from_mask(mask, bs, False)
        tm = O.token_mask_from_tiles(lists, H, S, S, origin=origin)
        if precision == "bf16":
            ref, _ = O.masked_attention(_np(q[0]), _np(k[0]), _np(v[0]), tm, dtype=np.float64)
            _check_attn(out[0], ref, f"cogvideox bs=128 origin={origin} step {step}", sparse=True)
        else:
            qz = ops.quantize_qkv(q, k, v, grid_origin=origin + 64)
            zn = dict(q8=qz.q8[0].cpu().numpy(), q_scale=qz.q_scale[0].cpu().numpy(),
                      k8=qz.k8[0].cpu().numpy(), k_scale=qz.k_scale[0].cpu().numpy(),
                      v8t=qz.v8t[0].cpu().numpy(), v_scale=qz.v_scale[0].cpu().numpy(),
                      k_mean=qz.k_mean[0].cpu().numpy(), q_kmean=qz.q_kmean[0].cpu().numpy())
            check_q8_model(out[0], zn, tm, origin=origin + 64,
                           tag=f"cogvideox bs=128 origin={origin} int8 step {step}")
        checked += 1
    assert checked == 2
