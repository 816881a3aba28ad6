"""HIP kernels on the golden fixture inputs (GPU only)."""
import numpy as np
import pytest
import torch

import mod_dit_amd as md
from mod_dit_amd import ops

from test_golden import load

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_golden_lines_mask_tiles():
    g = load("lines_mask_tiles")
    n = int(g["n"])
    sel = ops.select_lines(torch.from_numpy(g["x_cur"]).to(DEV), torch.from_numpy(g["x_last"]).to(DEV),
                           n, int(g["T"]), int(g["top_k"]))
    assert np.array_equal(sel.cpu().numpy(), g["sel"])
    modes = torch.from_numpy(g["modes"]).to(DEV)
    for tag, union in (("exact", False), ("union", True)):
        mask, tiles = ops.mask_from_lines(sel, modes, n=n, blocks_per_frame=int(g["bpf"]), layout=0,
                                          nb=n, text_blocks=0, block_size=64, union_rows=union)
        assert np.array_equal(mask.cpu().numpy(), g["mask"])
        c = tiles.counts.cpu().numpy()
        assert np.array_equal(c, g[f"counts_{tag}"])
        e = tiles.entries.cpu().numpy()
        want = g[f"entries_{tag}"]
        for h in range(c.shape[0]):
            for t in range(c.shape[1]):
                assert np.array_equal(e[h, t, :c[h, t]], want[h, t, :c[h, t]])


def test_golden_mts_and_fit():
    g = load("mts_fit")
    S = torch.from_numpy(g["S"]).to(DEV)
    bpf = int(g["bpf"])
    assert np.array_equal(md.compute_mts(S, bpf).cpu().numpy(), g["mts"])
    st = md.create_adaptive_mask_state("wan", 2, 48 * 64, 0, bpf * 64, 4, block_size=64)
    X = md.solve_lstsq(st, S, st["warmup_steps"], bpf, regularization=1.0)["_x"].cpu().numpy()
    assert np.abs(X - g["X"]).max() <= 1e-4 * np.abs(g["X"]).max()


def test_golden_replay_map_bit_exact():
    g = load("replay_dyadic")
    q = torch.from_numpy(g["q8"].astype(np.float32) / 8)[None].to(torch.bfloat16).to(DEV)
    k = torch.from_numpy(g["k8"].astype(np.float32) / 8)[None].to(torch.bfloat16).to(DEV)
    lse = torch.from_numpy(g["lse"])[None].to(DEV)
    bs = int(g["block"])
    m = md.cuda_sparsity_map(q, k, lse, softmax_scale=64 ** -0.5, log_threshold=float(g["log_threshold"]),
                             q_video_offset=0, k_video_offset=0, video_blocks=q.shape[2] // bs,
                             block_size=bs)
    assert np.array_equal(m[0].cpu().numpy(), g["map"])


@pytest.mark.parametrize("union", [False])
def test_golden_block_sparse_attention(union):
    g = load("attention_small")
    to_t = lambda b: torch.from_numpy((b.astype(np.uint32) << 16).view(np.float32))[None].to(torch.bfloat16).to(DEV)
    q, k, v = to_t(g["q_bf16"]), to_t(g["k_bf16"]), to_t(g["v_bf16"])
    tiles = ops.mask_to_tiles(torch.from_numpy(g["mask"]).to(DEV), int(g["block"]), union_rows=union)
    out, lse = ops.block_sparse_fwd(q, k, v, tiles, return_lse=True)
    err = np.abs(out[0].float().cpu().numpy() - g["out"])
    assert err.max() <= 2e-2 and err.mean() <= 2e-3
    got_lse = lse[0].cpu().numpy()
    fin = np.isfinite(g["lse"])
    assert np.array_equal(np.isneginf(got_lse), ~fin)
    assert np.abs(got_lse[fin] - g["lse"][fin]).max() <= 2e-3
