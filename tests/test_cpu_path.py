"""The torch-CPU restatement timed as bench.py's CPU baseline computes what the oracle
computes (CPU only): a baseline that timed something else would say nothing."""
import numpy as np
import torch

import oracle as O
import oracle.cpu_path as C


def test_mts_as_written_and_vectorized_equal_the_exact_sums():
    rng = np.random.default_rng(1)
    n, bpf, H = 23, 5, 2
    S = (rng.integers(0, 4097, size=(H, n, n)) / 4096.0).astype(np.float16)
    want = O.mts_exact(S, bpf)  # exact: dyadic values, sums below 2^24 ulps
    St = torch.from_numpy(S.astype(np.float32))
    assert np.array_equal(C.compute_mts_as_written(St, bpf).numpy(), want)
    assert np.array_equal(C.compute_mts_vectorized(St, bpf).numpy(), want)
    part = C.compute_mts_as_written(St, bpf, diagonals=[3, 22])
    assert np.array_equal(part[:, [3, 22]].numpy(), want[:, [3, 22]])


def test_mtm_and_cholesky_solve_equal_the_ridge_solution():
    rng = np.random.default_rng(2)
    n, bpf = 30, 6
    G = C.compute_mtm(n, bpf, 1.0, dtype=torch.float64)
    assert np.array_equal(G.numpy(), O.mtm_closed_form(n, bpf, 1.0))
    S = rng.random((2, n, n))
    mts = C.compute_mts_vectorized(torch.from_numpy(S), bpf)
    X = torch.cholesky_solve(mts.t().contiguous(), torch.linalg.cholesky(G)).t()
    np.testing.assert_allclose(X.numpy(), O.ridge_solve(S, bpf, 1.0), rtol=0, atol=1e-10)


def test_topk_and_mask_loop_equal_the_oracle():
    rng = np.random.default_rng(3)
    n, bpf, H, k = 40, 8, 3, 25
    xc = rng.normal(size=(H, 3 * n)).astype(np.float32)
    xl = rng.normal(size=(H, 3 * n)).astype(np.float32)
    sel = C.choose_topk(torch.from_numpy(xc), torch.from_numpy(xl), n, 10, k)
    ref = O.choose_topk_lines(xc, xl, n, 10, k)
    assert np.array_equal(np.sort(sel.numpy(), axis=1), ref)  # no ties in normal data
    modes = [O.MODE_SPARSE, O.MODE_BLOCK_DIAGONAL, O.MODE_SPARSE]
    bd = torch.tensor([m == O.MODE_BLOCK_DIAGONAL for m in modes])
    got = C.mask_from_lines_loop(sel, bd, n, bpf).numpy()
    want = O.generate_mask_from_lines(ref, modes, seq_len=n * 64, block_size=64,
                                      video_tokens=n * 64, text_tokens=0, bpf=bpf,
                                      model_type="wan")
    assert np.array_equal(got, want)


def test_probability_map_chunk_and_sparse_tile_equal_the_oracle():
    rng = np.random.default_rng(4)
    S, D, bs = 512, 64, 64
    q, k, v = (rng.normal(size=(S, D)).astype(np.float32) for _ in range(3))
    qt, kt, vt = (torch.from_numpy(x) for x in (q, k, v))
    _, m = C.probability_map_chunk(qt, kt, vt, 2, 5, bs, 1e-3)
    want = O.probability_map(q[None], k[None], 1e-3, bs, 0, 0, S)[0, 2:5]
    np.testing.assert_allclose(m.float().numpy(), want, rtol=0, atol=2 ** -11)
    mask = rng.random((1, S // bs, S // bs)) < 0.4
    counts, lists = O.tiles_from_mask(mask, bs, union_rows=False)
    tm = O.token_mask_from_tiles(lists, 1, S, S)
    ref, _ = O.masked_attention(q[None], k[None], v[None], tm, dtype=np.float64)
    for t in range(counts.shape[1]):
        got = C.block_sparse_attention_tile(qt, kt, vt, t, lists[0][t]).numpy()
        np.testing.assert_allclose(got, ref[0, t * 128:t * 128 + 128], rtol=0, atol=1e-5)
