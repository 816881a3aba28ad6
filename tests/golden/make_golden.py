"""Generate the golden fixtures under tests/golden/ from the CPU oracle.

The MOD-DiT reference ships no golden vectors (its tests generate inputs on the fly), so
these fixtures freeze small, seeded cases of every hot-path stage as data: inputs and
the oracle's outputs. tests/test_golden.py re-derives them on the CPU (the oracle must
keep reproducing them) and tests/test_gpu_golden.py runs the HIP kernels on the same
inputs.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle as O  # noqa: E402


def lines_mask_tiles(rng):
    """Features -> selected lines -> mask -> tile lists (wan layout, 64-token blocks)."""
    H, n, bpf, T, top_k = 4, 32, 8, 10, 20
    x_cur = rng.normal(size=(H, 3 * n)).astype(np.float32)
    x_last = rng.normal(size=(H, 3 * n)).astype(np.float32)
    x_cur[1, :5] = 0.25  # exact ties, resolved by index
    x_last[1, :5] = 0.25
    modes = np.array([O.MODE_SPARSE, O.MODE_BLOCK_DIAGONAL, O.MODE_SPARSE, O.MODE_FULL], np.uint8)
    sel = O.choose_topk_lines(x_cur, x_last, n, T, top_k)
    mask = O.generate_mask_from_lines(sel, list(modes), seq_len=n * 64, block_size=64,
                                      video_tokens=n * 64, text_tokens=0, bpf=bpf, model_type="wan")
    out = dict(x_cur=x_cur, x_last=x_last, modes=modes, n=n, bpf=bpf, T=T, top_k=top_k,
               sel=sel.astype(np.int32), mask=mask)
    for union in (False, True):
        counts, lists = O.tiles_from_mask(mask, 64, union)
        cap = n
        ent = np.full((H, counts.shape[1], cap), -1, np.int32)
        for h in range(H):
            for t in range(counts.shape[1]):
                ent[h, t, :counts[h, t]] = lists[h][t]
        tag = "union" if union else "exact"
        out[f"counts_{tag}"] = counts
        out[f"entries_{tag}"] = ent
    return out


def mts_fit(rng):
    """Dyadic fp16 map -> exact M^T S -> fp64 ridge features (lambda = 1)."""
    H, n, bpf = 2, 48, 12
    S = (rng.integers(0, 4097, size=(H, n, n)) / 4096.0).astype(np.float16)
    mts = O.mts_exact(S, bpf)
    X = O.ridge_solve(S.astype(np.float64), bpf, 1.0)
    return dict(S=S, bpf=bpf, mts=mts, X=X)


def replay_dyadic(rng):
    """Dyadic Q/K (d=64, scale 1/8 exact) + LSE -> bit-exact replayed fp16 map."""
    H, S, D, bs = 2, 192, 64, 64
    q = rng.integers(-4, 5, size=(H, S, D)).astype(np.float32) / 8
    k = rng.integers(-4, 5, size=(H, S, D)).astype(np.float32) / 8
    s = np.einsum("hqd,hkd->hqk", q.astype(np.float64), k.astype(np.float64)) / 8
    lse = np.log(np.exp(s).sum(-1)).astype(np.float32)
    thr = 1e-3
    m = O.replay_map(q, k, lse, scale=1 / 8, log_threshold=math.log(thr), q_off=0, k_off=0,
                     video_blocks=S // bs, block_size=bs)
    return dict(q8=(q * 8).astype(np.int8), k8=(k * 8).astype(np.int8), lse=lse,
                log_threshold=np.float32(math.log(thr)), map=m, block=bs)


def attention_small(rng):
    """bf16-representable Q/K/V + a 64x64 block mask -> fp64 masked attention."""
    H, S, D, bs = 2, 256, 64, 64
    q, k, v = (O.bf16_round(rng.normal(size=(H, S, D)).astype(np.float32)) for _ in range(3))
    nb = S // bs
    mask = rng.random((H, nb, nb)) < 0.5
    mask[:, np.arange(nb), np.arange(nb)] = True
    mask[1, 2, :] = False  # one query block with no key block
    out, lse = O.masked_attention(q, k, v, O.token_mask_from_blocks(mask, bs), dtype=np.float64)
    bits = lambda a: (a.view(np.uint32) >> 16).astype(np.uint16)  # exact: values are bf16
    return dict(q_bf16=bits(q), k_bf16=bits(k), v_bf16=bits(v), mask=mask,
                out=out.astype(np.float32), lse=lse.astype(np.float32), block=bs)


GENERATORS = {
    "lines_mask_tiles": (lines_mask_tiles, 101),
    "mts_fit": (mts_fit, 102),
    "replay_dyadic": (replay_dyadic, 103),
    "attention_small": (attention_small, 104),
}


def build(name: str) -> dict:
    fn, seed = GENERATORS[name]
    return fn(np.random.default_rng(seed))


def main() -> int:
    for name in GENERATORS:
        data = build(name)
        np.savez_compressed(HERE / f"{name}.npz", **data)
        print(f"wrote {name}.npz ({sum(np.asarray(v).nbytes for v in data.values())} bytes raw)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
