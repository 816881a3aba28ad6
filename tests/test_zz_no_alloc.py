"""The allocation-free fit entry point (moddit_fit_lines_noalloc) through the C ABI,
against moddit_fit_lines on the same inputs (GPU only). Its workspace is the library's
fixed device array, which keeps the last call's contents: two calls in a row, the second
smaller, must both equal the workspace-argument entry point bit for bit."""
import numpy as np
import pytest
import torch

from mod_dit_amd import _lib, lstsq, ops

pytestmark = pytest.mark.gpu


def test_fit_noalloc_matches_fit_lines_on_consecutive_calls():
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    for H, n, bpf in [(24, 1800, 60), (3, 270, 21)]:  # the headline shape, then smaller
        print(f"fit_lines_noalloc H={H} n={n} bpf={bpf}", flush=True)
        rng = np.random.default_rng(n)
        S = (rng.integers(0, 4097, size=(H, n, n)) / 4096.0).astype(np.float16)
        mts = ops.compute_mts(torch.from_numpy(S).to("cuda"), bpf)
        sinv = lstsq.get_factor(mts.device, n, bpf, 1.0)
        want = ops.fit_lines(sinv, mts, n, bpf, 1.0)
        got = torch.full_like(mts, float("nan"))
        rc = lib.moddit_fit_lines_noalloc(sinv.data_ptr(), mts.data_ptr(), got.data_ptr(), H, n,
                                          bpf, 1.0, stream)
        assert rc == _lib.MODDIT_OK, lib.moddit_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want)
    # beyond the fixed array: a clear error before anything is launched
    rc = lib.moddit_fit_lines_noalloc(sinv.data_ptr(), mts.data_ptr(), got.data_ptr(), 65, 2048,
                                      64, 1.0, stream)
    assert rc == _lib.MODDIT_EINVAL and b"scratch" in lib.moddit_last_error()
