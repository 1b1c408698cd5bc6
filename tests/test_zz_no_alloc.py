"""GPU check of the allocation-free MatMulNBits entry point (ha_mnb_forward_noalloc through the C ABI): its output
equals ha_mnb_forward's on the same inputs, on two calls in a row (the second with fewer rows, so it reuses the
per-GPU scratch array the first call left filled), for shapes whose K range is split (partials in the scratch)
and one that is not."""
import os
import sys

import numpy as np
import pytest

import hybrid_attention as ha

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "oracle"))
import mnb_oracle as mo  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = 2e-3  # max |err| / max |ref| against the fp64 oracle: f16 weights and outputs, fp32 accumulation


@pytest.mark.parametrize("N,K,Ms", [(2048, 6144, (1408, 200)), (12288, 2048, (256, 65)), (2048, 2048, (2048, 96))])
def test_noalloc_matches_allocating_entry_point(N, K, Ms):
    import torch
    dev = "cuda:0"
    rng = np.random.default_rng(N + K)
    words = rng.integers(0, 2 ** 32, (N, K // 32, 4), dtype=np.uint64).astype(np.uint32)
    sc = (0.005 + 0.01 * rng.random((N, K // 32))).astype(np.float16)
    q = torch.from_numpy(words.view(np.int32)).to(dev)
    s = torch.from_numpy(sc).to(dev)
    w = ha.MnbWeight(N, K, q, s)
    W = None
    for M in Ms:
        print("no-alloc GEMM N=%d K=%d M=%d" % (N, K, M), flush=True)
        a = ((rng.random((M, K)) - 0.5) * 2).astype(np.float16)
        ad = torch.from_numpy(a).to(dev)
        y0 = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
        y1 = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
        torch.cuda.synchronize()
        w.forward_noalloc(M, ad, y1)
        torch.cuda.synchronize()
        w.forward(M, ad, y0)
        torch.cuda.synchronize()
        g0, g1 = y0.cpu().numpy(), y1.cpu().numpy()
        assert np.isfinite(g1.astype(np.float32)).all()
        assert np.array_equal(g0.view(np.uint16), g1.view(np.uint16)), "no-alloc result differs from ha_mnb_forward"
        if W is None:
            W = mo.dequant(words, sc, N, K, 4, 32, False, None)
        rows = slice(0, min(M, 64))
        err = mo.rel_err(g1[rows].astype(np.float32), mo.matmul(a[rows], W))
        print("  rel_err vs oracle (first rows) %.2e" % err)
        assert err < TOL
    w.close()
