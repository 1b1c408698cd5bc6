"""GPU parity of the MatMulNBits projections (ha_mnb_forward through the C ABI) against the fp64 oracle: the model's
projection shapes (web/public/gemmbench/portable.js:18) across the three implementations (M <= 2: lanes kernel;
M <= 64: packed-weight MFMA GEMV; larger M: the tiled GEMM that dequantises weight tiles into LDS, with its K range
split over workgroups when there are few output tiles), every weight format of gemmbench/kernels.js:1-14, ragged
tile edges, the exporter's own int4 quantiser, and the FWHT input rotation."""
import os
import sys

import numpy as np
import pytest

import hybrid_attention as ha

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "oracle"))
import mnb_oracle as mo  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = 2e-3  # max |err| / max |ref|: f16 weights and outputs, fp32 accumulation


def _weights(N, K, bits=4, group=32, asym=False, seed=0):
    rng = np.random.default_rng(seed)
    words = rng.integers(0, 2 ** 32, (N, K // 32, mo.words_per_block(bits)), dtype=np.uint64).astype(np.uint32)
    sc = (0.005 + 0.01 * rng.random((N, K // group))).astype(np.float16)  # portable.js:29-30
    bi = ((rng.random((N, K // group)) - 0.5) * 0.1).astype(np.float16) if asym else None
    return words, sc, bi


def _run(words, sc, bi, N, K, Ms, bits=4, group=32, asym=False, seed=1):
    import torch
    dev = "cuda:0"
    q = torch.from_numpy(words.view(np.int32)).to(dev)
    s = torch.from_numpy(sc).to(dev)
    b = torch.from_numpy(bi).to(dev) if asym else None
    w = ha.MnbWeight(N, K, q, s, b, bits=bits, group=group, asym=asym)
    W = mo.dequant(words, sc, N, K, bits, group, asym, bi)
    rng = np.random.default_rng(seed)
    errs = {}
    for M in Ms:
        a = ((rng.random((M, K)) - 0.5) * 2).astype(np.float16)
        ad = torch.from_numpy(a).to(dev)
        y = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
        torch.cuda.synchronize()
        w.forward(M, ad, y)
        torch.cuda.synchronize()
        errs[M] = mo.rel_err(y.float().cpu().numpy(), mo.matmul(a, W))
    w.close()
    return errs


@pytest.mark.parametrize("K,N", [(2048, 12288), (6144, 2048), (2048, 8256), (2048, 5120), (2048, 2048)])
def test_projection_shapes_int4(K, N):
    words, sc, _ = _weights(N, K, seed=K + N)
    errs = _run(words, sc, None, N, K, [1, 2, 3, 5, 8, 9, 16, 17, 33, 64, 65, 68, 200, 512])
    print("K=%d N=%d" % (K, N), {m: "%.1e" % e for m, e in errs.items()})
    assert max(errs.values()) < TOL


@pytest.mark.parametrize("bits,group,asym", [(4, 64, False), (4, 32, True), (3, 32, False), (3, 64, True),
                                             (2, 32, False), (2, 64, True)])
def test_formats(bits, group, asym):
    N, K = 1024, 2048
    words, sc, bi = _weights(N, K, bits, group, asym, seed=bits * 100 + group)
    errs = _run(words, sc, bi, N, K, [1, 2, 3, 17, 64, 65, 200], bits, group, asym)
    print("bits=%d group=%d asym=%d" % (bits, group, asym), {m: "%.1e" % e for m, e in errs.items()})
    assert max(errs.values()) < TOL


def test_exporter_quantised_weights():
    # a dense matrix through the exporter's own quantiser (export_engine.py:17-26), packed bytes as u32 words
    rng = np.random.default_rng(5)
    N, K = 2048, 2048
    Wf = (rng.normal(size=(N, K)) * 0.02).astype(np.float32)
    packed, scale, deq = mo.quant_int4(Wf)
    words = packed.reshape(N, K // 32, 16).view(np.uint32)
    errs = _run(words, scale, None, N, K, [5, 300])
    print("exported int4", {m: "%.1e" % e for m, e in errs.items()})
    assert max(errs.values()) < TOL


@pytest.mark.parametrize("N,K", [(2048, 2048), (4096, 2048)])
def test_implementations_agree_at_the_boundaries(N, K):
    # the first rows computed with M = 2 (lanes kernel), 3 and 64 (MFMA GEMV), 65 and 200 (tiled GEMM, K split
    # over workgroups)
    import torch
    words, sc, _ = _weights(N, K, seed=9)
    dev = "cuda:0"
    w = ha.MnbWeight(N, K, torch.from_numpy(words.view(np.int32)).to(dev), torch.from_numpy(sc).to(dev), None)
    a = torch.from_numpy(((np.random.default_rng(2).random((200, K)) - 0.5) * 2).astype(np.float16)).to(dev)
    ys = {}
    for M in (2, 3, 64, 65, 200):
        ys[M] = torch.empty(M, N, dtype=torch.float16, device=dev)
        w.forward(M, a, ys[M])
    torch.cuda.synchronize()
    ref = ys[200][:2].float().cpu().numpy()
    for M, y in ys.items():
        e = mo.rel_err(y[:2].float().cpu().numpy(), ref)
        print("M=%d vs M=200 on the first two rows: %.1e" % (M, e))
        assert e < TOL
    w.close()


@pytest.mark.parametrize("N,K,Ms,bits,group,asym", [
    (1040, 2080, [49, 130, 257], 4, 32, False),   # N % 128 = 16, K % 64 = 32, M % 128 != 0
    (2064, 2048, [200], 3, 64, True),
    (16, 64, [1, 3, 50, 129], 2, 32, True),       # one 16-column tile, two blocks
])
def test_gemm_edges(N, K, Ms, bits, group, asym):
    words, sc, bi = _weights(N, K, bits, group, asym, seed=N + K)
    errs = _run(words, sc, bi, N, K, Ms, bits, group, asym)
    print("N=%d K=%d bits=%d group=%d asym=%d" % (N, K, bits, group, asym), {m: "%.1e" % e for m, e in errs.items()})
    assert max(errs.values()) < TOL


def test_gemm_large_m_sampled_rows():
    # one call with every row of a B = 8, T = 2048 prefill (M = 16384) on the largest input projection; a sample of
    # rows against the oracle (the full fp64 product is too slow on the CPU); rows 0..2047 bit-identical to an
    # M = 2048 call (same tiles, no K split), rows 0..63 within the bar of the M = 64 GEMV
    import torch
    N, K, M = 8256, 2048, 16384
    words, sc, _ = _weights(N, K, seed=77)
    dev = "cuda:0"
    w = ha.MnbWeight(N, K, torch.from_numpy(words.view(np.int32)).to(dev), torch.from_numpy(sc).to(dev), None)
    a = torch.from_numpy(((np.random.default_rng(3).random((M, K)) - 0.5) * 2).astype(np.float16)).to(dev)
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    y64 = torch.empty(64, N, dtype=torch.float16, device=dev)
    y2k = torch.empty(2048, N, dtype=torch.float16, device=dev)
    print("gemm M=%d N=%d K=%d" % (M, N, K), flush=True)
    w.forward(M, a, y)
    w.forward(64, a, y64)
    w.forward(2048, a, y2k)
    torch.cuda.synchronize()
    assert torch.equal(y[:2048], y2k), "rows differ between M = 16384 and M = 2048"
    assert mo.rel_err(y[:64].float().cpu().numpy(), y64.float().cpu().numpy()) < TOL
    assert not torch.isnan(y).any()
    rows = [0, 1, 127, 128, 5000, 8191, 12345, M - 1]
    W = mo.dequant(words, sc, N, K)
    e = mo.rel_err(y[rows].float().cpu().numpy(), mo.matmul(a[rows].cpu().numpy(), W))
    print("sampled rows rel_err %.1e" % e)
    assert e < TOL
    w.close()


@pytest.mark.parametrize("n", [64, 2048])
def test_fwht(n):
    import torch
    x = (np.random.default_rng(n).normal(size=(5, 2 * n))).astype(np.float16)
    xd = torch.from_numpy(x).to("cuda:0")
    ha.fwht(xd, x.size, n)
    torch.cuda.synchronize()
    ref = mo.fwht(x.astype(np.float64), n)
    e = mo.rel_err(xd.float().cpu().numpy(), ref)
    print("fwht n=%d rel_err %.1e" % (n, e))
    assert e < 2e-3


def test_errors():
    import torch
    s = torch.zeros(16, 64, dtype=torch.float16, device="cuda:0")
    q = torch.zeros(16, 64, 4, dtype=torch.int32, device="cuda:0")
    w = ha.MnbWeight(15, 2048, q, s, None)  # a table of any row count (an embedding) ...
    with pytest.raises(ha.HAError):
        w.forward(1, s, s)  # ... but a matmul needs N % 16 == 0
    w.close()
    with pytest.raises(ha.HAError):
        ha.MnbWeight(16, 2048, q, s, None, bits=5)
    with pytest.raises(ha.HAError):
        ha.MnbWeight(16, 2048, q, s, None, asym=True)  # no bias
    with pytest.raises(ha.HAError):
        ha.fwht(s, s.numel(), 48)  # not a power of two
