"""Pins of the MatMulNBits oracle (oracle/mnb_oracle.py) on the CPU: the weight formats of
web/public/gemmbench/kernels.js:1-14, the exporter's int4 quantiser (convert/export_engine.py:17-26) and the FWHT
input rotation (web/public/engine/wgsl.js:94-110)."""
import os
import sys

import numpy as np
import pytest
import scipy.linalg

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "oracle"))
import mnb_oracle as mo  # noqa: E402


def _bench_js_reference(A16, Bbytes, Sc, K, N, cols):
    """The reference's own CPU check (gemmbench/bench.js:48-50), restated loop for loop: byte (e >> 1) of the
    block, high nibble for odd e, (q - 8) * scale."""
    M = A16.shape[0]
    out = np.zeros((M, len(cols)))
    for j, n in enumerate(cols):
        for m in range(M):
            s = 0.0
            for b in range(K // 32):
                sc = float(Sc[n * (K // 32) + b])
                for e in range(32):
                    byte = int(Bbytes[(n * (K // 32) + b) * 16 + (e >> 1)])
                    q = (byte >> 4) if (e & 1) else (byte & 15)
                    s += float(A16[m, b * 32 + e]) * ((q - 8) * sc)
            out[m, j] = s
    return out


def test_int4_layout_matches_the_reference_check():
    rng = np.random.default_rng(0)
    N, K, M = 8, 64, 3
    Bbytes = rng.integers(0, 256, N * K // 2, dtype=np.uint8)
    Sc = (0.005 + 0.01 * rng.random(N * K // 32)).astype(np.float16)
    A16 = ((rng.random((M, K)) - 0.5) * 2).astype(np.float16)
    W = mo.dequant(Bbytes.view(np.uint32), Sc, N, K, bits=4, group=32)
    y = mo.matmul(A16, W)
    cols = [0, 1, N // 2, N - 1]
    ref = _bench_js_reference(A16, Bbytes, Sc, K, N, cols)
    np.testing.assert_allclose(y[:, cols], ref, rtol=1e-12, atol=1e-12)


def test_known_codes_each_width():
    # 4 bits: byte i = (2i+1) << 4 | 2i (mod 16) -> element e has code e % 16
    by = np.array([((2 * i + 1) % 16) << 4 | (2 * i) % 16 for i in range(16)], np.uint8)
    np.testing.assert_array_equal(mo.decode(by.view(np.uint32), 4), np.arange(32) % 16)
    # 2 bits: element e at bits 2(e%16) of word e/16; code e % 4
    w2 = np.zeros(2, np.uint32)
    for e in range(32):
        w2[e // 16] |= np.uint32((e % 4) << (2 * (e % 16)))
    np.testing.assert_array_equal(mo.decode(w2, 2), np.arange(32) % 4)
    # 3 bits: low two bits as the 2-bit layout, bit e of word 2 the high bit; code e % 8
    w3 = np.zeros(3, np.uint32)
    for e in range(32):
        c = e % 8
        w3[e // 16] |= np.uint32((c & 3) << (2 * (e % 16)))
        w3[2] |= np.uint32((c >> 2) << e)
    np.testing.assert_array_equal(mo.decode(w3, 3), np.arange(32) % 8)


@pytest.mark.parametrize("bits,group,asym", [(4, 32, False), (4, 64, True), (3, 32, False), (2, 64, True)])
def test_dequant_closed_form_and_one_hot_rows(bits, group, asym):
    rng = np.random.default_rng(bits * 10 + group)
    N, K = 16, 128
    nw = mo.words_per_block(bits)
    words = rng.integers(0, 2 ** 32, (N, K // 32, nw), dtype=np.uint64).astype(np.uint32)
    sc = (0.005 + 0.01 * rng.random((N, K // group))).astype(np.float16)
    bi = (rng.random((N, K // group)) - 0.5).astype(np.float16) if asym else None
    W = mo.dequant(words, sc, N, K, bits, group, asym, bi)
    q = mo.decode(words, bits).reshape(N, K)
    n, k = 5, 77
    g = k // group
    want = q[n, k] * float(sc[n, g]) + float(bi[n, g]) if asym else (q[n, k] - 2 ** (bits - 1)) * float(sc[n, g])
    assert W[n, k] == want
    # a one-hot row of a picks a column of W exactly
    a = np.zeros((2, K), np.float16)
    a[0, k] = 1.0
    a[1, 3] = 1.0
    y = mo.matmul(a, W)
    np.testing.assert_array_equal(y[0], W[:, k])
    np.testing.assert_array_equal(y[1], W[:, 3])


def test_quantiser_round_trip():
    rng = np.random.default_rng(3)
    Wf = rng.normal(size=(8, 256)).astype(np.float32)
    packed, scale, deq = mo.quant_int4(Wf)
    W = mo.dequant(packed.reshape(8, -1).view(np.uint32), scale, 8, 256, bits=4, group=32)
    np.testing.assert_array_equal(W, deq.astype(np.float64))
    # each block's largest-magnitude element gets code 0, i.e. -8 * scale, within the f16 rounding of the scale
    b = Wf.reshape(8, 8, 32)
    idx = np.abs(b).argmax(-1)
    q = mo.decode(packed.reshape(8, 8, 16).view(np.uint32).reshape(8, 8, 4), 4)
    np.testing.assert_array_equal(np.take_along_axis(q, idx[..., None], -1), 0)
    top = np.take_along_axis(b, idx[..., None], -1)[..., 0]
    np.testing.assert_allclose(-8.0 * scale.astype(np.float64), top, rtol=2 ** -10)
    # and every element is within half a quantisation step (or clamped at code 15 from the far side)
    err = np.abs(W.reshape(8, 8, 32) - b) / np.abs(scale.astype(np.float64))[..., None]
    assert err.max() <= 0.5 + 1e-6 or np.all((err <= 0.5 + 1e-6) | (q == 15))


@pytest.mark.parametrize("n", [2, 8, 64])
def test_fwht(n):
    rng = np.random.default_rng(n)
    x = rng.normal(size=(3, 2 * n))
    y = mo.fwht(x, n)
    H = scipy.linalg.hadamard(n) / np.sqrt(n)
    np.testing.assert_allclose(y.reshape(-1, n), x.reshape(-1, n) @ H.T, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(mo.fwht(y, n), x, rtol=1e-12, atol=1e-12)
    if n == 2:
        np.testing.assert_allclose(y[0, :2], [(x[0, 0] + x[0, 1]) / np.sqrt(2), (x[0, 0] - x[0, 1]) / np.sqrt(2)])
