"""Pins of the torso oracle (oracle/torso_oracle.py) on the CPU: EMBED, ADD_NORM, SILU_MUL and ADD_BIAS of
web/public/engine/wgsl.js:42-121, against torch's own rms_norm and silu, closed forms, and a scalar restatement of
EMBED's element indexing."""
import os
import sys

import numpy as np
import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "oracle"))
import mnb_oracle as mo  # noqa: E402
import torso_oracle as to  # noqa: E402


def test_add_norm_matches_torch_rms_norm_and_writes_back_the_sum():
    rng = np.random.default_rng(0)
    x, y = rng.normal(size=(5, 64)), rng.normal(size=(5, 64))
    w = rng.normal(size=64)
    h, x2 = to.add_norm(x, y, w, eps=1e-6)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x + y), (64,), torch.from_numpy(w), eps=1e-6).numpy()
    np.testing.assert_allclose(h, ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(x2, x + y)
    # no add, gathered rows: only the listed rows, in list order
    h2, x3 = to.add_norm(x, None, w, rows=[4, 1])
    ref2 = torch.nn.functional.rms_norm(torch.from_numpy(x[[4, 1]]), (64,), torch.from_numpy(w), eps=1e-6).numpy()
    np.testing.assert_allclose(h2, ref2, rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(x3, x)


def test_add_norm_closed_forms():
    w = np.linspace(0.5, 1.5, 16)
    # a constant row c normalises to sign(c) w (up to eps); scaling a row leaves the result unchanged
    h, _ = to.add_norm(np.full((1, 16), -3.0), None, w, eps=0.0)
    np.testing.assert_allclose(h[0], -w, rtol=1e-15)
    x = np.random.default_rng(1).normal(size=(1, 16))
    a, _ = to.add_norm(x, None, w, eps=0.0)
    b, _ = to.add_norm(7.5 * x, None, w, eps=0.0)
    np.testing.assert_allclose(a, b, rtol=1e-13)


def test_silu_mul_matches_torch_and_limits():
    rng = np.random.default_rng(2)
    big = rng.normal(size=(3, 32)) * 4
    mid = to.silu_mul(big, 16)
    ref = (torch.nn.functional.silu(torch.from_numpy(big[:, :16])) * torch.from_numpy(big[:, 16:])).numpy()
    np.testing.assert_allclose(mid, ref, rtol=1e-12, atol=1e-12)
    edge = to.silu_mul(np.array([[0.0, 40.0, 1.0, 1.0]]), 2)
    assert edge[0, 0] == 0.0 and abs(edge[0, 1] - 40.0) < 1e-12


def _embed_scalar(words, scales, ids, D, bits):
    """EMBED's own indexing (wgsl.js:51-58), restated per element: thread w of row t writes elements 8 w .. 8 w + 7
    of block id * D/32 + w / 4, element e = (w % 4) * 8 + j of that block, (q - 2^(bits-1)) * scale in f32."""
    nb = mo.words_per_block(bits)
    Q = np.asarray(words, np.uint64).reshape(-1)
    S = np.asarray(scales, np.float16).reshape(-1)
    out = np.zeros((len(ids), D), np.float32)
    for t, i in enumerate(ids):
        for w in range(D // 8):
            blk = i * (D // 32) + w // 4
            sc = np.float32(S[blk])
            for j in range(8):
                e = (w % 4) * 8 + j
                if bits == 4:
                    q = (int(Q[blk * 4 + e // 8]) >> (4 * (e % 8))) & 15
                else:
                    q = (int(Q[blk * bits + e // 16]) >> (2 * (e % 16))) & 3
                    if bits == 3:
                        q |= ((int(Q[blk * 3 + 2]) >> e) & 1) << 2
                out[t, w * 8 + j] = (np.float32(q) - np.float32(2 ** (bits - 1))) * sc
    return out


def test_embed_matches_the_reference_indexing_each_width():
    rng = np.random.default_rng(3)
    D, rows = 64, 6
    for bits in (4, 3, 2):
        words = rng.integers(0, 2 ** 32, (rows, D // 32, mo.words_per_block(bits)), dtype=np.uint64).astype(np.uint32)
        sc = (0.005 + 0.01 * rng.random((rows, D // 32))).astype(np.float16)
        ids = [5, 0, 5, 2]
        np.testing.assert_array_equal(to.embed(words, sc, ids, D, bits), _embed_scalar(words, sc, ids, D, bits))


def test_embed_known_codes_and_asymmetric_form():
    # one block with codes e % 16 (4 bits) and scale 0.5: row = (e % 16 - 8) / 2; bias form q * s + b
    by = np.array([((2 * i + 1) % 16) << 4 | (2 * i) % 16 for i in range(16)], np.uint8)
    words = by.view(np.uint32).reshape(1, 1, 4)
    x = to.embed(words, np.array([[0.5]], np.float16), [0], 32)
    np.testing.assert_array_equal(x[0], (np.arange(32) % 16 - 8) * 0.5)
    xa = to.embed(words, np.array([[0.5]], np.float16), [0], 32, asym=True, bias=np.array([[1.0]], np.float16))
    np.testing.assert_array_equal(xa[0], (np.arange(32) % 16) * 0.5 + 1.0)
