"""GPU parity of the torso ops around the mixers and projections (ha_embed, ha_add_norm, ha_silu_mul, ha_add_bias
through the C ABI) against the fp64 oracle: EMBED, ADD_NORM, SILU_MUL and ADD_BIAS of web/public/engine/wgsl.js:42-121
at the model's widths (D = 2048, I = 6144), the final norm's gathered rows in f32 (engine.js:283-284, 342), every
embedding format, and out-of-range indices (a NaN row, no out-of-bounds access)."""
import os
import sys

import numpy as np
import pytest

import hybrid_attention as ha

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "oracle"))
import mnb_oracle as mo  # noqa: E402
import torso_oracle as to  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _rel(a, b):
    return mo.rel_err(np.asarray(a, np.float64), np.asarray(b, np.float64))


@pytest.mark.parametrize("bits,group,asym", [(4, 32, False), (4, 64, True), (3, 32, False), (2, 64, True)])
def test_embed(bits, group, asym):
    import torch
    rng = np.random.default_rng(bits + group)
    rows, D = 300, 2048
    words = rng.integers(0, 2 ** 32, (rows, D // 32, mo.words_per_block(bits)), dtype=np.uint64).astype(np.uint32)
    sc = (0.005 + 0.01 * rng.random((rows, D // group))).astype(np.float16)
    bi = ((rng.random((rows, D // group)) - 0.5) * 0.1).astype(np.float16) if asym else None
    q, s = torch.from_numpy(words.view(np.int32)).to(DEV), torch.from_numpy(sc).to(DEV)
    b = torch.from_numpy(bi).to(DEV) if asym else None
    table = ha.MnbWeight(rows, D, q, s, b, bits=bits, group=group, asym=asym)
    ids = np.array([7, 0, 299, 7, 150, 1000], np.uint32)  # 1000 is outside the table
    x = torch.empty(len(ids), D, dtype=torch.float32, device=DEV)
    ha.embed(table, len(ids), torch.from_numpy(ids.view(np.int32)).to(DEV), x)
    torch.cuda.synchronize()
    got = x.cpu().numpy()
    ref = to.embed(words, sc, ids[:5], D, bits, group, asym, bi)
    np.testing.assert_array_equal(got[:5], ref.astype(np.float32))  # the same f32 arithmetic: bit-exact
    assert np.isnan(got[5]).all()
    table.close()


@pytest.mark.parametrize("add", [False, True])
@pytest.mark.parametrize("D", [2048, 1024, 4096])
def test_add_norm(add, D):
    import torch
    rng = np.random.default_rng(D + add)
    nx = 37
    x = (rng.normal(size=(nx, D)) * 3).astype(np.float32)
    y = rng.normal(size=(nx, D)).astype(np.float16)
    w = (1 + 0.1 * rng.normal(size=D)).astype(np.float32)
    xd, yd, wd = (torch.from_numpy(v).to(DEV) for v in (x, y, w))
    h = torch.empty(nx, D, dtype=torch.float16, device=DEV)
    ha.add_norm(nx, D, nx, xd, yd if add else None, wd, h)
    torch.cuda.synchronize()
    ref, x2 = to.add_norm(x, y if add else None, w)
    e = _rel(h.float().cpu().numpy(), ref)
    print("add_norm D=%d add=%d rel_err %.1e" % (D, add, e))
    assert e < 1e-3  # f16 output
    np.testing.assert_allclose(xd.cpu().numpy(), x2, rtol=1e-6, atol=1e-6)  # the residual sum, written back


def test_final_norm_gathered_rows_f32():
    # the final norm: residual add and norm only for the requested rows, f32 out (engine.js:283-284, 342);
    # a row index past the end gives a NaN row
    import torch
    rng = np.random.default_rng(9)
    nx, D = 50, 2048
    x = rng.normal(size=(nx, D)).astype(np.float32)
    y = rng.normal(size=(nx, D)).astype(np.float16)
    w = (1 + 0.1 * rng.normal(size=D)).astype(np.float32)
    rows = np.array([49, 0, 17, 50], np.uint32)
    xd, yd, wd = (torch.from_numpy(v).to(DEV) for v in (x, y, w))
    h = torch.empty(len(rows), D, dtype=torch.float32, device=DEV)
    ha.add_norm(len(rows), D, nx, xd, yd, wd, h, out_f32=True, rows=torch.from_numpy(rows.view(np.int32)).to(DEV))
    torch.cuda.synchronize()
    ref, x2 = to.add_norm(x, y, w, rows=rows[:3])
    got = h.cpu().numpy()
    e = _rel(got[:3], ref)
    print("final norm rel_err %.1e" % e)
    assert e < 1e-5
    assert np.isnan(got[3]).all()
    # rows not listed keep their residual stream untouched
    xa = xd.cpu().numpy()
    untouched = np.setdiff1d(np.arange(nx), rows[:3])
    np.testing.assert_array_equal(xa[untouched], x[untouched])
    np.testing.assert_allclose(xa[rows[:3]], x2[rows[:3]], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("L,I", [(1, 6144), (100, 6144), (3, 8)])
def test_silu_mul(L, I):
    import torch
    big = (np.random.default_rng(L).normal(size=(L, 2 * I)) * 3).astype(np.float16)
    mid = torch.empty(L, I, dtype=torch.float16, device=DEV)
    ha.silu_mul(L, I, torch.from_numpy(big).to(DEV), mid)
    torch.cuda.synchronize()
    e = _rel(mid.float().cpu().numpy(), to.silu_mul(big, I))
    print("silu_mul L=%d I=%d rel_err %.1e" % (L, I, e))
    assert e < 1e-3


def test_add_bias():
    import torch
    rng = np.random.default_rng(4)
    L, N = 70, 2048
    y = rng.normal(size=(L, N)).astype(np.float16)
    c = rng.normal(size=N).astype(np.float32)
    yd = torch.from_numpy(y).to(DEV)
    ha.add_bias(L, N, yd, torch.from_numpy(c).to(DEV))
    torch.cuda.synchronize()
    assert _rel(yd.float().cpu().numpy(), to.add_bias(y, c)) < 1e-3


def test_errors():
    import torch
    t = torch.zeros(64, dtype=torch.float32, device=DEV)
    with pytest.raises(ha.HAError):
        ha.add_norm(1, 12, 1, t, None, t, t)  # D % 8
    with pytest.raises(ha.HAError):
        ha.add_norm(4, 8, 2, t, None, t, t)  # more output rows than x without a row list
    with pytest.raises(ha.HAError):
        ha.silu_mul(1, 12, t, t)
    with pytest.raises(ha.HAError):
        ha.add_bias(1, 4, t, t)
