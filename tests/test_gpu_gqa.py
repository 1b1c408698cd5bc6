"""GPU parity of the gated GQA prep + MFMA attention kernels against the oracle (engine f16 storage points)."""
import numpy as np
import pytest

import hybrid_attention as ha
import synth
from harness import Runner, oracle_gqa, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-2  # north-star bar for fp16 MFMA attention


def test_config1_T2048():
    # one GQA layer at T=2048: 8 q heads, 2 KV heads, head_dim 256, f16 rows ~N(0,1), RoPE 64 dims base 1e7,
    # unit q/k norm gain, sigmoid gate
    x = synth.gqa_rows(2048)
    p = synth.gqa_params()
    r = Runner(["full_attention"])
    r.set_params(0, p)
    (out,), _ = r.forward([x])
    ref, _ = oracle_gqa(x, p, 4096)
    e = rel_err(out, ref)
    print("config1 T=2048 rel_err %.2e" % e)
    assert e < TOL


@pytest.mark.parametrize("T", [1, 31, 70, 257])
def test_small_batches_with_norm_weights(T):
    B = 2
    x = synth.gqa_rows(T, B, seed=3)
    p = synth.gqa_params(seed=3, noise=0.2)
    r = Runner(["full_attention"], batch=B, max_ctx=512)
    r.set_params(0, p)
    (out,), snap = r.forward([x], keep=True)
    ref, caches = oracle_gqa(x, p, 512)
    e = rel_err(out, ref)
    print("T=%d rel_err %.2e" % (T, e))
    assert e < TOL
    K = np.zeros((B, 2, T, 256), np.float16)
    snap.read(0, "K", K)
    for b in range(B):
        assert rel_err(K[b].astype(np.float32), caches[b].K[:, :T]) < 2e-3


def test_f32_rows():
    x = synth.gqa_rows(100, 1, seed=4).astype(np.float32)
    p = synth.gqa_params(seed=4, noise=0.1)
    r = Runner(["full_attention"], full_dtype=ha.F32, max_ctx=256)
    r.set_params(0, p)
    (out,), _ = r.forward([x])
    ref, _ = oracle_gqa(x, p, 256)
    assert rel_err(out, ref) < TOL


@pytest.mark.parametrize("P,L", [(100, 30), (64, 64), (1, 1), (33, 200)])
def test_prefix_suffix_bit_exact(P, L):
    x = synth.gqa_rows(P + L, 2, seed=5)
    p = synth.gqa_params(seed=5, noise=0.1)
    r = Runner(["full_attention"], batch=2, max_ctx=1024)
    r.set_params(0, p)
    (full,), _ = r.forward([x])
    (pre,), snap = r.forward([x[:, :P]], keep=True)
    (suf,), _ = r.forward([x[:, P:]], cache=snap)
    np.testing.assert_array_equal(pre, full[:, :P])
    np.testing.assert_array_equal(suf, full[:, P:])


@pytest.mark.parametrize("P,L", [(1000, 700), (1536, 64), (640, 1), (700, 1300), (1, 1998)])
def test_split_key_ranges_prefix_suffix_bit_exact(P, L):
    # one sequence: few (sequence, KV head) pairs, so the engine splits the key range of long query blocks over
    # workgroups (pieces of 8 tiles at absolute boundaries) and merges the partial results; a resumed suffix must
    # still equal the same rows of one forward bit for bit, whatever the blocks and pieces of the two calls
    x = synth.gqa_rows(P + L, 1, seed=6)
    p = synth.gqa_params(seed=6, noise=0.1)
    r = Runner(["full_attention"], batch=1, max_ctx=2048)
    r.set_params(0, p)
    (full,), _ = r.forward([x])
    (pre,), snap = r.forward([x[:, :P]], keep=True)
    (suf,), _ = r.forward([x[:, P:]], cache=snap)
    np.testing.assert_array_equal(pre, full[:, :P])
    np.testing.assert_array_equal(suf, full[:, P:])


def test_split_key_ranges_match_oracle_and_unsplit():
    # the same sequence through a one-sequence engine (split key ranges) and as sequence 0 of a two-sequence
    # engine (one workgroup per query block), both against the oracle
    T = 1500
    x1 = synth.gqa_rows(T, 1, seed=7)
    x5 = np.concatenate([x1, synth.gqa_rows(T, 1, seed=8)], 0)
    p = synth.gqa_params(seed=7, noise=0.1)
    r1 = Runner(["full_attention"], batch=1, max_ctx=2048)
    r5 = Runner(["full_attention"], batch=2, max_ctx=2048)
    r1.set_params(0, p)
    r5.set_params(0, p)
    (o1,), _ = r1.forward([x1])
    (o5,), _ = r5.forward([x5])
    ref, _ = oracle_gqa(x1, p, 2048)
    e1, e5, e15 = rel_err(o1, ref), rel_err(o5[:1], ref), rel_err(o1, o5[:1])
    print("split vs oracle %.2e, unsplit vs oracle %.2e, split vs unsplit %.2e" % (e1, e5, e15))
    assert e1 < TOL and e5 < TOL and e15 < TOL


@pytest.mark.parametrize("B,P,steps", [(2, 700, [1, 2, 32, 17]), (8, 1536, [1, 1, 8, 32]), (2, 3, [2, 5])])
def test_short_steps_bit_exact(B, P, steps):
    # calls of at most 32 rows run their own instantiation (the second half's waves copy the tiles); chained after a
    # longer prefix, every step must equal the same rows of one forward, which runs the other instantiation
    T = P + sum(steps)
    x = synth.gqa_rows(T, B, seed=7)
    r = Runner(["full_attention"], batch=B, max_ctx=2048)
    r.set_params(0, synth.gqa_params(seed=7, noise=0.1))
    (full,), _ = r.forward([x])
    (pre,), s = r.forward([x[:, :P]], keep=True)
    np.testing.assert_array_equal(pre, full[:, :P])
    a = P
    for L in steps:
        (o,), s = r.forward([x[:, a:a + L]], cache=s, keep=True)
        np.testing.assert_array_equal(o, full[:, a:a + L], err_msg="rows %d..%d" % (a, a + L))
        a += L
