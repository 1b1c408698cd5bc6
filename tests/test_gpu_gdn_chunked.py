"""GPU parity of the chunked (MFMA) gated-delta prefill against the fp64 sequential oracle and against the GPU's own
fp32 sequential kernel, plus bit-exact prefix + suffix for aligned and unaligned splits. Every test runs the three
implementations of the chunked form: the single fused kernel, the split form (chunk images, a sequential state pass,
then every chunk's outputs at once) and the paired form."""
import numpy as np
import pytest

import hybrid_attention as ha
import synth
from harness import Runner, gdn_inputs, oracle_gdn, rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-3  # north-star bar for the recurrence (max |err| / max |ref|)


@pytest.fixture(params=[ha.CHUNKED_FUSED, ha.CHUNKED_SPLIT, ha.CHUNKED_PAIRED], ids=["fused", "split", "paired"])
def mode(request):
    return request.param


def _state(snap, B=1):
    s = np.zeros((B, 16, 128, 128), np.float32)
    return snap.read(0, "state", s)


@pytest.mark.parametrize("gnorm", [False, True])
def test_config0_chunked(gnorm, mode):
    x = gdn_inputs(64)
    p = synth.gdn_params()
    r = Runner(["linear_attention"], gnorm=gnorm)
    r.set_params(0, p)
    (out,), snap = r.forward([x], keep=True, recurrence=mode)
    ref, st = oracle_gdn(x, p, gnorm=gnorm)
    e, es = rel_err(out, ref), rel_err(_state(snap)[0], st[0].S)
    print("config0 chunked gnorm=%s rel_err out %.2e state %.2e" % (gnorm, e, es))
    assert e < TOL and es < TOL
    assert snap.state_pos == 64 and snap.tail_rows == 3


@pytest.mark.parametrize("T", [100, 64 + 1, 130])
def test_snapshot_state_at_P(T, mode):
    # the snapshot's "state" is the state after all P = T rows, as the reference's snapshot holds it (engine.js:352),
    # although the stored state sits at the last 64-row boundary ("state_stored", what a resume starts from)
    x = gdn_inputs(T, 2, seed=13)
    p = synth.gdn_params(seed=13)
    r = Runner(["linear_attention"], batch=2)
    r.set_params(0, p)
    _, snap = r.forward([x], keep=True, recurrence=mode)
    assert snap.state_pos == 64 * (T // 64) < T
    _, st_P = oracle_gdn(x, p)
    _, st_s = oracle_gdn(x[:, :snap.state_pos], p)
    at_P = _state(snap, 2)
    stored = np.zeros_like(at_P)
    snap.read(0, "state_stored", stored)
    e_P = rel_err(at_P, np.stack([s.S for s in st_P]))
    e_s = rel_err(stored, np.stack([s.S for s in st_s]))
    print("T=%d state at P vs fp64 %.2e, stored state at %d vs fp64 %.2e" % (T, e_P, snap.state_pos, e_s))
    assert e_P < TOL and e_s < TOL
    snap.release()


def test_config2_T2048_against_oracle_and_sequential(mode):
    # one gated-delta layer at T=2048 with the T=64 case's input distributions; chunked result vs the sequential fp32 recurrence
    x = gdn_inputs(2048, seed=7)
    p = synth.gdn_params(seed=7)
    r = Runner(["linear_attention"], gnorm=False)
    r.set_params(0, p)
    (chunk,), csnap = r.forward([x], keep=True, recurrence=mode)
    (seq,), ssnap = r.forward([x], keep=True, recurrence=ha.SEQUENTIAL)
    ref, st = oracle_gdn(x, p, gnorm=False)
    e_o, e_s = rel_err(chunk, ref), rel_err(_state(csnap)[0], st[0].S)
    e_gpu = rel_err(chunk, seq)
    print("config2 chunked vs fp64: out %.2e state %.2e; vs GPU sequential fp32 %.2e; sequential vs fp64 %.2e"
          % (e_o, e_s, e_gpu, rel_err(seq, ref)))
    assert e_o < TOL and e_s < TOL and e_gpu < TOL
    assert rel_err(_state(csnap)[0], _state(ssnap)[0]) < TOL


def test_slow_decay_state_carry(mode):
    # alpha close to 1 keeps the state alive across many chunks, so inter-chunk error would compound
    x = gdn_inputs(1024, 2, seed=8)
    p = synth.gdn_params(seed=8, neg_exp_A=-0.02, dt_bias=-2.0)
    r = Runner(["linear_attention"], batch=2, gnorm=True)
    r.set_params(0, p)
    (out,), snap = r.forward([x], keep=True, recurrence=mode)
    ref, st = oracle_gdn(x, p, gnorm=True)
    e, es = rel_err(out, ref), max(rel_err(_state(snap, 2)[b], st[b].S) for b in range(2))
    print("slow decay rel_err out %.2e state %.2e" % (e, es))
    assert e < TOL and es < TOL


@pytest.mark.parametrize("T", [1, 3, 63, 65, 130, 200])
def test_unaligned_lengths_f16(T, mode):
    B = 2
    x = gdn_inputs(T, B, seed=9, dtype=np.float16)
    p = synth.gdn_params(seed=9, neg_exp_A=-0.5, dt_bias=0.3)
    r = Runner(["linear_attention"], batch=B, lin_dtype=ha.F16)
    r.set_params(0, p)
    (out,), snap = r.forward([x], keep=True, recurrence=mode)
    ref, _ = oracle_gdn(x.astype(np.float32), p)
    e = rel_err(out, ref)
    print("T=%d f16 rows rel_err %.2e" % (T, e))
    assert e < 1e-2  # f16 outputs
    assert snap.state_pos == 64 * (T // 64) and snap.tail_rows == T - snap.state_pos + 3


@pytest.mark.parametrize("P,L", [(1536, 64), (100, 30), (64, 1), (5, 200), (63, 2), (130, 126)])
def test_prefix_suffix_bit_exact(P, L, mode):
    x = gdn_inputs(P + L, 2, seed=10)
    p = synth.gdn_params(seed=10, neg_exp_A=-0.2)
    r = Runner(["linear_attention"], batch=2)
    r.set_params(0, p)
    (full,), fsnap = r.forward([x], keep=True, recurrence=mode)
    (pre,), snap = r.forward([x[:, :P]], keep=True, recurrence=mode)
    (suf,), ssnap = r.forward([x[:, P:]], cache=snap, keep=True, recurrence=mode)
    np.testing.assert_array_equal(pre, full[:, :P])
    np.testing.assert_array_equal(suf, full[:, P:])
    assert ssnap.state_pos == fsnap.state_pos
    np.testing.assert_array_equal(_state(ssnap, 2), _state(fsnap, 2))


def test_three_way_split_and_decode_steps(mode):
    # prefix, then several short calls (decode-like) must match one forward bit for bit
    x = gdn_inputs(90, 1, seed=11)
    p = synth.gdn_params(seed=11)
    r = Runner(["linear_attention"])
    r.set_params(0, p)
    (full,), _ = r.forward([x], recurrence=mode)
    (o1,), s = r.forward([x[:, :61]], keep=True, recurrence=mode)
    outs = [o1]
    for a, bnd in [(61, 62), (62, 66), (66, 67), (67, 90)]:
        (o,), s = r.forward([x[:, a:bnd]], cache=s, keep=True, recurrence=mode)
        outs.append(o)
    np.testing.assert_array_equal(np.concatenate(outs, 1), full)


@pytest.mark.parametrize("B,form", [(1, ha.CHUNKED_SPLIT), (2, ha.CHUNKED_SPLIT), (4, ha.CHUNKED_PAIRED)])
def test_default_form_by_shape(B, form):
    # HA_CHUNKED picks by batch x heads (16 heads here): the split form up to 32 sequence-heads, the paired form above
    x = gdn_inputs(200, B, seed=12)
    r = Runner(["linear_attention"], batch=B)
    r.set_params(0, synth.gdn_params(seed=12))
    (auto,), sa = r.forward([x], keep=True)
    (forced,), sf = r.forward([x], keep=True, recurrence=form)
    np.testing.assert_array_equal(auto, forced)
    np.testing.assert_array_equal(_state(sa, B), _state(sf, B))


@pytest.mark.parametrize("slow", [False, True], ids=["decay", "slow_decay"])
def test_large_v_headroom(slow, mode):
    # v columns (after the 2 x 16 x 128 q and k columns) scaled by 30: the chunked forms round v and the packed state
    # to f16 as MFMA operands, so large values must keep their relative error (no gated norm, which would rescale
    # the outputs; slow decay lets the state grow to many times |v|)
    x = gdn_inputs(512, 2, seed=13)
    x[:, :, 4096:6144] *= 30.0
    p = synth.gdn_params(seed=13, **(dict(neg_exp_A=-0.02, dt_bias=-2.0) if slow else {}))
    r = Runner(["linear_attention"], batch=2, gnorm=False)
    r.set_params(0, p)
    (out,), snap = r.forward([x], keep=True, recurrence=mode)
    ref, st = oracle_gdn(x, p, gnorm=False)
    e, es = rel_err(out, ref), max(rel_err(_state(snap, 2)[b], st[b].S) for b in range(2))
    print("large v (slow=%s): max |out| %.3g, max |S| %.3g, rel_err out %.2e state %.2e"
          % (slow, np.abs(ref).max(), max(np.abs(s.S).max() for s in st), e, es))
    assert np.isfinite(out).all() and e < TOL and es < TOL
