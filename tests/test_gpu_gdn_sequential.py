"""GPU parity of the sequential gated-delta kernel (decode / resume path) against the fp64 oracle."""
import numpy as np
import pytest

import hybrid_attention as ha
import synth
from harness import Runner, gdn_inputs, oracle_gdn, rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-3  # north-star bar for the fp32 recurrence (max |err| / max |ref|)


def _state(snap, B=1):
    s = np.zeros((B, 16, 128, 128), np.float32)
    return snap.read(0, "state", s)


@pytest.mark.parametrize("gnorm", [False, True])
def test_config0_sequential(gnorm):
    # the CPU-runnable case: T=64, 16 heads, fp32 rows, conv taps N(0, 0.5^2), negA = -1, dt_bias = 0, S0 = 0
    x = gdn_inputs(64)
    p = synth.gdn_params()
    r = Runner(["linear_attention"], gnorm=gnorm)
    r.set_params(0, p)
    (out,), snap = r.forward([x], keep=True, recurrence=ha.SEQUENTIAL)
    ref, st = oracle_gdn(x, p, gnorm=gnorm)
    e = rel_err(out, ref)
    print("config0 sequential gnorm=%s rel_err out %.2e" % (gnorm, e))
    assert e < TOL
    es = rel_err(_state(snap)[0], st[0].S)
    print("state rel_err %.2e" % es)
    assert es < TOL
    assert snap.P == 64 and snap.state_pos == 64 and snap.tail_rows == 3


def test_sequential_batch_f16_rows():
    B, T = 3, 50
    x = gdn_inputs(T, B, seed=1, dtype=np.float16)
    p = synth.gdn_params(seed=1, neg_exp_A=-0.3, dt_bias=0.5)
    r = Runner(["linear_attention"], batch=B, lin_dtype=ha.F16)
    r.set_params(0, p)
    (out,), _ = r.forward([x], recurrence=ha.SEQUENTIAL)
    ref, _ = oracle_gdn(x.astype(np.float32), p)
    e = rel_err(out, ref)
    print("B=3 f16 rows rel_err %.2e" % e)
    assert e < 1e-2  # f16 output rounding (2^-11) plus the fp32 recurrence


@pytest.mark.parametrize("P,L", [(37, 27), (1, 5), (64, 64), (3, 1)])
def test_sequential_prefix_suffix_bit_exact(P, L):
    x = gdn_inputs(P + L, 2, seed=2)
    p = synth.gdn_params(seed=2)
    r = Runner(["linear_attention"], batch=2)
    r.set_params(0, p)
    (full,), fsnap = r.forward([x], keep=True, recurrence=ha.SEQUENTIAL)
    (pre,), snap = r.forward([x[:, :P]], keep=True, recurrence=ha.SEQUENTIAL)
    (suf,), ssnap = r.forward([x[:, P:]], cache=snap, keep=True, recurrence=ha.SEQUENTIAL)
    np.testing.assert_array_equal(pre, full[:, :P])
    np.testing.assert_array_equal(suf, full[:, P:])
    np.testing.assert_array_equal(_state(ssnap, 2), _state(fsnap, 2))
