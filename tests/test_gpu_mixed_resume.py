"""Resuming across recurrence modes on the GPU. A snapshot taken after a chunked forward stores the state at the last
64-row boundary plus the raw rows since; a sequential resume replays those rows before its own (gdn_seq_kernel with
state_pos < P). A snapshot taken after a sequential forward stores the state at P (not a chunk boundary); a chunked
resume then starts its chunks there. Both must match the fp64 oracle of one uninterrupted sequence (bar 2e-3);
the forms round differently, so bit equality is only required within one form (the resume tests)."""
import numpy as np
import pytest

import hybrid_attention as ha
import synth
from harness import Runner, oracle_gdn, rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("first,second,P,L", [
    (ha.CHUNKED, ha.SEQUENTIAL, 100, 37),
    (ha.CHUNKED_SPLIT, ha.SEQUENTIAL, 64 * 3 + 5, 1),
    (ha.SEQUENTIAL, ha.CHUNKED, 100, 150),
    (ha.SEQUENTIAL, ha.CHUNKED_FUSED, 37, 64),
    (ha.SEQUENTIAL, ha.CHUNKED_SPLIT, 129, 70),
    (ha.CHUNKED_PAIRED, ha.SEQUENTIAL, 64 * 2 + 33, 9),
    (ha.SEQUENTIAL, ha.CHUNKED_PAIRED, 71, 100)])
def test_mixed_mode_resume(first, second, P, L):
    print("mixed resume: mode %d for %d rows, then mode %d for %d rows" % (first, P, second, L), flush=True)
    r = Runner(["linear_attention"], batch=2)
    prm = synth.gdn_params(seed=31)
    r.set_params(0, prm)
    x = synth.gdn_rows(P + L, B=2, seed=31)
    _, snap = r.forward([x[:, :P]], keep=True, recurrence=first)
    exp_pos = P if first == ha.SEQUENTIAL else 64 * (P // 64)
    assert snap.state_pos == exp_pos
    outs, snap2 = r.forward([x[:, P:]], cache=snap, keep=True, recurrence=second)
    ref, states = oracle_gdn(x, prm)
    err = rel_err(outs[0], ref[:, P:])
    print("  suffix vs oracle %.2e" % err)
    assert err < 2e-3
    if second == ha.SEQUENTIAL:
        S = np.empty((2, 16, 128, 128), np.float32)
        snap2.read(0, "state", S)
        es = rel_err(S, np.stack([s.S for s in states]))
        print("  final state vs oracle %.2e" % es)
        assert es < 2e-3
    snap.release()
    snap2.release()
