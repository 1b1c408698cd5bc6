"""The reference's context cap (engine.js:92,316: LT = 4096) on a one-sequence engine, where the gated-delta layer
runs the split chunked form (chunk-parallel preparation and output, a sequential state pass) and the GQA layer splits key ranges over workgroups: a 4000-row prefix kept as a
snapshot plus a 96-row suffix equals one 4096-row forward bit for bit, both match the fp64 oracle, and one row more
is refused with HA_ERR_CONTEXT."""
import numpy as np
import pytest

import hybrid_attention as ha
import synth
from harness import Runner, oracle_gdn, oracle_gqa, rel_err

pytestmark = pytest.mark.gpu
KINDS = ["linear_attention", "full_attention"]
LT = 4096


def _runner():
    r = Runner(KINDS, batch=1, max_ctx=LT)
    r.set_params(0, synth.gdn_params(seed=21))
    r.set_params(1, synth.gqa_params(seed=21, layer=1, noise=0.1))
    return r


def test_full_context_prefix_suffix_and_oracle():
    print("context cap: P=4000 + L=96 vs one 4096-row forward", flush=True)
    r = _runner()
    full_in = [synth.gdn_rows(LT, seed=21), synth.gqa_rows(LT, seed=21, layer=1)]
    full, _ = r.forward(full_in)
    P = 4000
    _, snap = r.forward([x[:, :P] for x in full_in], keep=True)
    suf, _ = r.forward([x[:, P:] for x in full_in], cache=snap)
    for i in range(2):
        np.testing.assert_array_equal(suf[i], full[i][:, P:], err_msg="layer %d" % i)
    ref_l, _ = oracle_gdn(full_in[0], synth.gdn_params(seed=21))
    ref_g, _ = oracle_gqa(full_in[1], synth.gqa_params(seed=21, layer=1, noise=0.1), LT)
    el, eg = rel_err(full[0], ref_l), rel_err(full[1], ref_g)
    print("  4096 rows vs oracle: gated-delta %.2e, GQA %.2e" % (el, eg))
    assert el < 2e-3 and eg < 1e-2
    # the last rows alone (attention over the whole cache)
    assert rel_err(full[1][:, -64:], ref_g[:, -64:]) < 1e-2
    with pytest.raises(ha.HAError) as ei:
        r.forward([synth.gdn_rows(97, seed=22), synth.gqa_rows(97, seed=22, layer=1)], cache=snap)
    assert ei.value.code == ha.HA_ERR_CONTEXT
    snap.release()
