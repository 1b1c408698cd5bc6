"""Call-time device buffers held by several engines (ha_share_scratch) and allocated on demand:
- engines holding one set (a one-sequence gated-delta engine, also forced to the paired form, a four-sequence one,
  also forced to the split and fused forms, and a one-sequence full-attention engine with split key ranges), called
  one after another on one stream, give bit for bit what engines with their own sets give, through every form
  (split, paired, fused, sequential, split GQA) and again on a second round of calls;
- the one-sequence shape picks the split form and the four-sequence shape the paired form, so the one-sequence
  engine's paired tile sets and the four-sequence engine's chunk images come from the first calls that force those
  forms: the latter's outputs also match the fp64 oracle."""
import numpy as np
import pytest

import hybrid_attention as ha
import synth
from harness import Runner, gdn_inputs, oracle_gdn, rel_err

pytestmark = pytest.mark.gpu


def _engines(torch, share):
    lin1 = Runner(["linear_attention"], batch=1, max_ctx=512)
    lin4 = Runner(["linear_attention"], batch=4, max_ctx=512)
    full = Runner(["full_attention"], batch=1, max_ctx=512)
    for r, seed in ((lin1, 3), (lin4, 4)):
        r.set_params(0, synth.gdn_params(seed=seed))
    full.set_params(0, synth.gqa_params(seed=5, noise=0.1))
    if share:
        st = torch.cuda.Stream(device="cuda:0").cuda_stream
        for r in (lin1, lin4, full):
            r.eng.set_stream(st)
        lin4.eng.share_scratch(lin1.eng)
        full.eng.share_scratch(lin1.eng)
    return lin1, lin4, full


def _calls(lin1, lin4, full):
    x1 = gdn_inputs(300, seed=3)
    x4 = gdn_inputs(130, 4, seed=4)
    q = synth.gqa_rows(300, seed=5).astype(np.float16)
    out = []
    for _ in range(2):
        out.append(lin1.forward([x1])[0][0])                                # split form by shape
        out.append(lin1.forward([x1], recurrence=ha.CHUNKED_PAIRED)[0][0])  # tile sets from a forced call
        out.append(full.forward([q])[0][0])                                 # split key ranges
        out.append(lin4.forward([x4], recurrence=ha.CHUNKED_SPLIT)[0][0])   # images from a forced call
        out.append(lin4.forward([x4[:, :40]], recurrence=ha.SEQUENTIAL)[0][0])
        out.append(lin4.forward([x4])[0][0])                                # paired form by shape
        out.append(lin4.forward([x4], recurrence=ha.CHUNKED_FUSED)[0][0])   # fused kernel, forced
    return out, x4


def test_shared_scratch_is_bit_identical_and_lazy_images_match_the_oracle():
    import torch
    print("own sets", flush=True)
    own, x4 = _calls(*_engines(torch, share=False))
    print("one shared set", flush=True)
    shared, _ = _calls(*_engines(torch, share=True))
    names = ["split B=1", "forced paired B=1", "GQA split", "forced split B=4", "sequential B=4", "paired B=4",
             "fused B=4"] * 2
    for n, a, b in zip(names, own, shared):
        assert np.array_equal(a, b), n
    for a, b in zip(own[:7], own[7:]):  # a second round of calls on the same buffers
        assert np.array_equal(a, b)
    ref, _ = oracle_gdn(x4, synth.gdn_params(seed=4))
    e = rel_err(own[3], ref)
    print("forced split form at B=4 vs fp64: %.2e" % e)
    assert e < 2e-3


def test_engines_sharing_a_set_stay_on_one_stream():
    # engines holding one set of call-time buffers use the same progress counters and tile-set slots, so they must
    # never run on two streams at once: sharing needs one stream, and an engine that moves to another stream gets a
    # set of its own first; its calls then compute what they computed before
    import torch
    lin1, lin4, _ = _engines(torch, share=False)
    s1 = torch.cuda.Stream(device="cuda:0").cuda_stream
    s2 = torch.cuda.Stream(device="cuda:0").cuda_stream
    lin1.eng.set_stream(s1)
    lin4.eng.set_stream(s2)
    with pytest.raises(ha.HAError) as ei:
        lin4.eng.share_scratch(lin1.eng)
    assert ei.value.code == ha.HA_ERR_ARG
    x4 = gdn_inputs(130, 4, seed=4)
    want = lin4.forward([x4])[0][0]
    lin4.eng.set_stream(s1)
    lin4.eng.share_scratch(lin1.eng)
    assert np.array_equal(lin4.forward([x4])[0][0], want)
    lin4.eng.set_stream(s2)  # leaves lin1's set for one of its own
    assert np.array_equal(lin4.forward([x4])[0][0], want)
    x1 = gdn_inputs(300, seed=3)
    a = lin1.forward([x1])[0][0]
    lin1.eng.set_stream(None)  # lin1 holds its set alone now: it keeps it
    assert np.array_equal(lin1.forward([x1])[0][0], a)
