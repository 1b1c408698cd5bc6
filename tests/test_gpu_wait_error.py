"""Bounded cross-workgroup waits that run out are reported, not computed over (engine.js:373 throws the device
errors a forward collected). ha_forward_opts.debug_unpublished_waits makes every such wait of one call look for a
value no workgroup of that launch publishes, for a few polls; every kernel still ends normally. The call then fails
with HA_ERR_DEVICE where it synchronises (or the engine's next call does), no snapshot of it is kept, and the
engine's next forward runs normally: bit for bit what a fresh engine computes."""
import numpy as np
import pytest

import hybrid_attention as ha
import synth
from harness import Runner, gdn_inputs

pytestmark = pytest.mark.gpu


def _dev(torch, x, dt):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0", dtype=dt)


def _call(torch, run, x, dt, **kw):
    """One forward of a one-layer engine on x; returns the output (host) and the result dict."""
    L = x.shape[1]
    xi = [_dev(torch, x, dt)]
    out = [torch.full((x.shape[0], L, 2048), float("nan"), dtype=dt, device="cuda:0")]
    torch.cuda.synchronize()
    res = run.eng.forward(L, xi, out, **kw)
    torch.cuda.synchronize()
    return out[0].float().cpu().numpy(), res


# the three bounded waits: the paired form's tile sets, the split form's packed states, the split-key GQA merge
CASES = [("paired", ["linear_attention"], 1, ha.CHUNKED_PAIRED, 200),
         ("split", ["linear_attention"], 1, ha.CHUNKED_SPLIT, 200),
         ("gqa-merge", ["full_attention"], 1, ha.CHUNKED, 1500)]


@pytest.mark.parametrize("name,kinds,B,rec,T", CASES, ids=[c[0] for c in CASES])
def test_wait_that_runs_out_is_reported(name, kinds, B, rec, T):
    import torch
    lin = kinds[0] == "linear_attention"
    print("wait error: %s B=%d T=%d" % (name, B, T), flush=True)
    if lin:
        x, dt, params = gdn_inputs(T, B, seed=21), torch.float32, synth.gdn_params(seed=21)
    else:
        x, dt, params = synth.gqa_rows(T, B, seed=21).astype(np.float16), torch.float16, synth.gqa_params(seed=21, noise=0.1)
    run = Runner(kinds, batch=B)
    run.set_params(0, params)
    want, _ = _call(torch, run, x, dt, recurrence=rec, sync=True)

    # reported where the call synchronises; no snapshot of the failed call is handed out
    with pytest.raises(ha.HAError) as ei:
        _call(torch, run, x, dt, recurrence=rec, sync=True, keep_cache=True, debug_unpublished_waits=True)
    assert ei.value.code == ha.HA_ERR_DEVICE, str(ei.value)
    assert "gave up waiting" in str(ei.value)
    # reported once: the next call runs, and computes what it computed before
    got, _ = _call(torch, run, x, dt, recurrence=rec, sync=True)
    assert np.array_equal(got, want)

    # without a synchronising call the failure is reported by the engine's next call, which does not run
    _call(torch, run, x, dt, recurrence=rec, debug_unpublished_waits=True)
    with pytest.raises(ha.HAError) as ei:
        _call(torch, run, x, dt, recurrence=rec, sync=True)
    assert ei.value.code == ha.HA_ERR_DEVICE
    got, _ = _call(torch, run, x, dt, recurrence=rec, sync=True)
    assert np.array_equal(got, want)

    # ... or by ha_synchronize
    _call(torch, run, x, dt, recurrence=rec, debug_unpublished_waits=True)
    with pytest.raises(ha.HAError) as ei:
        run.eng.synchronize()
    assert ei.value.code == ha.HA_ERR_DEVICE
    run.eng.synchronize()


def test_forms_without_waits_ignore_the_option():
    # the sequential and fused forms and an unsplit GQA launch have no cross-workgroup wait: nothing to report, and
    # the outputs are the usual ones
    import torch
    x = gdn_inputs(130, 4, seed=22)
    run = Runner(["linear_attention"], batch=4)
    run.set_params(0, synth.gdn_params(seed=22))
    for rec in (ha.SEQUENTIAL, ha.CHUNKED_FUSED):
        want, _ = _call(torch, run, x[:, :40] if rec == ha.SEQUENTIAL else x, torch.float32, recurrence=rec, sync=True)
        got, _ = _call(torch, run, x[:, :40] if rec == ha.SEQUENTIAL else x, torch.float32, recurrence=rec, sync=True,
                       debug_unpublished_waits=True)
        assert np.array_equal(got, want)
    q = synth.gqa_rows(300, 4, seed=22).astype(np.float16)
    full = Runner(["full_attention"], batch=4)  # 8 (sequence, KV head) pairs: no split key ranges
    full.set_params(0, synth.gqa_params(seed=22, noise=0.1))
    want, _ = _call(torch, full, q, torch.float16, sync=True)
    got, _ = _call(torch, full, q, torch.float16, sync=True, debug_unpublished_waits=True)
    assert np.array_equal(got, want)
