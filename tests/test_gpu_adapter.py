"""Layer-kind dispatch with the reference's third kind (engine.js:253-276): an `adapter` layer is a projection +
bias stand-in (engine.js:256-261) with no token mixer, so the engine keeps no state for it, ha_forward skips it
(its buffers may be NULL) and snapshots hold no part for it. The mixer layers around it must be unaffected: bit for
bit the outputs of the same engine without the adapter, including across a snapshot/resume."""
import numpy as np
import pytest

import hybrid_attention as ha
import synth

pytestmark = pytest.mark.gpu


def _engine(kinds):
    import torch
    eng = ha.Engine(ha.model_config(kinds, batch=2, max_ctx=512), device=0)
    for i, k in enumerate(kinds):
        if k == "linear_attention":
            for n, v in synth.gdn_params(seed=5, layer=0).items():
                eng.set_param(i, n, v)
        elif k == "full_attention":
            for n, v in synth.gqa_params(seed=5, layer=1, noise=0.1).items():
                eng.set_param(i, n, v)
    return eng, torch


def _run(kinds, rows):
    eng, torch = _engine(kinds)
    L = rows[0].shape[1]
    ins, outs, it = [], [], iter(rows)
    for k in kinds:
        if k == "adapter":
            ins.append(None)
            outs.append(None)
        else:
            dt = torch.float32 if k == "linear_attention" else torch.float16
            ins.append(torch.from_numpy(next(it)).to("cuda:0", dtype=dt))
            outs.append(torch.full((2, L, 2048), float("nan"), dtype=dt, device="cuda:0"))
    eng.forward(L, ins, outs, sync=True)
    return [o.float().cpu().numpy() for o in outs if o is not None]


def test_adapter_layer_is_skipped_and_neighbours_unchanged():
    with_adapter = ["linear_attention", "adapter", "full_attention"]
    without = ["linear_attention", "full_attention"]
    rows = [synth.gdn_rows(96, B=2, seed=5, layer=0), synth.gqa_rows(96, B=2, seed=5, layer=1)]
    a = _run(with_adapter, rows)
    b = _run(without, rows)
    for x, y in zip(a, b):
        assert np.isfinite(x).all()
        np.testing.assert_array_equal(x, y)


def test_adapter_layer_through_snapshot_and_resume():
    kinds = ["linear_attention", "adapter", "full_attention"]
    eng, torch = _engine(kinds)
    pre = [synth.gdn_rows(70, B=2, seed=6, layer=0, part=0), synth.gqa_rows(70, B=2, seed=6, layer=1, part=0)]
    suf = [synth.gdn_rows(30, B=2, seed=6, layer=0, part=1), synth.gqa_rows(30, B=2, seed=6, layer=1, part=1)]

    def fwd(rows, cache=None, keep=False):
        L = rows[0].shape[1]
        x0 = torch.from_numpy(rows[0]).to("cuda:0", dtype=torch.float32)
        x2 = torch.from_numpy(rows[1]).to("cuda:0", dtype=torch.float16)
        y0 = torch.full((2, L, 2048), float("nan"), dtype=torch.float32, device="cuda:0")
        y2 = torch.full((2, L, 2048), float("nan"), dtype=torch.float16, device="cuda:0")
        res = eng.forward(L, [x0, None, x2], [y0, None, y2], cache=cache, keep_cache=keep, sync=True)
        return [y0.float().cpu().numpy(), y2.float().cpu().numpy()], res["cache"]

    _, snap = fwd(pre, keep=True)
    outs, _ = fwd(suf, cache=snap)
    full, _ = fwd([np.concatenate([p, s], 1) for p, s in zip(pre, suf)])
    for o, f in zip(outs, full):
        np.testing.assert_array_equal(o, f[:, 70:])
    with pytest.raises(ha.HAError):  # the adapter layer has no snapshot part
        snap.read(1, "state", np.empty(1, np.float32))
    snap.release()
