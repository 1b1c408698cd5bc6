"""Config 4 on the GPU: the 24-layer hybrid stack (18 gated-delta + 6 GQA layers in the 3:1 pattern), B = 8
sequences, T = 8, 128, 512 and 2048, through the engine's default recurrence choice (the configuration bench.py
times). Inputs are drawn on the device (torch's seeded generator, as the bench does); the rows of the sampled
sequences are copied back for the oracle. Checks:
  - every output of every layer is finite;
  - every layer matches the fp64 oracle (bars 2e-3 and 1e-2): all 8 sequences at T <= 512, and at T = 2048 one
    sequence per layer, layer i checking sequence i % 8, so that every sequence is checked on three layers;
  - sequences 0 and 7 are bit-identical to the same rows run through a two-sequence engine of the same layers."""
import numpy as np
import pytest

import hybrid_attention as ha
import synth
from harness import oracle_gdn, oracle_gqa, rel_err

pytestmark = pytest.mark.gpu
KINDS = (["linear_attention"] * 3 + ["full_attention"]) * 6
LIN_TOL, GQA_TOL = 2e-3, 1e-2


def _params(i, k):
    return synth.gdn_params(seed=11, layer=i) if k == "linear_attention" else synth.gqa_params(seed=11, layer=i,
                                                                                                noise=0.1)


def _engine(kinds, batch, max_ctx):
    eng = ha.Engine(ha.model_config(kinds, batch=batch, max_ctx=max_ctx), device=0)
    for i, k in enumerate(kinds):
        for n, v in _params(i, k).items():
            eng.set_param(i, n, v)
    return eng


@pytest.mark.parametrize("T", [8, 128, 512, 2048])
def test_config4_stack(T):
    import torch
    B, dev = 8, "cuda:0"
    print("config 4 stack: B=%d T=%d, 24 layers" % (B, T), flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(1000 + T)
    ins, outs = [], []
    for k in KINDS:
        if k == "linear_attention":
            x = torch.randn(B, T, 8256, device=dev, generator=g)
            x[:, :, synth.lin_width():] = 0.0
            ins.append(x)
            outs.append(torch.full((B, T, 2048), float("nan"), device=dev))
        else:
            ins.append(torch.randn(B, T, 5120, device=dev, generator=g).half())
            outs.append(torch.full((B, T, 2048), float("nan"), device=dev, dtype=torch.float16))
    eng = _engine(KINDS, B, 2048)
    torch.cuda.synchronize()
    eng.forward(T, ins, outs, sync=True)
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert bool(torch.isfinite(o.float()).all()), "layer %d has non-finite outputs" % i

    worst = {"linear_attention": 0.0, "full_attention": 0.0}
    for i, k in enumerate(KINDS):
        seqs = list(range(B)) if T <= 512 else [i % B]
        x = ins[i][seqs].cpu().numpy()
        if k == "linear_attention":
            ref, _ = oracle_gdn(x, _params(i, k))
            e = rel_err(outs[i][seqs].cpu().numpy(), ref)
        else:
            ref, _ = oracle_gqa(x, _params(i, k), 2048)
            e = rel_err(outs[i][seqs].float().cpu().numpy(), ref)
        worst[k] = max(worst[k], e)
        assert e < (LIN_TOL if k == "linear_attention" else GQA_TOL), "layer %d (%s) sequences %s: rel_err %.2e" % (
            i, k, seqs, e)
    print("  every layer vs oracle: gated-delta worst %.2e (bar %.0e), GQA worst %.2e (bar %.0e)" % (
        worst["linear_attention"], LIN_TOL, worst["full_attention"], GQA_TOL))
    pick = [0, 7]

    # the same rows through a two-sequence engine of layers 0..4 with the same recurrence form
    sub = KINDS[:5]
    e2 = _engine(sub, 2, 2048)
    ins2 = [ins[i][pick].contiguous() for i in range(5)]
    outs2 = [torch.full_like(outs[i][pick], float("nan")) for i in range(5)]
    rec = ha.CHUNKED_PAIRED  # the form HA_CHUNKED picks for 8 x 16 sequence-heads
    torch.cuda.synchronize()
    e2.forward(T, ins2, outs2, recurrence=rec, sync=True)
    torch.cuda.synchronize()
    for i in range(5):
        a = outs[i][pick].cpu().numpy().view(np.uint16 if outs[i].dtype == torch.float16 else np.uint32)
        b = outs2[i].cpu().numpy().view(a.dtype)
        assert np.array_equal(a, b), "layer %d: B=8 rows differ from the two-sequence engine" % i
