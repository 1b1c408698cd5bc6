"""Shared helpers for the GPU tests: run the engine on seeded inputs through the C ABI, and the oracle beside it."""
import numpy as np

import hybrid_attention as ha
import oracle
import synth


class Runner:
    """One engine plus device buffers; inputs are numpy [B][L][stride] arrays (copied to HBM per call)."""

    def __init__(self, kinds, batch=1, max_ctx=4096, lin_dtype=ha.F32, full_dtype=ha.F16, gnorm=True):
        import torch
        self.torch = torch
        self.cfg = ha.model_config(kinds, batch=batch, max_ctx=max_ctx, lin_dtype=lin_dtype, full_dtype=full_dtype,
                                   lin_gnorm=gnorm)
        self.kinds = self.cfg["kinds"]
        self.B = batch
        self.eng = ha.Engine(self.cfg, device=0)

    def set_params(self, layer, params):
        for k, v in params.items():
            self.eng.set_param(layer, k, v)

    def _dt(self, kind):
        t = self.torch
        d = self.cfg["lin_dtype"] if kind == ha.LINEAR else self.cfg["full_dtype"]
        return t.float16 if d == ha.F16 else t.float32

    def forward(self, inputs, cache=None, keep=False, recurrence=ha.CHUNKED, layer_ms=False):
        t = self.torch
        L = inputs[0].shape[1]
        dev_in = [t.from_numpy(np.ascontiguousarray(x)).to("cuda:0", dtype=self._dt(k))
                  for x, k in zip(inputs, self.kinds)]
        dev_out = [t.full((self.B, L, 2048), float("nan"), dtype=self._dt(k), device="cuda:0") for k in self.kinds]
        t.cuda.synchronize()
        res = self.eng.forward(L, dev_in, dev_out, cache=cache, keep_cache=keep, recurrence=recurrence, sync=True,
                               layer_ms=layer_ms)
        t.cuda.synchronize()
        return [o.float().cpu().numpy() for o in dev_out], res["cache"]


def gdn_inputs(T, B=1, seed=0, layer=0, part=0, dtype=np.float32):
    x = synth.gdn_rows(T, B, seed=seed, layer=layer, part=part)
    return x.astype(dtype)


def oracle_gdn(rows_b, params, gnorm=True, states=None, chunk=0):
    """rows_b [B][T][stride] (any float dtype) -> outputs [B][T][2048], states."""
    B = rows_b.shape[0]
    states = states or [oracle.GdnState() for _ in range(B)]
    outs = [oracle.gdn_forward(rows_b[b].astype(np.float32), params, states[b], gnorm=gnorm, chunk=chunk)
            for b in range(B)]
    return np.stack(outs), states


def oracle_gqa(rows_b, params, LT, caches=None, f16=True):
    B = rows_b.shape[0]
    rope = oracle.rope_table(LT, 64, 1e7)
    caches = caches or [oracle.GqaCache(LT) for _ in range(B)]
    outs = [oracle.gqa_forward(rows_b[b].astype(np.float32), params, caches[b], rope, f16=f16) for b in range(B)]
    return np.stack(outs), caches


rel_err = oracle.rel_err
