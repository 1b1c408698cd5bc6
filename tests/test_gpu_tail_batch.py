"""Raw-row tails of many gated-delta layers. The engine gathers the tail copies of one call into launches of up to
32 layers, or launches one per layer when per-layer times are asked for. With 35 gated-delta layers, both launch
forms (32 + 3 layers, and 35 single ones) must leave tails that resume bit-exactly. A suffix resumed from a prefix
snapshot must equal the same rows of one longer forward, for every layer (resume engine.js:325-328; conv history
roll wgsl.js:420-434). The prefix (100 rows) ends inside a chunk, so every tail holds replay rows as well as the
conv history."""
import numpy as np
import pytest

import synth
from harness import Runner

pytestmark = pytest.mark.gpu
N = 35


def _inputs(T, part, B):
    return [synth.gdn_rows(T, B, seed=5, layer=i, part=part) for i in range(N)]


@pytest.mark.parametrize("batch,layer_ms", [(1, False), (3, False), (3, True)])
def test_many_layer_tails_resume_bit_exact(batch, layer_ms):
    print("tails: %d gated-delta layers, batch %d, layer_ms %s" % (N, batch, layer_ms), flush=True)
    r = Runner(["linear_attention"] * N, batch=batch)
    for i in range(N):
        r.set_params(i, synth.gdn_params(seed=5, layer=i))
    prefix, suffix = _inputs(100, 0, batch), _inputs(37, 1, batch)
    _, snap = r.forward(prefix, keep=True, layer_ms=layer_ms)
    assert snap.P == 100 and snap.state_pos == 64
    outs, _ = r.forward(suffix, cache=snap, layer_ms=layer_ms)
    full, _ = r.forward([np.concatenate([p, q], 1) for p, q in zip(prefix, suffix)], layer_ms=layer_ms)
    for i in range(N):
        assert np.isfinite(outs[i]).all(), i
        np.testing.assert_array_equal(outs[i], full[i][:, 100:], err_msg="layer %d" % i)
    snap.release()
