"""A whole torso forward (web/public/engine/engine.js:247-285, 313-376) on the GPU: embedding, a linear-attention, a full-
attention, an adapter and a second linear-attention layer, each with its projections, norms and MLP at the model's
widths (D = 2048, I = 6144), random int4 weights, then the final norm of a few rows. Three checks:
- the Node host API (Torso in js/engine.js over the N-API addon) gives, bit for bit, what the Python host mirror
  (hybrid_attention.Torso, the same C ABI calls) gives, for a prefix forward that keeps its cache and a suffix
  forward resumed from it;
- both against an fp64 composition of the oracles (oracle/ C restatement for the token mixers, mnb_oracle for the
  projections, torso_oracle for the rest) that rounds to f16 where the reference stores f16
  (wgsl.js: matmul inputs and outputs, the mixers' outputs);
- the resumed suffix against the same rows of one forward over the whole sequence (bit-exact at these lengths)."""
import json
import os
import shutil
import subprocess
import sys

import numpy as np
import pytest

import hybrid_attention as ha
import synth
from harness import oracle_gdn, oracle_gqa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import mnb_oracle as mo  # noqa: E402
import torso_oracle as to  # noqa: E402

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")]
TYPES = ["linear_attention", "full_attention", "adapter", "linear_attention"]
D, I, VOCAB, L0, L1 = 2048, 6144, 1000, 40, 9
ROWS0, ROWS1 = [0, 17, 39], [0, 8]


def _model(seed=11):
    rng = np.random.default_rng(seed)
    W, V, M = {}, {}, []

    def quant(name, N, K, scale=0.005):
        words = rng.integers(0, 2 ** 32, (N, K // 32, 4), dtype=np.uint64).astype(np.uint32)
        sc = (scale * (0.8 + 0.4 * rng.random((N, K // 32)))).astype(np.float16)
        W[name] = (words, sc, N, K)

    def vec(name, base=1.0, noise=0.1):
        V[name] = (base + noise * rng.normal(size=D)).astype(np.float32)

    quant("embed", VOCAB, D, scale=0.1)
    vec("final_norm")
    for i, t in enumerate(TYPES):
        p = "layers.%d." % i
        vec(p + "in_norm")
        if t == "adapter":
            quant(p + "proj", D, D)
            vec(p + "bias", 0.0, 0.05)
            continue
        if t == "linear_attention":
            quant(p + "in_proj", 8256, D)
            quant(p + "out_proj", D, 2048)
            for k, v in synth.gdn_params(seed=seed, layer=i).items():
                M.append((i, k, np.ascontiguousarray(v, np.float32)))
        else:
            quant(p + "qkv", 5120, D)
            quant(p + "o_proj", D, 2048)
            for k, v in synth.gqa_params(seed=seed, layer=i, noise=0.1).items():
                M.append((i, k, np.ascontiguousarray(v, np.float32)))
        vec(p + "post_norm")
        quant(p + "gate_up", 2 * I, D)
        quant(p + "down", D, I)
    return W, V, M


def _torso(W, V, M):
    """The Python host mirror (hybrid_attention.Torso) loaded with the same model."""
    import torch
    t = ha.Torso(TYPES, D=D, I=I)
    keep = []
    for name, (words, sc, N, K) in W.items():
        q, s = torch.from_numpy(words.view(np.int32)).to("cuda:0"), torch.from_numpy(sc).to("cuda:0")
        t.set_weight(name, ha.MnbWeight(N, K, q, s, None))
    for k, x in V.items():
        t.set_param(k, x)
    for i, k, x in M:
        t.set_param("layers.%d.%s" % (i, k), x)
    return t


def _oracle(W, V, M, ids, rows, deq=None, trace=None):
    """fp64 composition, rounding to f16 where the reference stores f16; one forward over all of ids. `deq` keeps
    the dequantised weights between calls on one model; `trace` (a list) receives the residual stream x entering
    each layer after the first (after the residual add that opens it)."""
    f16 = lambda a: np.asarray(a, np.float64).astype(np.float16).astype(np.float64)  # noqa: E731
    deq = {} if deq is None else deq

    def mm(a, name):
        words, sc, N, K = W[name]
        if name not in deq:
            deq[name] = mo.dequant(words, sc, N, K)
        return f16(mo.matmul(a.astype(np.float16), deq[name]))

    params = {}
    for i, k, x in M:
        params.setdefault(i, {})[k] = x
    words, sc, _, _ = W["embed"]
    x = to.embed(words, sc, ids, D)
    y = None
    for i, t in enumerate(TYPES):
        p = "layers.%d." % i
        h, x = to.add_norm(x, y, V[p + "in_norm"])
        if trace is not None and i > 0:
            trace.append(np.array(x, np.float64))
        h = f16(h)
        if t == "adapter":
            y = f16(mm(h, p + "proj") + V[p + "bias"][None, :])
            continue
        if t == "linear_attention":
            big = mm(h, p + "in_proj")
            out, _ = oracle_gdn(big[None].astype(np.float16), params[i], gnorm=True)
        else:
            big = mm(h, p + "qkv")
            out, _ = oracle_gqa(big[None].astype(np.float16), params[i], 4096)
        o = f16(out[0])
        y = mm(o, p + ("out_proj" if t == "linear_attention" else "o_proj"))
        h, x = to.add_norm(x, y, V[p + "post_norm"])
        g = mm(f16(h), p + "gate_up")
        y = mm(f16(to.silu_mul(g, I)), p + "down")
    hid, _ = to.add_norm(x, y, V["final_norm"], rows=rows)
    return hid


def test_torso_forward_node_matches_c_abi_and_oracle(tmp_path):
    d = str(tmp_path)
    W, V, M = _model()
    rng = np.random.default_rng(5)
    ids = rng.integers(0, VOCAB, L0 + L1).astype(np.uint32)
    spec = {"types": TYPES, "D": D, "I": I, "L0": L0, "L1": L1, "rows0": ROWS0, "rows1": ROWS1,
            "weights": {k: {"N": v[2], "K": v[3]} for k, v in W.items()}, "vectors": sorted(V),
            "mixer": [[i, k] for i, k, _ in M]}
    for k, (words, sc, N, K) in W.items():
        words.tofile(os.path.join(d, "w_%s.q" % k))
        sc.tofile(os.path.join(d, "w_%s.s" % k))
    for k, x in V.items():
        x.tofile(os.path.join(d, "v_%s.bin" % k))
    for i, k, x in M:
        x.tofile(os.path.join(d, "m_%d_%s.bin" % (i, k)))
    ids[:L0].tofile(os.path.join(d, "ids0.bin"))
    ids[L0:].tofile(os.path.join(d, "ids1.bin"))
    with open(os.path.join(d, "spec.json"), "w") as f:
        json.dump(spec, f)
    print("node torso: layers %s L0=%d L1=%d" % (TYPES, L0, L1), flush=True)
    r = subprocess.run([shutil.which("node"), os.path.join(ROOT, "tests", "js", "napi_torso.js"), d],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    info = json.loads(r.stdout.strip().splitlines()[-1])
    js0 = np.fromfile(os.path.join(d, "hidden0.bin"), np.float32).reshape(len(ROWS0), D)
    js1 = np.fromfile(os.path.join(d, "hidden1.bin"), np.float32).reshape(len(ROWS1), D)

    t = _torso(W, V, M)
    py0, snaps = t.forward(ids[:L0], ROWS0, keep=True)
    py1, _ = t.forward(ids[L0:], ROWS1, cache=snaps)
    full, _ = t.forward(ids, ROWS0 + [L0 + r for r in ROWS1])
    assert np.array_equal(js0, py0), "prefix hidden rows differ between Node and the C ABI"
    assert np.array_equal(js1, py1), "resumed hidden rows differ between Node and the C ABI"

    ref = _oracle(W, V, M, ids, ROWS0 + [L0 + r for r in ROWS1])
    e0 = mo.rel_err(py0, ref[:len(ROWS0)])
    e1 = mo.rel_err(py1, ref[len(ROWS0):])
    ef = mo.rel_err(full[len(ROWS0):], py1)
    print("torso vs oracle: prefix %.1e, resumed suffix %.1e; resumed vs one forward %.1e" % (e0, e1, ef))
    assert e0 < 1e-2 and e1 < 1e-2
    # the mixers' prefix + suffix is bit-exact, and at 9 and 49 rows the projections take the same per-row path
    # (the MFMA GEMV, M <= 64), so the resumed rows equal those of one forward bit for bit
    assert np.array_equal(full[len(ROWS0):], py1)

    # diagnostics (engine.js:292-307, 331-348): the residual stream entering layers 1.. against the oracle's and, bit
    # for bit, the Python mirror's; the GPU time of the forward; a per-step profile naming every kind of step
    trace = []
    _oracle(W, V, M, ids[:L0], ROWS0, trace=trace)
    js_layers = np.fromfile(os.path.join(d, "layers.bin"), np.float32).reshape(len(TYPES) - 1, L0, D)
    t.forward(ids[:L0], ROWS0, timestamps=True, debug_layers=True)
    assert info["n_layers"] == len(TYPES) - 1 and len(t.diag["layers"]) == len(TYPES) - 1
    for i, (a, b, ref_x) in enumerate(zip(js_layers, t.diag["layers"], trace)):
        assert np.array_equal(a, b), "layer %d residual differs between Node and the C ABI" % (i + 1)
        e = mo.rel_err(a, ref_x)
        print("residual entering layer %d vs oracle: %.1e" % (i + 1, e))
        assert e < 1e-2
    print("gpu_ms Node %.3f, Python %.3f; fetch_ms %.3f; profile %s" % (
        info["gpu_ms"], t.diag["gpu_ms"], info["fetch_ms"], info["profile"]))
    assert 0 < info["gpu_ms"] < 1000 and 0 < t.diag["gpu_ms"] < 1000
    prof, pyprof = info["profile"], t.profile(ids[:L0])
    for step in ("embed", "in_norm", "in_proj", "gdn", "out_proj", "qkv", "attn", "o_proj", "proj", "bias",
                 "post_norm", "gate_up", "silu", "down"):
        assert step in prof and step in pyprof, step
    assert list(prof.values()) == sorted(prof.values(), reverse=True)
