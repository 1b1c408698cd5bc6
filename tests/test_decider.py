"""The worker-level host (strands-decider-web_amd/js/decider.js) on the CPU, through Node:
- prompt rendering against the reference's recorded prompts for its fixtures (tests/golden/decider_cases.json, from
  ref/fixtures.json + ref/reference_cpu.json): state + question text, byte for byte;
- the answer derivation against the recorded answers: choice confidence (n p_max - 1) / (n - 1), the score's mean
  and ordinal confidence, noul, from the recorded probabilities;
- option positions with a byte-level tokenizer (one token per byte): the last token of each option line;
- the pointer head against a numpy restatement (LayerNorm eps 1e-5 -> q / k projections -> scaled dot product /
  temperature -> softmax) on random weights from a safetensors file;
- the LRU(4) prefix cache: the least recently used snapshot is released first."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which("node")
MOD = os.path.join(ROOT, "strands-decider-web_amd", "js", "decider.js")
pytestmark = pytest.mark.skipif(NODE is None or not os.path.exists(
    os.path.join(ROOT, "strands-decider-web_amd", "js", "ha_napi.node")), reason="node or the built addon is missing")
CASES = json.load(open(os.path.join(ROOT, "tests", "golden", "decider_cases.json"), encoding="utf-8"))


def _node(js):
    r = subprocess.run([NODE, "-e", "const D = require(%r);\n" % MOD + js], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_prompts_match_the_reference_fixtures():
    out = _node("const c = %s; console.log(JSON.stringify(c.map((x) => [D.renderState(x.state) + "
                "D.renderQuestion(x.question).text, D.renderQuestion(x.question).labels])));" % json.dumps(CASES))
    for (text, labels), c in zip(out, CASES):
        assert text == c["prompt"], c["name"]
        assert labels == c["labels"], c["name"]


def test_answers_match_the_reference_fixtures():
    # a noul answer records only p(true); its two probabilities are 1 - noul and noul
    probs = [[1 - c["answer"]["noul"], c["answer"]["noul"]] if c["kind"] == "noul"
             else [c["answer"]["probabilities"][l] for l in c["labels"]] for c in CASES]
    out = _node("const c = %s; const p = %s; console.log(JSON.stringify(c.map((x, i) => "
                "D.readAnswer(D.renderQuestion(x.question), p[i], 0.1))));" % (json.dumps(CASES), json.dumps(probs)))
    for got, c in zip(out, CASES):
        want = c["answer"]
        assert got["type"] == want["type"]
        for k in ("confidence", "score", "noul"):
            if k in want:
                assert abs(got[k] - want[k]) < 1e-3, (c["name"], k, got[k], want[k])  # recorded to 4 decimals
        if "choice" in want:
            assert got["choice"] == want["choice"]


def test_option_positions_with_a_byte_tokenizer():
    js = ("const tok = { encode: (t) => { const b = Buffer.from(t, 'utf8'); return { ids: Array.from(b),"
          " tokens: Array.from(b, (x) => String.fromCharCode(x)) }; } };"
          "const q = {type: 'choice', instructions: 'Pick éè', options: ['alpha', 'bêta']};"
          "const b = D.buildInputs(tok, 'stäte', q, 4096);"
          "const t = D.renderQuestion(q).text;"
          "console.log(JSON.stringify({b: b, s: D.renderState('stäte'), t: t}));")
    out = _node(js)
    b, s, t = out["b"], out["s"], out["t"]
    sb, tb = s.encode(), t.encode()
    assert b["stateLen"] == len(sb) and b["ids"] == list(sb) + list(tb)
    for pos, label in zip(b["optIdx"], ["alpha", "bêta"]):
        line = ("%d. %s" % (1 if label == "alpha" else 2, label)).encode()
        end = tb.index(line) + len(line)  # the option line's last byte
        assert pos == len(sb) + end - 1


def test_pointer_head_matches_numpy(tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(0)
    d, e = 64, 16
    H = {"norm.weight": rng.normal(size=d), "norm.bias": rng.normal(size=d), "q.weight": rng.normal(size=(e, d)),
         "q.bias": rng.normal(size=e), "k.weight": rng.normal(size=(e, d)), "k.bias": rng.normal(size=e)}
    H = {k: v.astype(np.float32) for k, v in H.items()}
    p = os.path.join(str(tmp_path), "head.safetensors")
    save_file(H, p)
    hid = rng.normal(size=(5, d)).astype(np.float32)
    out = _node("const H = D.loadHead(require('fs').readFileSync(%r)); const h = new Float32Array(%s);"
                "console.log(JSON.stringify(D.pointerLogits(H, h, %d, 4, [0, 2, 3], 0.7)));"
                % (p, json.dumps(hid.ravel().tolist()), d))

    def proj(name, x):
        xn = (x - x.mean()) / np.sqrt(x.var() + 1e-5) * H["norm.weight"] + H["norm.bias"]
        return H[name + ".weight"].astype(np.float64) @ xn + H[name + ".bias"]

    q = proj("q", hid[4].astype(np.float64))
    lg = np.array([proj("k", hid[i].astype(np.float64)) @ q / np.sqrt(e) / 0.7 for i in (0, 2, 3)])
    pr = np.exp(lg - lg.max())
    pr /= pr.sum()
    np.testing.assert_allclose(out["logits"], lg, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(out["probs"], pr, rtol=1e-4, atol=1e-5)


def test_prefix_cache_lru():
    out = _node("const c = new D.PrefixCache(4); const rel = [];"
                "const snap = (n) => ({ release: () => rel.push(n) });"
                "[1, 2, 3, 4].forEach((n) => c.put(String(n), snap(n)));"
                "c.get([1]);"                       # 1 becomes most recent
                "c.put('5', snap(5));"              # evicts 2
                "c.put('6', snap(6));"              # evicts 3
                "console.log(JSON.stringify({rel: rel, hit1: !!c.get([1]).hit, hit2: !!c.get([2]).hit}));")
    assert out == {"rel": [2, 3], "hit1": True, "hit2": False}
