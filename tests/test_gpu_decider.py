"""The worker-level host (js/decider.js) on the GPU, over an export loaded by js/loader.js:
- decide on a whole prompt against an fp64 composition of the oracles: the torso oracle chain of
  tests/test_gpu_torso_model.py over the same prompt ids (byte tokenizer), then the pointer head of head.js in
  numpy (LayerNorm eps 1e-5, q / k projections, q . k / sqrt(64) / temperature, softmax) on the option rows and the
  last row: logits and probabilities;
- decideMany (the state encoded once, each question's suffix resumed from its snapshot, worker.js:216-236) gives the
  answers that separate decide calls on the whole prompt give (within f16 storage steps: the suffix's projections
  see fewer rows); a decide on a cached state runs only the suffix; the prefix cache keeps 4 states and releases the
  least recently used."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from export_fixture import write_export
from test_gpu_loader import CONFIG
from test_gpu_torso_model import _model, _oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
pytestmark = [pytest.mark.gpu, pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")]
TEMPERATURE = {"choice": 1.0, "noul": 1.0, "score": 0.5}  # the config napi_decider.js passes


@pytest.fixture(scope="module")
def run(tmp_path_factory):
    from safetensors.numpy import save_file
    tmp_path = tmp_path_factory.mktemp("decider")
    W, V, M = _model(seed=31)
    Vall = dict(V)
    for i, k, x in M:
        Vall["layers.%d.%s" % (i, k)] = x
    exp, work = str(tmp_path / "export"), str(tmp_path / "work")
    os.makedirs(work)
    write_export(exp, CONFIG, W, Vall)
    rng = np.random.default_rng(1)
    d, e = 2048, 64
    head = {"norm.weight": 1 + 0.1 * rng.normal(size=d), "norm.bias": 0.1 * rng.normal(size=d),
            "q.weight": rng.normal(size=(e, d)) / np.sqrt(d), "q.bias": 0.1 * rng.normal(size=e),
            "k.weight": rng.normal(size=(e, d)) / np.sqrt(d), "k.bias": 0.1 * rng.normal(size=e)}
    head = {k: v.astype(np.float32) for k, v in head.items()}
    save_file(head, os.path.join(work, "head.safetensors"))
    cases = {"state": "Help! My payouts have been failing for 3 days!",
             "questions": {"team": {"type": "choice", "instructions": "Which team should handle this?",
                                    "options": ["billing", "sales", "retail"]},
                           "urgent": {"type": "noul", "instructions": "Does this convey urgency?"},
                           "mood": {"type": "score", "instructions": "How frustrated is the writer?",
                                    "options": ["calm", "frustrated", "depressed"]}},
             "states": ["state two", "state three", "state four", "state five"]}
    with open(os.path.join(work, "cases.json"), "w") as f:
        json.dump(cases, f)
    print("decider: %d questions, %d more states" % (len(cases["questions"]), len(cases["states"])), flush=True)
    r = subprocess.run([shutil.which("node"), os.path.join(ROOT, "tests", "js", "napi_decider.js"), exp, work],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1]), cases, (W, V, M), head


def _head_fp64(head, hid, temperature):
    """head.js in fp64: rows [options..., answer] of final-normed hidden states -> logits, probabilities."""
    H = {k: v.astype(np.float64) for k, v in head.items()}

    def proj(name, x):
        xn = (x - x.mean()) / np.sqrt(x.var() + 1e-5) * H["norm.weight"] + H["norm.bias"]
        return H[name + ".weight"] @ xn + H[name + ".bias"]

    q = proj("q", hid[-1])
    lg = np.array([proj("k", h) @ q for h in hid[:-1]]) / np.sqrt(len(q)) / temperature
    p = np.exp(lg - lg.max())
    return lg, p / p.sum()


def test_decide_matches_the_oracle_composition(run):
    out, cases, (W, V, M), head = run
    deq = {}
    for name, q in cases["questions"].items():
        s = out["single"][name]
        ids = np.array(s["ids"], np.uint32)
        rows = s["optIdx"] + [len(ids) - 1]
        print("oracle: %s, %d prompt tokens, rows %s" % (name, len(ids), rows), flush=True)
        hid = _oracle(W, V, M, ids, rows, deq)
        lg, p = _head_fp64(head, hid, TEMPERATURE[q["type"]])
        got_p = np.array([s["answer"]["probabilities"][l] for l in
                          (["false", "true"] if q["type"] == "noul" else
                           q["options"] if q["type"] == "choice" else [str(i) for i in range(len(q["options"]))])])
        dl = np.abs(np.array(s["logits"]) - lg).max()
        dp = np.abs(got_p - p).max()
        print("  logits %s vs oracle %s: max |d| %.2e; probabilities max |d| %.2e" % (
            np.round(s["logits"], 4), np.round(lg, 4), dl, dp))
        # the hidden rows carry f16 storage steps (about 1e-3 relative); through the head that is a few 1e-3
        assert dl < 0.02 * max(1.0, np.abs(lg).max()), (name, s["logits"], lg)
        assert dp < 5e-3, (name, got_p, p)


def test_decide_many_matches_single_and_cache_policy(run):
    out, cases, _, _ = run
    for name in cases["questions"]:
        a, b = out["many"][name], out["single"][name]["answer"]
        assert out["single"][name]["cached"] == 0
        assert a["type"] == b["type"]
        for lab, p in a["probabilities"].items():
            assert abs(p - b["probabilities"][lab]) < 2e-3, (name, lab, p, b["probabilities"][lab])
        print(name, a)
    assert out["again_cached"] > 0          # the state was cached by decideMany: only the suffix ran
    assert out["released"] == 1 and out["cache_size"] == 4  # a fifth state evicted the least recently used
