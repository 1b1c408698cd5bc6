"""The worker-level host (js/decider.js) on the GPU, over an export loaded by js/loader.js: decideMany (the state
encoded once, each question's suffix resumed from its snapshot, worker.js:216-236) gives the answers that separate
decide calls on the whole prompt give (within f16 storage steps: the suffix's projections see fewer rows); a decide
on a cached state runs only the suffix; the prefix cache keeps 4 states and releases the least recently used."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from export_fixture import write_export
from test_gpu_loader import CONFIG
from test_gpu_torso_model import _model

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
pytestmark = [pytest.mark.gpu, pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")]


def test_decide_many_matches_single_and_cache_policy(tmp_path):
    from safetensors.numpy import save_file
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
    save_file({k: v.astype(np.float32) for k, v in head.items()}, os.path.join(work, "head.safetensors"))
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
    out = json.loads(r.stdout.strip().splitlines()[-1])
    for name in cases["questions"]:
        a, b = out["many"][name], out["single"][name]["answer"]
        assert out["single"][name]["cached"] == 0
        assert a["type"] == b["type"]
        for lab, p in a["probabilities"].items():
            assert abs(p - b["probabilities"][lab]) < 2e-3, (name, lab, p, b["probabilities"][lab])
        print(name, a)
    assert out["again_cached"] > 0          # the state was cached by decideMany: only the suffix ran
    assert out["released"] == 1 and out["cache_size"] == 4  # a fifth state evicted the least recently used
