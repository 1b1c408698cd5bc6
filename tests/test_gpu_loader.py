"""The Node loader (strands-decider-web_amd/js/loader.js) on the GPU: an export in the reference converter's format
(convert/export_engine.py:33-40,83-85: manifest.json, 256-byte aligned tensors in shards split between tensors) of a
4-layer model at real widths, loaded and run by loadTorso, gives bit for bit what the Python Torso built from the
same arrays gives. Also for the packed "wire" form (8-bit log-coded scales, web/public/engine/wire.js:1-46; the
reference side uses the scales the code decodes to) and for a lazy embedding (bundled rows + rows fetched by byte
range on first use, engine.js:113-172) whose slots overflow between the two forwards."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from export_fixture import write_export
from test_gpu_torso_model import D, I, TYPES, VOCAB, _model, _torso

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
pytestmark = [pytest.mark.gpu, pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")]
CONFIG = {"hidden_size": D, "intermediate_size": I, "num_hidden_layers": len(TYPES), "layer_types": TYPES,
          "num_attention_heads": 8, "num_key_value_heads": 2, "head_dim": 256, "linear_num_key_heads": 16,
          "linear_key_head_dim": 128, "linear_value_head_dim": 128, "linear_conv_kernel_dim": 4,
          "rms_norm_eps": 1e-6, "vocab_size": VOCAB, "rope_theta": 10000000, "rotary_dim": 64}
ROWS = [[0, 20, 39], [0, 29]]


@pytest.mark.parametrize("form", ["plain", "wire", "lazy", "lazy-create"])
def test_loaded_export_matches_the_arrays(tmp_path, form):
    # "lazy-create": the lazy export through the async Engine.create(base, {onProgress, fetchShard}) (engine.js:63-87)
    create = form.endswith("-create")
    form = form.replace("-create", "")
    W, V, M = _model(seed=21)
    Vall = dict(V)
    for i, k, x in M:
        Vall["layers.%d.%s" % (i, k)] = x
    exp, work = str(tmp_path / "export"), str(tmp_path / "work")
    os.makedirs(work)
    lazy = {"bundled_ids": list(range(0, VOCAB, 10)), "slots": 40} if form == "lazy" else None
    scales = write_export(exp, CONFIG, W, Vall, shard_limit=24 << 20, wire=form == "wire", lazy=lazy)
    rng = np.random.default_rng(3)
    ids0, ids1 = rng.integers(0, VOCAB, 40).astype(np.uint32), rng.integers(0, VOCAB, 30).astype(np.uint32)
    ids0.tofile(os.path.join(work, "ids0.bin"))
    ids1.tofile(os.path.join(work, "ids1.bin"))
    with open(os.path.join(work, "rows.json"), "w") as f:
        json.dump(ROWS, f)
    print("loader: %s export, %d shard files" % (form, len([p for p in os.listdir(exp) if p.startswith(("weights", "wire"))])),
          flush=True)
    r = subprocess.run([shutil.which("node"), os.path.join(ROOT, "tests", "js", "napi_loader.js"), exp, work] +
                       (["create"] if create else []), capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    info = json.loads(r.stdout.strip().splitlines()[-1])
    assert info["ok"] and info["shards"] > 1
    # the projection kernel of each forward (40 and 30 rows: the packed-weight GEMV), as the reference's plan.kernel;
    # and the device guard finds nothing to object to on this GPU
    assert info["kernels"] == ["mnb_gemv", "mnb_gemv"] and info["problems"] == []
    if form == "lazy":
        assert info["evictions"] == 1  # the second forward found the 40 slots full and refilled them
    js = [np.fromfile(os.path.join(work, "hidden%d.bin" % k), np.float32).reshape(len(ROWS[k]), D) for k in (0, 1)]

    Wref = {k: (w, scales[k], N, K) for k, (w, _, N, K) in W.items()}
    t = _torso(Wref, V, M)
    py0, _ = t.forward(ids0, ROWS[0])
    py1, _ = t.forward(ids1, ROWS[1])
    assert np.array_equal(js[0], py0) and np.array_equal(js[1], py1), "loaded export differs from the arrays"
    if form == "wire":  # the wire scales are a lossy code of the originals
        assert any(not np.array_equal(scales[k], W[k][1]) for k in W)
