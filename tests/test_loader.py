"""The Node loader's wire-format decoder (strands-decider-web_amd/js/loader.js decodeScales, the 8-bit log-coded
scales of web/public/engine/wire.js:1-46) against the decode formula restated in numpy
(tests/export_fixture.decode_scales: f64 product, rounded to f32 then f16), on the CPU."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from export_fixture import decode_scales, encode_scales

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which("node")
pytestmark = pytest.mark.skipif(NODE is None or not os.path.exists(
    os.path.join(ROOT, "strands-decider-web_amd", "js", "ha_napi.node")), reason="node or the built addon is missing")


def test_wire_scale_decoder_matches_the_formula(tmp_path):
    rng = np.random.default_rng(0)
    N, G = 64, 64
    sc = (rng.random((N, G)) * 0.02 * np.where(rng.random((N, G)) < 0.3, -1, 1)).astype(np.float16)
    sc[3] = 0          # an all-zero row
    sc[5, :10] = 6e-8  # f16 subnormals
    sc[7, 0] = 60000   # near the f16 maximum
    head, codes = encode_scales(sc)
    blob = np.concatenate([head, codes])
    p = os.path.join(str(tmp_path), "blob.bin")
    blob.tofile(p)
    js = ("const L = require(%r); const b = require('fs').readFileSync(%r); const d = new Uint16Array(%d);"
          "L.decodeScales(new Uint8Array(b.buffer, b.byteOffset, b.byteLength), 0, %d, %d, d, 0);"
          "console.log(JSON.stringify(Array.from(d)));") % (
        os.path.join(ROOT, "strands-decider-web_amd", "js", "loader.js"), p, N * G, N, G)
    r = subprocess.run([NODE, "-e", js], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    got = np.array(json.loads(r.stdout), np.uint16)
    want = decode_scales(head, codes, N, G).view(np.uint16).reshape(-1)
    np.testing.assert_array_equal(got, want)
    # and on rows of ordinary range the code is close to the scales it encodes (8-bit log steps; the rows made
    # extreme above span 12 decades and get coarse steps)
    dec = decode_scales(head, codes, N, G).astype(np.float64)
    ok = np.ones(N, bool)
    ok[[3, 5, 7]] = False
    ref = sc.astype(np.float64)[ok]
    nz = np.abs(ref) > 1e-6
    assert np.max(np.abs(dec[ok][nz] - ref[nz]) / np.abs(ref[nz])) < 0.05
