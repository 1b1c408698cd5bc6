"""The Node host side over the N-API addon, without a GPU: the addon builds and loads under the image's Node, the
manifest config maps to the engine config the C ABI expects, and a failing C call surfaces as a thrown Error with
the C status as its code (the reference throws Errors from Engine.create / forward, engine.js:66,316,373)."""
import json
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "strands-decider-web_amd", "js", "ha_napi.node")
NODE = shutil.which("node")

pytestmark = pytest.mark.skipif(NODE is None or not os.path.exists(ADDON), reason="node or the built addon is missing")

SCRIPT = r"""
const m = require(%r);
const out = {abi: m.abiVersion(), exports: Object.keys(m).sort()};
out.cfg = m.configFromManifest({layer_types: ['linear_attention', 'linear_attention', 'linear_attention',
  'full_attention'], linear_num_key_heads: 16, linear_key_head_dim: 128, linear_value_head_dim: 128,
  linear_conv_kernel_dim: 4, num_attention_heads: 8, num_key_value_heads: 2, head_dim: 256,
  partial_rotary_factor: 0.25, rope_theta: 10000000, rms_norm_eps: 1e-6}, {batch: 8});
try { m.configFromManifest({layer_types: ['mamba']}); } catch (e) { out.bad_kind = e.message; }
out.adapter = m.configFromManifest({layer_types: ['linear_attention', 'adapter', 'full_attention']}).layerKinds;
try { m.Engine.createSync(out.cfg, {device: 0}); out.created = true; } catch (e) { out.err = [e.code, e.message]; }
out.problems = m.engineProblems(0);
const nat = require(require('path').join(require('path').dirname(%r), 'ha_napi.node'));
try { nat.mnbForward({}, 1, BigInt(0), BigInt(0), null); } catch (e) { out.bad_handle = e.name + ': ' + e.message; }
try { new m.MatMulNBits(null, 16, 2048, BigInt(16), BigInt(16), null, {bits: 5}); } catch (e) { out.bad_shape = e.code; }
try { new m.MatMulNBits(null, 16, 2048, BigInt(16), BigInt(16), null); } catch (e) { out.no_dev = e.code; }
m.Engine.create(out.cfg).then(function () { out.async = 'resolved'; }, function (e) { out.async = e.code; })
  .then(function () { console.log(JSON.stringify(out)); });
"""


def _run():
    mod = os.path.join(ROOT, "strands-decider-web_amd", "js", "engine.js")
    js = SCRIPT % (mod, mod)
    r = subprocess.run([NODE, "-e", js], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_addon_loads_and_maps_manifest_config():
    out = _run()
    with open(os.path.join(ROOT, "include", "ha.h")) as f:
        assert "#define HA_ABI_VERSION %d\n" % out["abi"] in f.read()
    assert {"Engine", "Snapshot", "DeviceBuffer", "configFromManifest", "CHUNKED", "SEQUENTIAL", "MatMulNBits",
            "fwht", "engineProblems", "projectionKernel"} <= set(out["exports"])
    # a handle of the wrong kind is a TypeError from the addon, not a crash
    assert out["bad_handle"] == "TypeError: not a MatMulNBits handle"
    # format checks come before any device access (bits 5): HA_ERR_ARG
    assert out["bad_shape"] == "HA_1"
    c = out["cfg"]
    assert c["layerKinds"] == [0, 0, 0, 1] and c["batch"] == 8
    # the engine's fused row strides (export_engine.py:52,61): 8256 = 64-padded q|k|v|z|a|b, 5120 = q|gate|k|v
    assert c["linStride"] == 8256 and c["fullStride"] == 5120 and c["rotDim"] == 64
    assert c["ropeTheta"] == 1e7 and abs(c["eps"] - 1e-6) < 1e-12
    assert "unsupported layer type mamba" in out["bad_kind"]
    # adapter layers (engine.js:256-261) carry no token mixer: kind 2, skipped by the forward
    assert out["adapter"] == [0, 2, 1]


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is visible: creation would succeed")
def test_create_without_device_throws_with_status_code():
    out = _run()
    assert "created" not in out
    assert out["err"][0] == "HA_4" and "no HIP device" in out["err"][1]
    assert out["no_dev"] == "HA_4"  # ha_mnb_create: the device query fails without a GPU, as for the engine
    assert out["async"] == "HA_4"
    # the adapter guard's counterpart (engine.js:50-52) names the reason instead of throwing
    assert out["problems"] == ["no HIP device is visible"]
