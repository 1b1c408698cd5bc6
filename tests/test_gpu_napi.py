"""The Node host path on the GPU: tests/js/napi_forward.js drives engine.js -> ha_napi.node -> libha.so through a
prefix forward with keepCache, a suffix forward resumed from the snapshot, and release() (engine.js:313-375 usage).
Its outputs must equal, bit for bit, the same calls made through the C ABI from Python on the same inputs (same
kernels, same order), and the prefix must match the CPU oracle within the north-star tolerances."""
import json
import os
import shutil
import subprocess
import sys

import numpy as np
import pytest

import hybrid_attention as ha
import synth
from harness import Runner, oracle_gdn, oracle_gqa, rel_err

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")]
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KINDS = ["linear_attention", "full_attention"]
B, T0, T1 = 2, 100, 40


def _inputs(T, part):
    return [synth.gdn_rows(T, B, seed=5, layer=0, part=part).astype(np.float32),
            synth.gqa_rows(T, B, seed=5, layer=1, part=part).astype(np.float16)]


def _params():
    return [synth.gdn_params(seed=5, layer=0), synth.gqa_params(seed=5, layer=1, noise=0.1)]


@pytest.mark.parametrize("rec", [ha.CHUNKED, ha.CHUNKED_PAIRED], ids=["default-split", "paired"])
def test_node_forward_resume_release(tmp_path, rec):
    d = str(tmp_path)
    params = _params()
    # the same recurrence in both hosts, while this process is alive and has run that form itself: the engine's
    # default for B * H = 32 (the split form) and the paired form (the default from B * H = 48 on, the form of the
    # B = 8 stack)
    spec = {"kinds": KINDS, "batch": B, "maxCtx": 4096, "T0": T0, "T1": T1, "params": [], "recurrence": rec}
    for i, p in enumerate(params):
        names = {}
        for k, v in p.items():
            f = "p_%d_%s.bin" % (i, k)
            np.ascontiguousarray(v, dtype=np.float32).tofile(os.path.join(d, f))
            names[k] = f
        spec["params"].append(names)
    ins = {0: _inputs(T0, 0), 1: _inputs(T1, 1)}
    for part, xs in ins.items():
        for i, x in enumerate(xs):
            x.tofile(os.path.join(d, "in_%d_%d.bin" % (i, part)))
    with open(os.path.join(d, "spec.json"), "w") as f:
        json.dump(spec, f)
    print("node forward: B=%d T0=%d T1=%d" % (B, T0, T1), flush=True)
    r = subprocess.run([shutil.which("node"), os.path.join(ROOT, "tests", "js", "napi_forward.js"), d],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert json.loads(r.stdout.strip().splitlines()[-1])["ok"]

    def js_out(i, part, T):
        dt = np.float32 if i == 0 else np.float16
        return np.fromfile(os.path.join(d, "out_%d_%d.bin" % (i, part)), dtype=dt).reshape(B, T, 2048).astype(np.float32)

    run = Runner(KINDS, batch=B)
    for i, p in enumerate(params):
        run.set_params(i, p)
    out0, snap = run.forward(ins[0], keep=True, recurrence=rec)
    out1, _ = run.forward(ins[1], cache=snap, recurrence=rec)
    for i in range(2):
        assert np.array_equal(js_out(i, 0, T0), out0[i]), "prefix layer %d differs from the C ABI run" % i
        assert np.array_equal(js_out(i, 1, T1), out1[i]), "suffix layer %d differs from the C ABI run" % i
    st = np.zeros((B, 16, 128, 128), np.float32)
    snap.read(0, "state", st)
    assert np.array_equal(np.fromfile(os.path.join(d, "state_0.bin"), dtype=np.float32).reshape(st.shape), st)

    ref_g, _ = oracle_gdn(ins[0][0], params[0], gnorm=True)
    ref_a, _ = oracle_gqa(ins[0][1], params[1], 4096)
    e_g, e_a = rel_err(js_out(0, 0, T0), ref_g), rel_err(js_out(1, 0, T0), ref_a)
    print("node prefix vs oracle: gated-delta %.2e, gqa %.2e" % (e_g, e_a))
    assert e_g < 2e-3 and e_a < 1e-2


@pytest.mark.parametrize("bits,group,asym", [(4, 32, False), (3, 64, True)])
def test_node_matmulnbits(tmp_path, bits, group, asym):
    # the MatMulNBits projection through engine.js -> ha_napi.node -> libha.so: bit-identical to the same call
    # through the C ABI from Python (the GEMV kernels at M <= 48 here, the tiled GEMM at M = 70), and within the
    # projection bar of the fp64 oracle
    import torch

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import mnb_oracle as mo

    import hybrid_attention as ha
    d = str(tmp_path)
    N, K, Ms = 1024, 2048, [1, 5, 40, 70]
    rng = np.random.default_rng(bits)
    words = rng.integers(0, 2 ** 32, (N, K // 32, bits), dtype=np.uint64).astype(np.uint32)
    sc = (0.005 + 0.01 * rng.random((N, K // group))).astype(np.float16)
    bi = ((rng.random((N, K // group)) - 0.5) * 0.1).astype(np.float16) if asym else None
    a = ((rng.random((max(Ms), K)) - 0.5) * 2).astype(np.float16)
    words.tofile(os.path.join(d, "q.bin"))
    sc.tofile(os.path.join(d, "s.bin"))
    if asym:
        bi.tofile(os.path.join(d, "b.bin"))
    a.tofile(os.path.join(d, "a.bin"))
    with open(os.path.join(d, "spec.json"), "w") as f:
        json.dump({"N": N, "K": K, "Ms": Ms, "bits": bits, "group": group, "asym": asym}, f)
    print("node matmulnbits: bits=%d group=%d asym=%d" % (bits, group, asym), flush=True)
    r = subprocess.run([shutil.which("node"), os.path.join(ROOT, "tests", "js", "napi_mnb.js"), d],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert json.loads(r.stdout.strip().splitlines()[-1])["ok"]

    dev = "cuda:0"
    qd, sd = torch.from_numpy(words.view(np.int32)).to(dev), torch.from_numpy(sc).to(dev)
    bd = torch.from_numpy(bi).to(dev) if asym else None
    w = ha.MnbWeight(N, K, qd, sd, bd, bits=bits, group=group, asym=asym)
    ad = torch.from_numpy(a).to(dev)
    W = mo.dequant(words, sc, N, K, bits, group, asym, bi)
    for M in Ms:
        y = torch.empty(M, N, dtype=torch.float16, device=dev)
        w.forward(M, ad, y)
        torch.cuda.synchronize()
        yj = np.fromfile(os.path.join(d, "y_%d.bin" % M), dtype=np.float16).reshape(M, N)
        assert np.array_equal(yj, y.cpu().numpy()), "M=%d differs from the C ABI call" % M
        assert mo.rel_err(yj.astype(np.float64), mo.matmul(a[:M], W)) < 2e-3
    w.close()
    fj = np.fromfile(os.path.join(d, "fwht.bin"), dtype=np.float16).astype(np.float64)
    assert mo.rel_err(fj, mo.fwht(a[0, :64].astype(np.float64), 64)) < 2e-3
