#!/usr/bin/env python3
"""Benchmark of the hybrid-attention hot path on one MI355X.

Headline metric: ms per forward of the 24-layer hybrid attention stack (18 gated-delta + 6 gated
GQA layers in the 3:1 pattern) at T = 2048 for a batch of B = 8 independent sequences (the benchmark's B=8, T=2048 configuration,
projections excluded, synthetic post-projection rows ~N(0,1) already resident in HBM). One "step" is one such
forward: every layer in stack order on one stream.

Also reported, on the same line:
  roofline      the chunked gated-delta kernel (the dominant one): algorithmic HBM bytes per launch / the kernel's
                time (median of 30 launches, HIP events on the launch stream around it), against 8 TB/s
  roofline_gqa  the GQA layer's two kernels: algorithmic MFMA flops / their time (measured the same way), against
                2.5 PFLOP/s dense f16
  sweep         the stack at T = 8, 128, 512 (B = 8) and at T = 2048 with B = 1
  cpu_baseline  a PyTorch CPU fp32 restatement of the same layers (oracle/torch_cpu.py: chunk-64 gated-delta,
                F.conv1d(groups=C), explicit masked-softmax GQA) on the host cores, one full B=8, T=2048 layer of
                each kind on the same PCG64 inputs as the GPU stack, scaled by the layer counts (18, 6)
  projections   the MatMulNBits projections either side of the path: per-forward time at M = 1 (HBM roofline)
                and M = 2048 (MFMA roofline), with their own CPU baseline (the numpy oracle)
  torso         ms per whole torso forward (embedding to final norm, the reference torso's layer counts) at
                8 / 68 / 512 / 2048 tokens, next to the reference's published M4 Pro times per forward
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "strands-decider-web_amd"))

KINDS = (["linear_attention"] * 3 + ["full_attention"]) * 6
H, DK, DV, STRIDE_LIN, HQ, HK, HD, STRIDE_FULL = 16, 128, 128, 8256, 8, 2, 256, 5120
LIN_W = 2 * H * DK + H * DV + H * DV + 2 * H


def gdn_bytes_per_token(esz=4, gnorm=True):
    """Algorithmic HBM bytes per token of one gated-delta layer: qkv + a/b rows in, z (gated norm) in, out."""
    return (2 * H * DK + H * DV) * esz + 2 * H * esz + (H * DV * esz if gnorm else 0) + H * DV * esz


def gqa_flops(T, P=0):
    """4 * HQ * HD * (T(T+1)/2 + P T): QK^T and PV over the unmasked (causal) pairs."""
    return 4 * HQ * HD * (T * (T + 1) // 2 + P * T)


COPY_BYTES = 512 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gdn_duo_B8_T2048_hbm_traffic.md")
GDN_SOURCE = os.path.join(ROOT, "strands-decider-web_amd", "csrc", "gdn_duo.hip")


def measured_traffic():
    """HBM bytes per launch of the gated-delta kernel from the committed rocprofv3 --pmc summary (FETCH_SIZE and
    WRITE_SIZE per dispatch, each scaled by the same counter's reading for a copy kernel of known size), used only
    if that summary was taken on the kernel source that is built now; otherwise None."""
    import hashlib
    try:
        with open(TRAFFIC_FILE) as f:
            text = f.read()
        with open(GDN_SOURCE, "rb") as f:
            sha = hashlib.sha256(f.read()).hexdigest()
    except OSError:
        return None
    vals = {}
    for line in text.splitlines():
        line = line.strip().lstrip("-* ")
        if ":" in line and line.startswith(("traffic_bytes_per_launch", "kernel_source_sha256")):
            k, v = line.split(":", 1)
            vals[k.strip()] = v.strip().strip("` ")
    if vals.get("kernel_source_sha256") != sha:
        return None
    try:
        return int(vals["traffic_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def make_engine(ha, kinds, B, max_ctx, stream):
    import synth
    eng = ha.Engine(ha.model_config(kinds, batch=B, max_ctx=max_ctx, lin_dtype=ha.F32, full_dtype=ha.F16),
                    device=0, stream=stream)
    for i, k in enumerate(kinds):
        ps = synth.gdn_params(seed=0, layer=i) if k == "linear_attention" else synth.gqa_params(seed=0, layer=i)
        for n, v in ps.items():
            eng.set_param(i, n, v)
    return eng


def host_inputs(B, T, seed=0):
    """One post-projection input per layer kind, NumPy PCG64 (synth.py, one stream per tensor): the rows every layer
    of that kind reads in the headline stack, and the rows the CPU baseline runs on."""
    import synth
    return {"linear_attention": synth.gdn_rows(T, B, seed=seed), "full_attention": synth.gqa_rows(T, B, seed=seed)}


def make_buffers(torch, kinds, B, T, seed=0, host=None):
    """Device inputs and outputs for one forward. With `host` (host_inputs()), each kind's rows are uploaded once
    and shared by all layers of that kind; otherwise every layer gets its own rows from torch's GPU generator."""
    g = torch.Generator(device="cuda:0")
    g.manual_seed(seed)
    ins, outs = [], []
    shared = {}
    if host is not None:
        shared = {"linear_attention": torch.from_numpy(host["linear_attention"]).to("cuda:0"),
                  "full_attention": torch.from_numpy(host["full_attention"]).to("cuda:0")}
    for k in kinds:
        if k in shared:
            ins.append(shared[k])
            outs.append(torch.empty(B, T, H * DV if k == "linear_attention" else HQ * HD, device="cuda:0",
                                    dtype=torch.float32 if k == "linear_attention" else torch.float16))
            continue
        if k == "linear_attention":
            x = torch.zeros(B, T, STRIDE_LIN, device="cuda:0", dtype=torch.float32)
            x[:, :, :LIN_W] = torch.randn(B, T, LIN_W, device="cuda:0", generator=g)
            outs.append(torch.empty(B, T, H * DV, device="cuda:0", dtype=torch.float32))
        else:
            x = torch.randn(B, T, STRIDE_FULL, device="cuda:0", generator=g).to(torch.float16)
            outs.append(torch.empty(B, T, HQ * HD, device="cuda:0", dtype=torch.float16))
        ins.append(x)
    return ins, outs


def time_forwards(torch, eng, T, ins, outs, steps, warmup, stream):
    for _ in range(warmup):
        eng.forward(T, ins, outs)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        eng.forward(T, ins, outs)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return wall, e0.elapsed_time(e1) / steps


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(host, B=8, T=2048, reps=3):
    """PyTorch CPU fp32 restatement (oracle/torch_cpu.py) of one gated-delta and one GQA layer over the whole
    B x T workload, on the same PCG64 rows the GPU stack reads; warm-up 1, median of `reps`, scaled by the layer
    counts (18, 6). Threads: the host cores this process may use (OMP_NUM_THREADS caps it, as on the GPU box)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import torch

    import synth
    import torch_cpu
    cores = len(os.sched_getaffinity(0))
    threads = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))
    torch.set_num_threads(threads)
    x = torch.from_numpy(host["linear_attention"])
    p = {k: torch.from_numpy(v) for k, v in synth.gdn_params(seed=0, layer=0).items()}
    xa = torch.from_numpy(host["full_attention"])
    pa = {k: torch.from_numpy(v) for k, v in synth.gqa_params(seed=0, layer=3).items()}
    cos, sin = torch_cpu.rope_table(T)
    tg, ta = [], []
    with torch.no_grad():
        for r in range(reps + 1):
            t0 = time.perf_counter()
            torch_cpu.gdn_layer(x, p["conv"], p["neg_exp_A"], p["dt_bias"], p["gnorm"])
            t1 = time.perf_counter()
            torch_cpu.gqa_layer(xa, pa["q_norm"], pa["k_norm"], cos, sin)
            t2 = time.perf_counter()
            if r:
                tg.append(t1 - t0)
                ta.append(t2 - t1)
    tg, ta = sorted(tg)[len(tg) // 2], sorted(ta)[len(ta) // 2]
    ms = (18 * tg + 6 * ta) * 1e3
    return {"value": round(ms, 1), "unit": "ms", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "torch_threads": torch.get_num_threads(), "host_cores_visible": cores,
            "tokens_per_s": round(B * T / (ms * 1e-3)),
            "sample": "PyTorch %s CPU fp32 (oracle/torch_cpu.py): one gated-delta layer (chunk-64 WY form, "
                      "F.conv1d(groups=C), gated RMSNorm) and one GQA layer (explicit masked softmax), each over "
                      "the whole B=%d, T=%d workload on the GPU stack's PCG64 rows; warm-up 1, median of %d; "
                      "per layer %.0f / %.0f ms; scaled x (18, 6) layers" % (torch.__version__, B, T, reps,
                                                                           tg * 1e3, ta * 1e3)}


def decode_measure(torch, ha, stream, steps=50, P=1536):
    """Decode and resume from a prefix cache: a P-row prefix through the engine (chunked prefill) kept as a snapshot,
    then calls of L new rows resumed from it, each timed alone (HIP events on the engine's stream around one call,
    median over `steps`).
      gdn_seq   one gated-delta layer, L = 1 and 8 rows, HA_SEQUENTIAL, B = 1 and 8: GB/s against the algorithmic
                bytes (fp32 state in and out, 64 KiB each per head, plus the rows read and written)
      stack     the 24-layer stack at B = 1 and 8, L = 1 (sequential recurrence for the gated-delta layers)
      resume    the prefix-cache case: 3 gated-delta + 1 GQA layers, one 64-row suffix at P = 1536 (B = 1, default
                recurrence), with and without keeping a snapshot of the result"""
    import numpy as np
    res = {}

    def timed(fn):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ts = []
        for i in range(steps + 3):
            e0.record(stream)
            fn()
            e1.record(stream)
            e1.synchronize()
            if i >= 3:
                ts.append(e0.elapsed_time(e1))
        return float(np.median(ts))

    for B in (1, 8):
        eng = make_engine(ha, ["linear_attention"], B, 4096, stream.cuda_stream)
        pi, po = make_buffers(torch, ["linear_attention"], B, P, seed=7)
        snap = eng.forward(P, pi, po, keep_cache=True)["cache"]
        for L in (1, 8):
            si, so = make_buffers(torch, ["linear_attention"], B, L, seed=8)
            ms = timed(lambda: eng.forward(L, si, so, cache=snap, recurrence=ha.SEQUENTIAL))
            byt = B * (2 * H * DK * DV * 4 + L * gdn_bytes_per_token())
            res["gdn_seq_B%d_L%d" % (B, L)] = {"us": round(ms * 1e3, 2), "GB_per_s": round(byt / (ms * 1e-3) / 1e9, 1),
                                               "bytes": byt, "frac": round(byt / (ms * 1e-3) / 8e12, 4)}
            del si, so
        snap.release()
        del eng, pi, po
        es = make_engine(ha, KINDS, B, 4096, stream.cuda_stream)
        pi, po = make_buffers(torch, KINDS, B, P, seed=9)
        snap = es.forward(P, pi, po, keep_cache=True)["cache"]
        si, so = make_buffers(torch, KINDS, B, 1, seed=10)
        ms = timed(lambda: es.forward(1, si, so, cache=snap, recurrence=ha.SEQUENTIAL))
        res["stack_B%d_L1" % B] = {"ms": round(ms, 4), "tokens_per_s": round(B / (ms * 1e-3))}
        snap.release()
        del es, pi, po, si, so
        torch.cuda.empty_cache()
    kinds = ["linear_attention", "linear_attention", "linear_attention", "full_attention"]
    er = make_engine(ha, kinds, 1, 4096, stream.cuda_stream)
    pi, po = make_buffers(torch, kinds, 1, P, seed=11)
    snap = er.forward(P, pi, po, keep_cache=True)["cache"]
    si, so = make_buffers(torch, kinds, 1, 64, seed=12)
    res["resume_P1536_L64"] = {"ms": round(timed(lambda: er.forward(64, si, so, cache=snap)), 4)}
    kept = []

    def with_keep():
        kept.append(er.forward(64, si, so, cache=snap, keep_cache=True)["cache"])

    res["resume_P1536_L64_keep"] = {"ms": round(timed(with_keep), 4)}
    for k in kept:
        k.release()
    snap.release()
    res["workload"] = ("resume from a %d-row prefix snapshot: gated-delta decode steps (HA_SEQUENTIAL), the 24-layer "
                       "stack at L = 1, and the prefix-cache case (3 gated-delta + 1 GQA, 64-row suffix)" % P)
    return res


# The model's int4 projection shapes (K, N) and how many of each one forward runs, as the reference's matmul
# benchmark weighs them (web/public/gemmbench/portable.js:18 and :69).
MNB_SHAPES = [(2048, 12288, 15), (6144, 2048, 15), (2048, 8256, 11), (2048, 5120, 4), (2048, 2048, 16)]
MNB_MS = (1, 2048)  # decode (one token) and one 2048-token prefill, the reference's default M ends


def mnb_weights(torch, N, K, seed):
    """Random packed int4 blocks and scales 0.005..0.015 (portable.js:29-30), on the GPU."""
    import numpy as np
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 2 ** 32, (N, K // 32, 4), dtype=np.uint64).astype(np.uint32).view(np.int32)
    s = (0.005 + 0.01 * rng.random((N, K // 32))).astype(np.float16)
    return torch.from_numpy(q).to("cuda:0"), torch.from_numpy(s).to("cuda:0")


def mnb_measure(torch, ha, stream, steps=20, Ms=MNB_MS):
    """Per-forward time of the MatMulNBits projections (shape x count) at each M, from HIP events on the launch
    stream around `steps` back-to-back calls per shape; the M = 1 line against the HBM peak (packed weights + scales
    + a + y bytes), the large-M line against the dense f16 MFMA peak (2 M N K flops)."""
    out = {}
    per = {M: {"ms": 0.0, "bytes": 0, "flops": 0, "shapes": {}} for M in Ms}
    for i, (K, N, cnt) in enumerate(MNB_SHAPES):
        q, s = mnb_weights(torch, N, K, seed=i)
        w = ha.MnbWeight(N, K, q, s, None)
        for M in Ms:
            a = torch.randn(M, K, device="cuda:0").to(torch.float16)
            y = torch.empty(M, N, device="cuda:0", dtype=torch.float16)
            for _ in range(3):
                w.forward(M, a, y, stream.cuda_stream)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(steps):
                w.forward(M, a, y, stream.cuda_stream)
            e1.record(stream)
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / steps
            p = per[M]
            p["ms"] += cnt * ms
            p["bytes"] += cnt * (N * K // 2 + N * K // 32 * 2 + 2 * M * K + 2 * M * N)
            p["flops"] += cnt * 2 * M * N * K
            p["shapes"]["%dx%d" % (N, K)] = round(ms * 1e3, 2)
            del a, y
        w.close()
        del q, s
        torch.cuda.empty_cache()
    for M, p in per.items():
        d = {"ms_per_forward": round(p["ms"], 4), "us_per_call": p["shapes"]}
        if M == 1:
            gbs = p["bytes"] / (p["ms"] * 1e-3) / 1e9
            d["roofline"] = {"bound": "hbm", "kernel": "mnb_gemv_lanes_kernel", "achieved": round(gbs, 1),
                             "peak": 8000.0, "unit": "GB/s", "frac": round(gbs / 8000.0, 4),
                             "bytes_per_forward": p["bytes"], "traffic": None}
        else:
            tf = p["flops"] / (p["ms"] * 1e-3) / 1e12
            d["roofline"] = {"bound": "mfma", "kernel": "mnb_gemm_kernel",
                             "achieved": round(tf, 1), "peak": 2500.0, "unit": "TFLOP/s",
                             "frac": round(tf / 2500.0, 4), "flops_per_forward": p["flops"], "traffic": None}
        out["M%d" % M] = d
    return out


def mnb_cpu_baseline():
    """The numpy oracle (oracle/mnb_oracle.py: dequantise in fp64, then the product) at M = 1 on each shape once,
    scaled by the per-forward counts."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import mnb_oracle as mo
    tot = 0.0
    for i, (K, N, cnt) in enumerate(MNB_SHAPES):
        rng = np.random.default_rng(i)
        words = rng.integers(0, 2 ** 32, (N, K // 32, 4), dtype=np.uint64).astype(np.uint32)
        sc = (0.005 + 0.01 * rng.random((N, K // 32))).astype(np.float16)
        a = ((rng.random((1, K)) - 0.5) * 2).astype(np.float16)
        t0 = time.perf_counter()
        mo.matmul(a, mo.dequant(words, sc, N, K))
        tot += cnt * (time.perf_counter() - t0)
    return {"value": round(tot * 1e3, 1), "unit": "ms per forward's projections at M=1", "cores": 1, "kind": "port",
            "sample": "numpy oracle (fp64 dequantise + product) at M=1, each of the 5 shapes once, x per-forward "
                      "counts"}


# The reference's own torso (web/public/gemmbench/portable.js:69 counts its matmuls per forward: 11 in_proj, 4 qkv,
# 15 MLPs, 16 2048 x 2048 projections): 11 gated-delta, 4 GQA and 1 adapter layer. The order is not published and
# does not change the work.
REF_TORSO = (["linear_attention"] * 3 + ["full_attention"]) * 3 + ["linear_attention"] * 2 + ["adapter"] + \
    ["full_attention"]
# README.md:90-91, M4 Pro GPU time per forward; at 8 tokens the raw forward latency of README.md:33-37 (the fastest
# engine row), the only published figure at that length
REF_TORSO_MS = {8: 12.8, 68: 29.0, 512: 161.0, 2048: 646.0}


def torso_measure(torch, ha, Ls=(8, 68, 512, 2048), steps=5, types=REF_TORSO, vocab=4096):
    """ms per whole torso forward (embedding, every layer's norms, projections, token mixer and MLP, final norm of
    the last row) through hybrid_attention.Torso, batch 1, random int4 weights (scales as portable.js:29-30) and
    synthetic mixer parameters, HIP events on the torso's stream around `steps` forwards after one warm-up."""
    import numpy as np

    import synth
    D, I = 2048, 6144
    t = ha.Torso(types, D=D, I=I)
    g = torch.Generator(device="cuda:0")
    g.manual_seed(0)

    def quant(N, K):
        q = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K // 32, 4), dtype=torch.int32, device="cuda:0", generator=g)
        s = (0.004 + 0.002 * torch.rand(N, K // 32, device="cuda:0", generator=g)).to(torch.float16)
        return ha.MnbWeight(N, K, q, s, None)

    rng = np.random.default_rng(0)
    vec = lambda: (1 + 0.1 * rng.normal(size=D)).astype(np.float32)  # noqa: E731
    t.set_weight("embed", quant(vocab, D))
    t.set_param("final_norm", vec())
    for i, k in enumerate(types):
        p = "layers.%d." % i
        t.set_param(p + "in_norm", vec())
        if k == "adapter":
            t.set_weight(p + "proj", quant(D, D))
            t.set_param(p + "bias", (0.05 * rng.normal(size=D)).astype(np.float32))
            continue
        lin = k == "linear_attention"
        t.set_weight(p + ("in_proj" if lin else "qkv"), quant(8256 if lin else 5120, D))
        t.set_weight(p + ("out_proj" if lin else "o_proj"), quant(D, 2048))
        t.set_param(p + "post_norm", vec())
        t.set_weight(p + "gate_up", quant(2 * I, D))
        t.set_weight(p + "down", quant(D, I))
        ps = synth.gdn_params(seed=0, layer=i) if lin else synth.gqa_params(seed=0, layer=i, noise=0.1)
        for n, v in ps.items():
            t.set_param(p + n, v)
    res = {}
    for L in Ls:
        ids = rng.integers(0, vocab, L)
        t.forward(ids, [L - 1])
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(t.stream)
        for _ in range(steps):
            t.forward(ids, [L - 1])
        e1.record(t.stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        res["L%d" % L] = {"ms": round(ms, 3), "tokens_per_s": round(L / (ms * 1e-3)),
                          "reference_m4pro_ms": REF_TORSO_MS.get(L)}
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-sweep", action="store_true", help="skip the T / B sweep")
    ap.add_argument("--no-mnb", action="store_true", help="skip the MatMulNBits projection measurement")
    ap.add_argument("--no-torso", action="store_true", help="skip the whole-torso forward measurement")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode / resume measurement")
    ap.add_argument("--profile-kernel", choices=["gdn", "gdn-seq", "gqa", "copy", "mnb", "torso", "decode"],
                    help="run only one layer kind (T=2048, B=--profile-batch) --steps times, for rocprofv3; 'copy' runs a plain "
                         "512 MiB device-to-device copy kernel, the reference point that scales FETCH_SIZE / "
                         "WRITE_SIZE to bytes")
    ap.add_argument("--profile-batch", type=int, default=8, help="batch size for --profile-kernel gdn / gqa")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the hybrid-attention path is benchmarked on a single GPU in this build "
              "(multi-GPU sharding is a design note only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    import hybrid_attention as ha
    ha.load_library()
    stream = torch.cuda.Stream()
    B, T = 8, 2048
    if args.profile_kernel == "copy":
        with torch.cuda.stream(stream):
            src = torch.ones(COPY_BYTES // 4, device="cuda:0", dtype=torch.float32)
            dst = torch.empty_like(src)
            for _ in range(args.warmup):
                dst.copy_(src)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(args.steps):
                dst.copy_(src)
            torch.cuda.synchronize()
        print(json.dumps({"profile_kernel": "copy", "bytes_read": COPY_BYTES, "bytes_written": COPY_BYTES,
                          "ms_per_launch": (time.perf_counter() - t0) * 1e3 / args.steps}), flush=True)
        return
    if args.profile_kernel == "torso":
        t0 = time.perf_counter()
        res = torso_measure(torch, ha, Ls=(2048,), steps=args.steps)
        print(json.dumps({"profile_kernel": "torso", "steps": args.steps, "result": res,
                          "wall_s": round(time.perf_counter() - t0, 2)}), flush=True)
        return
    if args.profile_kernel == "decode":
        with torch.cuda.stream(stream):
            res = decode_measure(torch, ha, stream, steps=args.steps)
        print(json.dumps({"profile_kernel": "decode", "steps": args.steps, "result": res}), flush=True)
        return
    if args.profile_kernel == "mnb":
        t0 = time.perf_counter()
        res = mnb_measure(torch, ha, stream, steps=args.steps)
        print(json.dumps({"profile_kernel": "mnb", "steps": args.steps, "result": res,
                          "wall_s": round(time.perf_counter() - t0, 2)}), flush=True)
        return
    if args.profile_kernel in ("gdn", "gqa"):
        # exactly the bench line's roofline leg (same engine and seeds): --warmup forwards, then --steps forwards
        # back to back timed by HIP events on the launch stream; a kernel trace of this command covers those launches
        kind = "full_attention" if args.profile_kernel == "gqa" else "linear_attention"
        B = args.profile_batch
        with torch.cuda.stream(stream):
            e = make_engine(ha, [kind], B, 4096, stream.cuda_stream)
            i, o = make_buffers(torch, [kind], B, T, seed=1 if kind == "linear_attention" else 2)
            _, ms = time_forwards(torch, e, T, i, o, args.steps, args.warmup, stream)
        print(json.dumps({"profile_kernel": args.profile_kernel, "B": B, "T": T, "warmup": args.warmup,
                          "steps": args.steps, "ms_per_launch": round(ms, 5)}), flush=True)
        return
    if args.profile_kernel:
        kind = "linear_attention"
        rec = ha.SEQUENTIAL
        B = args.profile_batch
        with torch.cuda.stream(stream):
            e = make_engine(ha, [kind], B, 4096, stream.cuda_stream)
            i, o = make_buffers(torch, [kind], B, T)
            for _ in range(args.warmup):
                e.forward(T, i, o, recurrence=rec)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(args.steps):
                e.forward(T, i, o, recurrence=rec)
            torch.cuda.synchronize()
        print(json.dumps({"profile_kernel": args.profile_kernel, "B": B, "T": T, "steps": args.steps,
                          "ms_per_launch": (time.perf_counter() - t0) * 1e3 / args.steps}), flush=True)
        return
    host = host_inputs(B, T)
    with torch.cuda.stream(stream):
        eng = make_engine(ha, KINDS, B, 4096, stream.cuda_stream)
        ins, outs = make_buffers(torch, KINDS, B, T, host=host)
        torch.cuda.synchronize()
        wall_ms, ev_ms = time_forwards(torch, eng, T, ins, outs, args.steps, args.warmup, stream)
        res = eng.forward(T, ins, outs, timestamps=True, layer_ms=True)
        lms = res["layer_ms"]
        gdn_ms = sum(m for m, k in zip(lms, KINDS) if k == "linear_attention")
        gqa_ms = sum(m for m, k in zip(lms, KINDS) if k == "full_attention")
        del ins, outs
        torch.cuda.empty_cache()

        # dominant kernel: the gated-delta kernel of one layer (the paired form at this shape), timed alone on its
        # stream
        e1 = make_engine(ha, ["linear_attention"], B, 4096, stream.cuda_stream)
        i1, o1 = make_buffers(torch, ["linear_attention"], B, T, seed=1)
        _, gdn_launch_ms = time_forwards(torch, e1, T, i1, o1, 30, 3, stream)
        gdn_bytes = B * T * gdn_bytes_per_token() + B * H * DK * DV * 4  # + final state write
        achieved = gdn_bytes / (gdn_launch_ms * 1e-3) / 1e9
        del e1, i1, o1
        # GQA layer (K/V prep + attention kernels) against the dense f16 MFMA peak
        e2 = make_engine(ha, ["full_attention"], B, 4096, stream.cuda_stream)
        i2, o2 = make_buffers(torch, ["full_attention"], B, T, seed=2)
        _, gqa_launch_ms = time_forwards(torch, e2, T, i2, o2, 30, 3, stream)
        gqa_tf = B * gqa_flops(T) / (gqa_launch_ms * 1e-3) / 1e12
        del e2, i2, o2
        torch.cuda.empty_cache()

        sweep = {}
        if not args.no_sweep:
            for (bb, tt) in [(8, 8), (8, 128), (8, 512), (1, 2048)]:
                es = make_engine(ha, KINDS, bb, 4096, stream.cuda_stream)
                si, so = make_buffers(torch, KINDS, bb, tt, seed=3)
                _, ms = time_forwards(torch, es, tt, si, so, max(5, args.steps // 2), 2, stream)
                sweep["B%d_T%d" % (bb, tt)] = {"ms": round(ms, 4), "tokens_per_s": round(bb * tt / (ms * 1e-3))}
                del es, si, so
                torch.cuda.empty_cache()

    line = {
        "metric": "ms/forward of hybrid attention stack at T=2048; HBM GB/s and MFMA util %",
        "value": round(wall_ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "gpu_event_ms_per_step": round(ev_ms, 4),
        "tokens_per_s": round(B * T / (wall_ms * 1e-3)),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 recurrence state + f16 MFMA operands (f32 accumulate); gated-delta rows f32, GQA rows f16",
        "data": "synthetic: post-projection rows ~N(0,1) (NumPy PCG64, one input per layer kind shared by that "
                "kind's layers), conv taps ~N(0,0.5^2), unit q/k norm gain",
        "config": {"workload": "24-layer hybrid stack (18 gated-delta + 6 GQA, 3:1), "
                               "B=8 sequences, T=2048, projections excluded",
                   "batch": B, "seq_len": T, "layers": len(KINDS),
                   "gdn_recurrence": "chunked, paired form (32-row chunks, 2 workgroups per sequence-head)"},
        "per_kind_ms": {"gated_delta_18": round(gdn_ms, 4), "gqa_6": round(gqa_ms, 4)},
        "roofline": {"bound": "hbm", "kernel": "gdn_duo_kernel",
                     "achieved": round(achieved, 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(achieved / 8000.0, 4), "traffic": measured_traffic(),
                     "bytes_per_launch": gdn_bytes, "bytes_per_token": gdn_bytes_per_token(),
                     "launch_ms": round(gdn_launch_ms, 5),
                     "timing": "30 back-to-back one-layer forwards after 3 warm-up, HIP events on the launch stream; "
                               "includes the layer's 3-row tail copy kernel (about 2% of it)"},
        "roofline_gqa": {"bound": "mfma", "kernel": "gqa_kv_kernel + gqa_attn_kernel",
                         "achieved": round(gqa_tf, 1), "peak": 2500.0, "unit": "TFLOP/s",
                         "frac": round(gqa_tf / 2500.0, 4), "flops_per_launch": B * gqa_flops(T),
                         "launch_ms": round(gqa_launch_ms, 5),
                         "timing": "30 back-to-back one-layer forwards after 3 warm-up, HIP events on the launch "
                                   "stream"},
        "sweep": sweep,
    }
    if not args.no_decode:
        with torch.cuda.stream(stream):
            line["decode"] = decode_measure(torch, ha, stream)
    if not args.no_mnb:
        line["projections"] = mnb_measure(torch, ha, stream)
        line["projections"]["workload"] = ("MatMulNBits int4 group-32 projections of one forward, shapes x counts of "
                                           "web/public/gemmbench/portable.js:18,69, random weights")
    if not args.no_torso:
        line["torso"] = torso_measure(torch, ha)
        line["torso"]["workload"] = ("whole torso forward, batch 1: embedding, 11 gated-delta + 4 GQA + 1 adapter "
                                     "layers (the reference torso's counts) with norms, int4 projections and MLPs, "
                                     "final norm of the last row; random weights")
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(host, B, T)
        if "projections" in line:
            line["projections"]["cpu_baseline"] = mnb_cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
