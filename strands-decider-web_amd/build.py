"""Build the MI355X hybrid-attention library (libha.so, gfx950) and its N-API addon in-tree.

Every HIP source is compiled with hipcc for gfx950 only; packed-fp32 instruction forms are disabled
(-target-feature -packed-fp32-ops). Objects go to _build/, the shared library next to this file.
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(ROOT, "_build")
LIB = os.path.join(HERE, "libha.so")
NAPI_OUT = os.path.join(HERE, "js", "ha_napi.node")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["engine.cpp", "gdn_seq.hip", "gdn_chunk.hip", "gdn_duo.hip", "gdn_split.hip", "gqa.hip", "tail.hip", "mnb.hip", "torso.hip"]
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I" + os.path.join(ROOT, "include"), "-I" + CSRC]
# Per-source additions. -amdgpu-mfma-vgpr-form keeps MFMA accumulators in VGPRs: the state passes scale their fp32
# accumulators on the VALU every chunk, which with AGPR accumulators costs a read and a write-back per element.
FILE_FLAGS = {"gdn_split.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "unknown target feature" not in l and "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("build step failed: %s\n%s" % (" ".join(cmd), out))
    if verbose and out.strip():
        print(out)


def build_lib(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    objs = []
    jobs = []
    for src in SOURCES:
        obj = os.path.join(BUILD, src.replace(".", "_") + ".o")
        objs.append(obj)
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        jobs.append([HIPCC] + HIP_FLAGS + FILE_FLAGS.get(src, []) + lang + ["-c", os.path.join(CSRC, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        list(ex.map(lambda c: _run(c, verbose), jobs))
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs, verbose)
    os.replace(tmp, LIB)
    return LIB


def build_napi(verbose=False):
    """N-API addon for Node (the reference's host language): a thin layer over libha.so."""
    node_inc = "/usr/include/node"
    src = os.path.join(HERE, "napi", "ha_napi.c")
    if not os.path.exists(src) or not os.path.exists(os.path.join(node_inc, "node_api.h")):
        return None
    _run(["gcc", "-O2", "-fPIC", "-shared", "-Wall", "-I" + node_inc, "-I" + os.path.join(ROOT, "include"), src,
          "-o", NAPI_OUT, "-L" + HERE, "-lha", "-Wl,-rpath,$ORIGIN/.."], verbose)
    return NAPI_OUT


def build_oracle(verbose=False):
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], verbose)


def build(verbose=False):
    build_lib(verbose)
    build_napi(verbose)
    build_oracle(verbose)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", LIB)
