"""Two processes on one GPU both running the paired gated-delta form at the same time. The form is an ordinary launch
whose producer workgroups never wait for their consumers, so a consumer that is resident waits only for a producer
that is resident or done, however the two kernels share the CUs: every forward of both processes gives bit for bit
this process's result from a quiet GPU, which is within the oracle bar."""
import os
import subprocess
import sys

import numpy as np
import pytest

import hybrid_attention as ha
import synth
from harness import Runner, oracle_gdn, rel_err

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHILD = r"""
import sys
sys.path[:0] = sys.argv[3].split(":")
import numpy as np
import hybrid_attention as ha
import synth
from harness import Runner
r = Runner(["linear_attention"], batch=8, max_ctx=1024)
r.set_params(0, synth.gdn_params(seed=9))
x = synth.gdn_rows(1000, 8, seed=9)
outs = [r.forward([x], recurrence=ha.CHUNKED_PAIRED)[0][0] for _ in range(int(sys.argv[2]))]
np.save(sys.argv[1], np.stack(outs))
print("child done", flush=True)
"""


def test_two_processes_run_the_paired_form_together(tmp_path):
    r = Runner(["linear_attention"], batch=8, max_ctx=1024)
    p = synth.gdn_params(seed=9)
    r.set_params(0, p)
    x = synth.gdn_rows(1000, 8, seed=9)
    (quiet,), _ = r.forward([x], recurrence=ha.CHUNKED_PAIRED)
    out = str(tmp_path / "child.npy")
    paths = ":".join([os.path.join(ROOT, "strands-decider-web_amd"), os.path.join(ROOT, "tests"),
                      os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests", "golden")])
    print("child process: 12 paired forwards at B=8 while this process runs its own", flush=True)
    c = subprocess.Popen([sys.executable, "-c", CHILD, out, "12", paths], stdout=subprocess.PIPE,
                         stderr=subprocess.STDOUT, text=True)
    mine = [r.forward([x], recurrence=ha.CHUNKED_PAIRED)[0][0] for _ in range(24)]
    log, _ = c.communicate(timeout=240)
    assert c.returncode == 0, log
    child = np.load(out)
    for i, o in enumerate(mine):
        assert np.array_equal(o, quiet), "this process, forward %d" % i
    for i, o in enumerate(child):
        assert np.array_equal(o, quiet), "child, forward %d" % i
    ref, _ = oracle_gdn(x[[0, 7]], p)
    e = rel_err(quiet[[0, 7]], ref)
    print("paired B=8 vs fp64, sequences 0 and 7: %.2e" % e)
    assert e < 2e-3
