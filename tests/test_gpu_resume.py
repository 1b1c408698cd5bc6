"""The prefix-cache case on the GPU: a 1,536-token prefix through 3 gated-delta layers + 1 GQA layer, snapshot, then
5 independent 64-token suffixes resumed from it; each must equal the last 64 rows of a full 1,600-token forward
bit for bit (the reference claims the same for its engine, README.md:60-61). Also the failure paths of the
snapshot boundary (engine.js:316 context guard, released / foreign handles)."""
import numpy as np
import pytest

import hybrid_attention as ha
import synth
from harness import Runner, oracle_gdn, oracle_gqa, rel_err

pytestmark = pytest.mark.gpu
KINDS = ["linear_attention", "linear_attention", "linear_attention", "full_attention"]


def _inputs(T, part, seed=3):
    return [synth.gdn_rows(T, seed=seed, layer=i, part=part) if k == "linear_attention"
            else synth.gqa_rows(T, seed=seed, layer=i, part=part) for i, k in enumerate(KINDS)]


def _runner(recurrence_mode=None):
    r = Runner(KINDS)
    for i, k in enumerate(KINDS):
        r.set_params(i, synth.gdn_params(seed=3, layer=i) if k == "linear_attention"
                     else synth.gqa_params(seed=3, layer=i, noise=0.1))
    return r


def test_config3_prefix_cache_bit_exact():
    r = _runner()
    prefix = _inputs(1536, part=0)
    _, snap = r.forward(prefix, keep=True)
    assert snap.P == 1536 and snap.state_pos == 1536
    for s in range(5):
        suffix = _inputs(64, part=1 + s)
        outs, _ = r.forward(suffix, cache=snap)
        full_in = [np.concatenate([p, q], 1) for p, q in zip(prefix, suffix)]
        full, _ = r.forward(full_in)
        for i in range(len(KINDS)):
            np.testing.assert_array_equal(outs[i], full[i][:, 1536:], err_msg="suffix %d layer %d" % (s, i))
    snap.release()
    snap.release()  # idempotent


def test_config3_suffix_matches_oracle():
    r = _runner()
    prefix, suffix = _inputs(1536, 0), _inputs(64, 1)
    _, snap = r.forward(prefix, keep=True)
    outs, _ = r.forward(suffix, cache=snap)
    for i, k in enumerate(KINDS):
        if k == "linear_attention":
            p = synth.gdn_params(seed=3, layer=i)
            _, st = oracle_gdn(prefix[i], p)
            ref, _ = oracle_gdn(suffix[i], p, states=st)
            assert rel_err(outs[i], ref) < 2e-3, i
        else:
            p = synth.gqa_params(seed=3, layer=i, noise=0.1)
            _, caches = oracle_gqa(prefix[i], p, 4096)
            ref, _ = oracle_gqa(suffix[i], p, 4096, caches=caches)
            assert rel_err(outs[i], ref) < 1e-2, i


def test_snapshot_errors():
    r = Runner(["linear_attention", "full_attention"], max_ctx=128)
    x = [synth.gdn_rows(100), synth.gqa_rows(100)]
    _, snap = r.forward(x, keep=True)
    with pytest.raises(ha.HAError) as ei:  # 100 + 40 > 128
        r.forward([synth.gdn_rows(40), synth.gqa_rows(40)], cache=snap)
    assert ei.value.code == ha.HA_ERR_CONTEXT and "exceeds 128" in str(ei.value)
    other = Runner(["linear_attention", "full_attention"], max_ctx=128)
    with pytest.raises(ha.HAError) as ei:
        other.forward([synth.gdn_rows(4), synth.gqa_rows(4)], cache=snap)
    assert ei.value.code == ha.HA_ERR_HANDLE
    snap.release()
    with pytest.raises(ha.HAError) as ei:
        r.forward([synth.gdn_rows(4), synth.gqa_rows(4)], cache=snap)
    assert ei.value.code == ha.HA_ERR_HANDLE and "released" in str(ei.value)
    with pytest.raises(ha.HAError) as ei:
        r.eng.set_param(0, "q_norm", np.ones(256))
    assert ei.value.code == ha.HA_ERR_PARAM


def test_resumes_without_restore_copy():
    # Calls resumed from one snapshot back to back: the working K/V caches already hold its rows, so the engine does
    # not copy them again. Between them a kept snapshot, a resume from that one (again no copy) and a return to the
    # first (copied again). Every suffix must still equal the same rows of one full forward.
    r = _runner()
    prefix = _inputs(1536, part=0)
    _, snap = r.forward(prefix, keep=True)
    sufs = [_inputs(L, part=10 + j) for j, L in enumerate([1, 7, 1, 33])]
    o1, _ = r.forward(sufs[0], cache=snap)
    o2, _ = r.forward(sufs[1], cache=snap)
    o3, kept = r.forward(sufs[2], cache=snap, keep=True)
    o4, _ = r.forward(sufs[3], cache=kept)
    o5, _ = r.forward(sufs[1], cache=snap)
    cases = [([sufs[0]], o1), ([sufs[1]], o2), ([sufs[2]], o3), ([sufs[2], sufs[3]], o4), ([sufs[1]], o5)]
    for n, (parts, outs) in enumerate(cases):
        full_in = [np.concatenate([p] + [q[i] for q in parts], 1) for i, p in enumerate(prefix)]
        full, _ = r.forward(full_in)
        start = full_in[0].shape[1] - outs[0].shape[1]
        for i in range(len(KINDS)):
            np.testing.assert_array_equal(outs[i], full[i][:, start:], err_msg="call %d layer %d" % (n + 1, i))


def test_snapshot_block_reuse():
    # A released snapshot's device block becomes its engine's spare, and the next snapshot that fits takes it: that
    # snapshot must hold its own context (a suffix resumed from it equals the same rows of one full forward), and the
    # released one is refused.
    r = _runner()
    long_in, short_in, sfx = _inputs(900, part=20), _inputs(700, part=21), _inputs(16, part=22)
    _, s1 = r.forward(long_in, keep=True)
    s1.release()
    _, s2 = r.forward(short_in, keep=True)
    outs, _ = r.forward(sfx, cache=s2)
    full, _ = r.forward([np.concatenate([p, q], 1) for p, q in zip(short_in, sfx)])
    for i in range(len(KINDS)):
        np.testing.assert_array_equal(outs[i], full[i][:, 700:], err_msg="layer %d" % i)
    with pytest.raises(ha.HAError):
        r.forward(sfx, cache=s1)


def test_restore_copy_invalidates_other_snapshots():
    # After a resume from an unrelated snapshot u (longer than snap, so its restore copy rewrites all of snap's rows),
    # a resume from snap must copy snap's rows back; and a fresh forward invalidates both. Each suffix must equal the
    # same rows of one full forward of its own context.
    r = _runner()
    prefix, other = _inputs(1536, part=30), _inputs(1600, part=31)
    sfx = _inputs(5, part=32)
    _, snap = r.forward(prefix, keep=True)
    _, u = r.forward(other, keep=True)  # a fresh forward: the working caches now hold u's rows only
    runs = []
    for cache, ctx in [(snap, prefix), (u, other), (snap, prefix), (snap, prefix), (u, other)]:
        outs, _ = r.forward(sfx, cache=cache)
        runs.append((outs, ctx))
    for n, (outs, ctx) in enumerate(runs):
        full, _ = r.forward([np.concatenate([p, q], 1) for p, q in zip(ctx, sfx)])
        P = ctx[0].shape[1]
        for i in range(len(KINDS)):
            np.testing.assert_array_equal(outs[i], full[i][:, P:], err_msg="call %d layer %d" % (n + 1, i))
