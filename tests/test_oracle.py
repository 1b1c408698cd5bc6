"""Pins the CPU oracle (oracle/ha_oracle.c) before anything is compared against it.

Each oracle function is checked against (i) the golden fixtures made by the independent numpy restatement
(tests/golden/brute.py via make_golden.py), (ii) closed forms and known answers the mathematics fixes, and
(iii) invariants (history / prefix-state composition, sequential == chunked). The reference ships no vectors
for this path, so these are the pins; each check is chosen so that a plausible slip (a dropped tap, a wrong
sign in the rotation, q and k swapped, a missing decay factor, an off-by-one in the mask) fails it.
"""
import os

import numpy as np
import pytest

import brute
import oracle

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _gdn_params(conv, negA, dtb, gnorm):
    return {"conv": conv, "neg_exp_A": negA, "dt_bias": dtb, "gnorm": gnorm}


# ------------------------------------------------------------------------------------------------ helpers
def test_f16_round_matches_numpy():
    g = np.random.default_rng(1)
    xs = np.concatenate([g.standard_normal(2000) * s for s in (1e-7, 1e-5, 1e-3, 1, 100, 3e4)]
                        + [np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e6, 2 ** -24, 2 ** -25, 3 * 2 ** -26])])
    xs = xs.astype(np.float32)
    got = np.array([oracle.f16_round(x) for x in xs], np.float32)
    want = xs.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(got, want)


def test_rope_table_closed_form():
    LT, RD, theta = 50, 64, 1e7
    tab = oracle.rope_table(LT, RD, theta)
    t = np.arange(LT)[:, None]
    i = np.arange(RD // 2)[None, :]
    ang = t / theta ** (2.0 * i / RD)
    np.testing.assert_allclose(tab[:, 0::2], np.cos(ang), rtol=0, atol=1e-7)
    np.testing.assert_allclose(tab[:, 1::2], np.sin(ang), rtol=0, atol=1e-7)
    assert np.all(tab[0, 0::2] == 1.0) and np.all(tab[0, 1::2] == 0.0)  # position 0: identity rotation


# ------------------------------------------------------------------------------------------------ conv
def test_conv_direct_sum():
    g = np.random.default_rng(2)
    T, C, KC, stride = 9, 11, 4, 13
    rows = g.standard_normal((T, stride)).astype(np.float32)
    w = g.standard_normal((C, KC)).astype(np.float32)
    hist = g.standard_normal((KC - 1, C)).astype(np.float32)
    h0 = hist.copy()
    u = oracle.conv_silu(rows, w, hist)
    x = np.concatenate([h0, rows[:, :C]], 0).astype(np.float64)
    for t in range(T):
        s = sum(w[:, j].astype(np.float64) * x[t + j] for j in range(KC))
        np.testing.assert_allclose(u[t], brute.silu(s), rtol=1e-13, atol=1e-15)
    np.testing.assert_array_equal(hist, rows[T - 3:, :C])  # history roll keeps the last 3 pre-conv rows


def test_conv_single_current_tap_is_silu():
    g = np.random.default_rng(3)
    T, C = 6, 8
    rows = g.standard_normal((T, C)).astype(np.float32)
    w = np.zeros((C, 4), np.float32)
    w[:, 3] = 1.0  # only the current token (tap 3, as F.conv1d(pad=3)[:T])
    u = oracle.conv_silu(rows, w, g.standard_normal((3, C)).astype(np.float32))
    np.testing.assert_allclose(u, brute.silu(rows.astype(np.float64)), rtol=1e-14)


def test_conv_history_equivalence():
    g = np.random.default_rng(4)
    T, C = 10, 5
    rows = g.standard_normal((T, C)).astype(np.float32)
    w = g.standard_normal((C, 4)).astype(np.float32)
    full = oracle.conv_silu(rows, w, np.zeros((3, C), np.float32))
    part = oracle.conv_silu(rows[3:], w, rows[:3].copy())
    np.testing.assert_array_equal(full[3:], part)


def test_conv_short_call_history_roll():
    # a call shorter than the history keeps older history rows (HIST_UPDATE reads them for src < 0)
    g = np.random.default_rng(5)
    C = 4
    hist = g.standard_normal((3, C)).astype(np.float32)
    h0 = hist.copy()
    rows = g.standard_normal((2, C)).astype(np.float32)
    oracle.conv_silu(rows, np.zeros((C, 4), np.float32), hist)
    np.testing.assert_array_equal(hist, np.concatenate([h0[2:], rows], 0))


# ------------------------------------------------------------------------------------------------ gated delta
def test_gdn_golden_fixture():
    f = np.load(os.path.join(GOLD, "gdn_tiny.npz"))
    H, DK, DV = int(f["H"]), int(f["DK"]), int(f["DV"])
    p = _gdn_params(f["conv"], f["negA"], f["dtb"], f["gnorm"])
    st = oracle.GdnState(H, DK, DV)
    out1 = oracle.gdn_forward(f["rows1"], p, st, H, DK, DV)
    out2 = oracle.gdn_forward(f["rows2"], p, st, H, DK, DV)
    np.testing.assert_allclose(out1, f["out1"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out2, f["out2"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(st.S, f["S2"], rtol=1e-12, atol=1e-14)
    np.testing.assert_array_equal(st.hist, f["hist2"].astype(np.float32))
    raw = oracle.gdn_forward(f["rows1"], p, oracle.GdnState(H, DK, DV), H, DK, DV, gnorm=False)
    np.testing.assert_allclose(raw, f["raw1"], rtol=1e-5, atol=1e-7)


def _identity_conv(C):
    w = np.zeros((C, 4), np.float32)
    w[:, 3] = 1.0
    return w


def _rows_for(u_target_pre, H, DK, DV, a, b, stride):
    T = u_target_pre.shape[0]
    C = 2 * H * DK + H * DV
    rows = np.zeros((T, stride), np.float32)
    rows[:, :C] = u_target_pre
    rows[:, C + H * DV:C + H * DV + H] = a
    rows[:, C + H * DV + H:C + H * DV + 2 * H] = b
    return rows


def test_gdn_one_token_closed_form():
    # from S = 0 one token gives S = beta k^ v^T and o = beta (k^ . q^) v   (v = silu(x_v), conv tap 3 only)
    g = np.random.default_rng(6)
    H, DK, DV = 2, 8, 8
    C = 2 * H * DK + H * DV
    x = g.standard_normal((1, C)).astype(np.float32)
    a, b = g.standard_normal(H).astype(np.float32), g.standard_normal(H).astype(np.float32)
    rows = _rows_for(x, H, DK, DV, a, b, C + H * DV + 2 * H)
    p = _gdn_params(_identity_conv(C), np.full(H, -1.0, np.float32), np.zeros(H, np.float32), np.ones(DV, np.float32))
    st = oracle.GdnState(H, DK, DV)
    o = oracle.gdn_forward(rows, p, st, H, DK, DV, gnorm=False)
    u = brute.silu(x[0].astype(np.float64))
    for h in range(H):
        q, k, v = u[h * DK:(h + 1) * DK], u[H * DK + h * DK:H * DK + (h + 1) * DK], u[2 * H * DK + h * DV:2 * H * DK + (h + 1) * DV]
        qn, kn = q / np.sqrt(q @ q + 1e-6) / np.sqrt(DK), k / np.sqrt(k @ k + 1e-6)
        beta = 1 / (1 + np.exp(-float(b[h])))
        np.testing.assert_allclose(st.S[h], beta * np.outer(kn, v), rtol=1e-12, atol=1e-15)
        np.testing.assert_allclose(o[0, h * DV:(h + 1) * DV], beta * (kn @ qn) * v, rtol=1e-6, atol=1e-9)


def test_gdn_beta_zero_is_pure_decay():
    # beta = 0 (b -> -inf): S_T = prod(alpha) S_0 and o_t = prod_{s<=t}(alpha_s) S_0^T q^_t
    g = np.random.default_rng(7)
    H, DK, DV, T = 2, 8, 8, 5
    C = 2 * H * DK + H * DV
    x = g.standard_normal((T, C)).astype(np.float32)
    a = g.standard_normal((T, H)).astype(np.float32)
    rows = _rows_for(x, H, DK, DV, a, np.full((T, H), -1e4, np.float32), C + H * DV + 2 * H)
    negA = np.array([-0.7, -1.3], np.float32)
    dtb = np.array([0.2, -0.1], np.float32)
    p = _gdn_params(_identity_conv(C), negA, dtb, np.ones(DV, np.float32))
    st = oracle.GdnState(H, DK, DV)
    S0 = g.standard_normal((H, DK, DV))
    st.S[:] = S0
    o = oracle.gdn_forward(rows, p, st, H, DK, DV, gnorm=False)
    u = brute.silu(x.astype(np.float64))
    for h in range(H):
        cum = 1.0
        for t in range(T):
            cum *= np.exp(negA[h] * brute.softplus(float(a[t, h]) + float(dtb[h])))
            q = u[t, h * DK:(h + 1) * DK]
            qn = q / np.sqrt(q @ q + 1e-6) / np.sqrt(DK)
            np.testing.assert_allclose(o[t, h * DV:(h + 1) * DV], cum * (S0[h].T @ qn), rtol=1e-6, atol=1e-9)
        np.testing.assert_allclose(st.S[h], cum * S0[h], rtol=1e-12)


def test_gdn_orthonormal_keys_are_recalled():
    # alpha = 1 (a -> -inf), beta = 1 (b -> +inf), keys e_0..e_{T-1}: the delta rule stores v_i exactly at k_i
    H, DK, DV, T = 1, 8, 8, 6
    C = 2 * H * DK + H * DV
    g = np.random.default_rng(8)
    x = np.zeros((T, C), np.float32)
    x[:, :DK] = g.standard_normal((T, DK))
    for i in range(T):
        x[i, DK + i] = 30.0  # silu(30) e_i, normalised -> e_i (up to the 1e-6 epsilon)
    x[:, 2 * DK:] = g.standard_normal((T, DV))
    rows = _rows_for(x, H, DK, DV, np.full((T, H), -1e4, np.float32), np.full((T, H), 1e4, np.float32), C + H * DV + 2 * H)
    p = _gdn_params(_identity_conv(C), np.full(H, -1.0, np.float32), np.zeros(H, np.float32), np.ones(DV, np.float32))
    st = oracle.GdnState(H, DK, DV)
    oracle.gdn_forward(rows, p, st, H, DK, DV, gnorm=False)
    v = brute.silu(x[:, 2 * DK:].astype(np.float64))
    for i in range(T):
        np.testing.assert_allclose(st.S[0][i], v[i], rtol=1e-8, atol=1e-8)
    assert np.abs(st.S[0][T:]).max() < 1e-12


def test_gdn_prefix_state_composition_bit_exact():
    g = np.random.default_rng(9)
    H, DK, DV, T, P = 2, 8, 8, 13, 5
    C = 2 * H * DK + H * DV
    stride = C + H * DV + 2 * H
    rows = g.standard_normal((T, stride)).astype(np.float32)
    p = _gdn_params((0.5 * g.standard_normal((C, 4))).astype(np.float32), np.array([-1.0, -0.5], np.float32),
                    np.zeros(H, np.float32), np.ones(DV, np.float32))
    full_st = oracle.GdnState(H, DK, DV)
    full = oracle.gdn_forward(rows, p, full_st, H, DK, DV)
    st = oracle.GdnState(H, DK, DV)
    a = oracle.gdn_forward(rows[:P], p, st, H, DK, DV)
    b = oracle.gdn_forward(rows[P:], p, st, H, DK, DV)
    np.testing.assert_array_equal(np.concatenate([a, b]), full)
    np.testing.assert_array_equal(st.S, full_st.S)


@pytest.mark.parametrize("chunk", [1, 7, 64])
def test_gdn_sequential_equals_chunked(chunk):
    g = np.random.default_rng(10)
    H, DK, DV, T = 2, 16, 8, 130
    C = 2 * H * DK + H * DV
    stride = C + H * DV + 2 * H
    rows = g.standard_normal((T, stride)).astype(np.float32)
    p = _gdn_params((0.5 * g.standard_normal((C, 4))).astype(np.float32), np.array([-1.0, -0.05], np.float32),
                    np.zeros(H, np.float32), np.ones(DV, np.float32))
    s1, s2 = oracle.GdnState(H, DK, DV), oracle.GdnState(H, DK, DV)
    s1.S[:] = s2.S[:] = g.standard_normal((H, DK, DV)) * 0.1
    o1 = oracle.gdn_forward(rows, p, s1, H, DK, DV, gnorm=False, chunk=0)
    o2 = oracle.gdn_forward(rows, p, s2, H, DK, DV, gnorm=False, chunk=chunk)
    assert oracle.rel_err(o2, o1) < 1e-11
    assert oracle.rel_err(s2.S, s1.S) < 1e-11


def test_gdn_gated_norm_closed_form():
    g = np.random.default_rng(11)
    H, DK, DV, T = 2, 8, 8, 4
    C = 2 * H * DK + H * DV
    stride = C + H * DV + 2 * H
    rows = g.standard_normal((T, stride)).astype(np.float32)
    p = _gdn_params((0.5 * g.standard_normal((C, 4))).astype(np.float32), np.full(H, -1.0, np.float32),
                    np.zeros(H, np.float32), (1 + 0.3 * g.standard_normal(DV)).astype(np.float32))
    raw = oracle.gdn_forward(rows, p, oracle.GdnState(H, DK, DV), H, DK, DV, gnorm=False).astype(np.float64)
    y = oracle.gdn_forward(rows, p, oracle.GdnState(H, DK, DV), H, DK, DV, gnorm=True)
    for h in range(H):
        o = raw[:, h * DV:(h + 1) * DV]
        z = rows[:, C + h * DV:C + (h + 1) * DV].astype(np.float64)
        want = p["gnorm"] * o / np.sqrt(np.mean(o * o, 1, keepdims=True) + 1e-6) * brute.silu(z)
        np.testing.assert_allclose(y[:, h * DV:(h + 1) * DV], want, rtol=2e-6, atol=1e-7)


# ------------------------------------------------------------------------------------------------ GQA
def _gqa_oracle(rows, qw, kw, HQ, HK, HD, RD, theta, LT, cache=None, f16=False):
    cache = cache or oracle.GqaCache(LT, HK, HD)
    rope = oracle.rope_table(LT, RD, theta)
    out = oracle.gqa_forward(rows, {"q_norm": qw, "k_norm": kw}, cache, rope, HQ, HK, HD, RD, f16=f16)
    return out, cache


def test_gqa_golden_fixture_and_prefix_composition():
    f = np.load(os.path.join(GOLD, "gqa_tiny.npz"))
    HQ, HK, HD, RD, theta = int(f["HQ"]), int(f["HK"]), int(f["HD"]), int(f["RD"]), float(f["theta"])
    out1, cache = _gqa_oracle(f["rows1"], f["qw"], f["kw"], HQ, HK, HD, RD, theta, 16)
    out2, cache = _gqa_oracle(f["rows2"], f["qw"], f["kw"], HQ, HK, HD, RD, theta, 16, cache)
    np.testing.assert_allclose(out1, f["out1"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out2, f["out2"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(cache.K[:, :9], f["K"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(cache.V[:, :9], f["V"], rtol=0, atol=0)
    full, _ = _gqa_oracle(np.concatenate([f["rows1"], f["rows2"]]), f["qw"], f["kw"], HQ, HK, HD, RD, theta, 16)
    np.testing.assert_array_equal(np.concatenate([out1, out2]), full)


def test_gqa_first_position_identity_and_rms_norm():
    g = np.random.default_rng(12)
    HQ, HK, HD, RD = 4, 2, 16, 8
    stride = HQ * 2 * HD + 2 * HK * HD
    rows = g.standard_normal((1, stride)).astype(np.float32)
    kw = (1 + 0.2 * g.standard_normal(HD)).astype(np.float32)
    out, cache = _gqa_oracle(rows, np.ones(HD, np.float32), kw, HQ, HK, HD, RD, 1e7, 4)
    for kh in range(HK):
        k = rows[0, HQ * 2 * HD + kh * HD:HQ * 2 * HD + (kh + 1) * HD].astype(np.float64)
        np.testing.assert_allclose(cache.K[kh, 0], k / np.sqrt(np.mean(k * k) + 1e-6) * kw, rtol=1e-6)
    # one key only: softmax weight 1, so out = v * sigmoid(gate) for every head of the group
    for h in range(HQ):
        kh = h // (HQ // HK)
        v = rows[0, HQ * 2 * HD + HK * HD + kh * HD:HQ * 2 * HD + HK * HD + (kh + 1) * HD].astype(np.float64)
        gate = rows[0, h * 2 * HD + HD:(h + 1) * 2 * HD].astype(np.float64)
        np.testing.assert_allclose(out[0, h * HD:(h + 1) * HD], v / (1 + np.exp(-gate)), rtol=1e-6, atol=1e-7)


def test_gqa_head_map_and_rotation_sign():
    # brute force on a prefilled cache with strongly different KV heads; catches kh = h % HK, a flipped
    # rotate-half sign or a mask off by one
    g = np.random.default_rng(13)
    HQ, HK, HD, RD, theta = 4, 2, 16, 8, 100.0
    stride = HQ * 2 * HD + 2 * HK * HD
    rows = g.standard_normal((9, stride)).astype(np.float32)
    rows[:, HQ * 2 * HD + HK * HD + HD:] *= 10  # kv head 1 values differ in scale
    qw, kw = (1 + 0.1 * g.standard_normal(HD)).astype(np.float32), (1 + 0.1 * g.standard_normal(HD)).astype(np.float32)
    want, Kb, _ = brute.gqa(rows, qw, kw, HQ, HK, HD, RD, theta)
    got, cache = _gqa_oracle(rows, qw, kw, HQ, HK, HD, RD, theta, 12)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(cache.K[:, :9], Kb, rtol=1e-5, atol=1e-6)


def test_gqa_f16_points_stay_close_to_fp64():
    g = np.random.default_rng(14)
    HQ, HK, HD, RD = 8, 2, 256, 64
    stride = 5120
    rows = g.standard_normal((40, stride)).astype(np.float16).astype(np.float32)
    ones = np.ones(HD, np.float32)
    exact, _ = _gqa_oracle(rows, ones, ones, HQ, HK, HD, RD, 1e7, 64, f16=False)
    half, cache = _gqa_oracle(rows, ones, ones, HQ, HK, HD, RD, 1e7, 64, f16=True)
    assert oracle.rel_err(half, exact) < 5e-3
    # stored K/V are f16 values
    np.testing.assert_array_equal(cache.K[:, :40], cache.K[:, :40].astype(np.float16).astype(np.float32))
