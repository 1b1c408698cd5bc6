"""Seeded synthetic inputs for the hybrid-attention path (the benchmark configs use no real weights).

One NumPy PCG64 stream per tensor, ``SeedSequence([seed, layer, tensor_id])``, so adding a tensor never shifts
the others. Rows follow the engine's fused layouts (web/public/engine/engine.js:264-274,
convert/export_engine.py:52,61): linear rows qkv | z | a | b (padded to the stride), full rows
[q|gate] x HQ | k x HK | v x HK.
"""
import numpy as np

TENSOR_IDS = {"rows": 1, "conv": 2, "gnorm": 3, "q_norm": 4, "k_norm": 5, "neg_exp_A": 6, "dt_bias": 7}


def rng(seed, layer, name):
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, layer, TENSOR_IDS[name]])))


def lin_width(H=16, DK=128, DV=128):
    return 2 * H * DK + H * DV + H * DV + 2 * H


def gdn_rows(T, B=1, H=16, DK=128, DV=128, stride=8256, seed=0, layer=0, part=0):
    """[B][T][stride] float32: every used column ~N(0,1) (q/k/v pre-conv, z, a, b); padding columns 0.
    ``part`` selects an independent block of rows (e.g. distinct suffixes after a shared prefix)."""
    g = np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, layer, TENSOR_IDS["rows"], part])))
    w = lin_width(H, DK, DV)
    out = np.zeros((B, T, stride), np.float32)
    out[:, :, :w] = g.standard_normal((B, T, w), dtype=np.float32)
    return out


def gdn_params(H=16, DK=128, DV=128, KC=4, seed=0, layer=0, neg_exp_A=-1.0, dt_bias=0.0, gnorm_noise=0.1):
    """conv taps ~N(0, 0.5^2) ("N(0,0.5)" read as std 0.5), negA / dt_bias constants
    (alpha = exp(negA * softplus(a + dt_bias))), gated-norm weight 1 + gnorm_noise * N(0,1)."""
    C = 2 * H * DK + H * DV
    conv = (0.5 * rng(seed, layer, "conv").standard_normal((C, KC))).astype(np.float32)
    gn = (1.0 + gnorm_noise * rng(seed, layer, "gnorm").standard_normal(DV)).astype(np.float32)
    return {"conv": conv, "neg_exp_A": np.full(H, neg_exp_A, np.float32), "dt_bias": np.full(H, dt_bias, np.float32),
            "gnorm": gn}


def gqa_rows(T, B=1, HQ=8, HK=2, HD=256, stride=5120, seed=0, layer=0, part=0):
    """[B][T][stride] float16 values (returned as float16): every used column ~N(0,1)."""
    g = np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, layer, TENSOR_IDS["rows"], part])))
    w = HQ * 2 * HD + 2 * HK * HD
    out = np.zeros((B, T, stride), np.float16)
    out[:, :, :w] = g.standard_normal((B, T, w), dtype=np.float32).astype(np.float16)
    return out


def gqa_params(HD=256, seed=0, layer=0, noise=0.0):
    """q_norm / k_norm as stored by the manifest (1 + w); noise = 0 gives unit gain."""
    q = (1.0 + noise * rng(seed, layer, "q_norm").standard_normal(HD)).astype(np.float32)
    k = (1.0 + noise * rng(seed, layer, "k_norm").standard_normal(HD)).astype(np.float32)
    return {"q_norm": q, "k_norm": k}
