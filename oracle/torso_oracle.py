"""CPU restatement of the torso ops around the token mixers and the projections (numpy, fp64). TEST INFRASTRUCTURE
ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import this module; the product library
never loads it. Each function cites the reference lines it restates:

- embed: EMBED, web/public/engine/wgsl.js:33-52. Row `id` of a quantised table in the MatMulNBits formats of
  gemmbench/kernels.js:1-14 (decode as oracle/mnb_oracle.py), symmetric (q - 2^(bits-1)) * scale or asymmetric
  q * scale + bias, in f32.
- add_norm: ADD_NORM, wgsl.js:55-78. Output row r reads source row rows[r]; with y the residual add x += y
  (written back) comes first; then h = x * (mean(x^2) + eps)^-1/2 * w. The weight is used as given (the exporter
  stores 1 + w for the zero-centred norms, export_engine.py).
- silu_mul: SILU_MUL, wgsl.js:81-90. mid = silu(g) * u, with big[t] = [g (I) | u (I)].
- add_bias: ADD_BIAS, wgsl.js:113-121. y += c per column.

Pins (tests/test_oracle_torso.py):
- torch's own rms_norm and silu (library routines);
- scale invariance and the constant-row closed form of the norm;
- silu(0) = 0 and silu(x) -> x;
- a scalar restatement of EMBED's element indexing;
- hand-built blocks with known codes.
"""
import numpy as np

import mnb_oracle as mo


def embed(words, scales, ids, D, bits=4, group=32, asym=False, bias=None):
    """Table [rows][D/32][bits] u32 + scales [rows][D/group] (+ bias) -> x [L][D] (float32 values, fp64 array)."""
    rows = np.asarray(words).reshape(-1, D // 32, mo.words_per_block(bits)).shape[0]
    ids = np.asarray(ids, np.int64)
    q = mo.decode(np.asarray(words).reshape(rows, D // 32, mo.words_per_block(bits))[ids], bits).reshape(len(ids), D)
    sc = np.repeat(np.asarray(scales, np.float16).reshape(rows, D // group)[ids].astype(np.float32), group, axis=1)
    if asym:
        bi = np.repeat(np.asarray(bias, np.float16).reshape(rows, D // group)[ids].astype(np.float32), group, axis=1)
        return (q.astype(np.float32) * sc + bi).astype(np.float64)
    return ((q - 2 ** (bits - 1)).astype(np.float32) * sc).astype(np.float64)


def add_norm(x, y, w, rows=None, eps=1e-6):
    """x [nx][D] (updated copy returned), y [nx][D] or None, w [D] -> (h [R][D] fp64, x after the add)."""
    x = np.asarray(x, np.float64).copy()
    src = np.arange(x.shape[0]) if rows is None else np.asarray(rows, np.int64)
    if y is not None:
        x[src] = x[src] + np.asarray(y, np.float64)[src]
    xs = x[src]
    inv = 1.0 / np.sqrt((xs * xs).mean(axis=1, keepdims=True) + eps)
    return xs * inv * np.asarray(w, np.float64)[None, :], x


def silu_mul(big, I):
    """big [L][2I] -> mid [L][I] fp64."""
    big = np.asarray(big, np.float64)
    g, u = big[:, :I], big[:, I:2 * I]
    return g / (1.0 + np.exp(-g)) * u


def add_bias(y, c):
    return np.asarray(y, np.float64) + np.asarray(c, np.float64)[None, :]
