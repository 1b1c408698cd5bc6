"""CPU restatement of the MatMulNBits projections (numpy, fp64). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import this module; the product library
never loads it. Each function cites the reference lines it restates:

- quant_int4: the exporter's int4 RTN quantiser, convert/export_engine.py:17-26 (symmetric, block 32, the scale
  is the block's largest-magnitude value / -8 rounded to f16, q = clamp(round(w / scale) + 8, 0, 15), element 2i in
  the low nibble of byte i).
- decode / dequant: the weight formats of web/public/gemmbench/kernels.js:1-14 and their decode, kernels.js:22-36
  (4 bits: element e at bits 4(e%8) of word e/8; 2 bits: bits 2(e%16) of word e/16; 3 bits: 2-bit low words plus
  bit e of word 2; one f16 scale per `group` values of a row, symmetric (q - 2^(bits-1)) * scale, asymmetric
  q * scale + bias).
- matmul: y[M][N] = a[M][K] . W[N][K]^T in fp64 (the reference's own check, gemmbench/bench.js:48-50, is this sum
  in fp32 on a few columns).
- fwht: the orthonormal Walsh-Hadamard transform of each n-block, web/public/engine/wgsl.js:94-110 (Sylvester
  order, scaled by 1/sqrt(n)).

Pins (tests/test_oracle_mnb.py): a scalar restatement of bench.js:48-50's nibble indexing; hand-built blocks with
known codes for every bit width; the quantiser's own dequantised values and its exact -8 code for each block's
largest-magnitude element; one-hot rows of a that pick weight columns exactly; FWHT against scipy's Hadamard matrix
and H^2 = I.
"""
import numpy as np


def quant_int4(W):
    """W [N][K] float -> (packed u8 [N][K/32][16], scales f16 [N][K/32], dequantised f32 [N][K])."""
    W = np.asarray(W, np.float32)
    N, K = W.shape
    assert K % 32 == 0
    b = W.reshape(N, K // 32, 32)
    idx = np.abs(b).argmax(-1)[..., None]
    scale = np.take_along_axis(b, idx, -1) / np.float32(-8.0)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float16).astype(np.float32)
    q = np.clip(np.round(b / scale) + 8, 0, 15).astype(np.uint8)
    packed = (q[..., 0::2] | (q[..., 1::2] << 4)).astype(np.uint8)
    deq = ((q.astype(np.float32) - 8) * scale).reshape(N, K)
    return packed, scale[..., 0].astype(np.float16), deq


def words_per_block(bits):
    return {4: 4, 3: 3, 2: 2}[bits]


def decode(words, bits):
    """Packed blocks u32 [..., bits] -> codes [..., 32] (ints)."""
    w = np.asarray(words, np.uint64)
    e = np.arange(32, dtype=np.uint64)
    if bits == 4:
        return ((w[..., e // 8] >> (4 * (e % 8))) & 15).astype(np.int64)
    lo = (w[..., e // 16] >> (2 * (e % 16))) & 3
    if bits == 2:
        return lo.astype(np.int64)
    hi = (w[..., 2:3] >> e) & 1
    return (lo | (hi << 2)).astype(np.int64)


def dequant(words, scales, N, K, bits=4, group=32, asym=False, bias=None):
    """Packed [N][K/32][bits] u32, scales f16 [N][K/group] (+ bias) -> W fp64 [N][K]."""
    q = decode(np.asarray(words).reshape(N, K // 32, words_per_block(bits)), bits).reshape(N, K).astype(np.float64)
    sc = np.repeat(np.asarray(scales, np.float16).astype(np.float64).reshape(N, K // group), group, axis=1)
    if asym:
        bi = np.repeat(np.asarray(bias, np.float16).astype(np.float64).reshape(N, K // group), group, axis=1)
        return q * sc + bi
    return (q - 2 ** (bits - 1)) * sc


def matmul(a, W):
    """a [M][K] (f16 values), W [N][K] -> y [M][N] fp64."""
    return np.asarray(a, np.float16).astype(np.float64) @ np.asarray(W, np.float64).T


def fwht(x, n):
    """Orthonormal Walsh-Hadamard transform (Sylvester order) of every contiguous n-block of x (fp64)."""
    y = np.asarray(x, np.float64).reshape(-1, n).copy()
    h = 1
    while h < n:
        y = y.reshape(-1, n // (2 * h), 2, h)
        u, v = y[:, :, 0, :].copy(), y[:, :, 1, :].copy()
        y[:, :, 0, :], y[:, :, 1, :] = u + v, u - v
        y = y.reshape(-1, n)
        h *= 2
    return (y / np.sqrt(n)).reshape(np.shape(x))


def rel_err(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))
