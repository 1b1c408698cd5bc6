"""ctypes wrapper of the CPU oracle (oracle/ha_oracle.c). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import this module; the product
library never loads the oracle.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
_lib = None

F = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
D = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("oracle/liboracle.so is not built (make -C oracle)")
        l = ctypes.CDLL(LIB_PATH)
        i, vp = ctypes.c_int, ctypes.c_void_p
        l.orc_f16_round.argtypes = [ctypes.c_float]
        l.orc_f16_round.restype = ctypes.c_float
        l.orc_rope_table.argtypes = [i, i, ctypes.c_double, F]
        l.orc_rope_table.restype = None
        l.orc_conv_silu.argtypes = [i, i, i, i, F, F, F, D]
        l.orc_conv_silu.restype = None
        l.orc_gdn_forward.argtypes = [i, i, i, i, i, i, F, F, F, F, vp, F, D, F, i]
        l.orc_gdn_forward.restype = i
        l.orc_gqa_forward.argtypes = [i, i, i, i, i, i, i, i, F, F, F, F, F, F, F, i]
        l.orc_gqa_forward.restype = i
        _lib = l
    return _lib


def f16_round(x):
    return lib().orc_f16_round(float(x))


def rope_table(LT, RD, theta):
    out = np.zeros((LT, RD), np.float32)
    lib().orc_rope_table(LT, RD, theta, out)
    return out


def conv_silu(rows, w, hist):
    """rows [T][stride] f32 (channels [0, C) used), w [C][KC], hist [KC-1][C] (updated in place) -> u [T][C] f64."""
    T, stride = rows.shape
    C, KC = w.shape
    u = np.zeros((T, C), np.float64)
    lib().orc_conv_silu(T, C, KC, stride, np.ascontiguousarray(rows, np.float32), np.ascontiguousarray(w, np.float32),
                        hist, u)
    return u


class GdnState:
    """Per-sequence gated-delta context: conv history [KC-1][C] (f32) and state [H][DK][DV] (f64)."""

    def __init__(self, H=16, DK=128, DV=128, KC=4):
        C = 2 * H * DK + H * DV
        self.hist = np.zeros((KC - 1, C), np.float32)
        self.S = np.zeros((H, DK, DV), np.float64)

    def copy(self):
        c = GdnState.__new__(GdnState)
        c.hist, c.S = self.hist.copy(), self.S.copy()
        return c


def gdn_forward(rows, params, state, H=16, DK=128, DV=128, gnorm=True, chunk=0):
    """One sequence, one layer: rows [T][stride] f32 -> out [T][H*DV] f32; state updated in place."""
    T, stride = rows.shape
    out = np.zeros((T, H * DV), np.float32)
    gw = np.ascontiguousarray(params["gnorm"], np.float32) if gnorm else None
    rc = lib().orc_gdn_forward(T, H, DK, DV, params["conv"].shape[1], stride, np.ascontiguousarray(rows, np.float32),
                               np.ascontiguousarray(params["conv"], np.float32),
                               np.ascontiguousarray(params["neg_exp_A"], np.float32),
                               np.ascontiguousarray(params["dt_bias"], np.float32),
                               gw.ctypes.data if gw is not None else None, state.hist, state.S, out, chunk)
    assert rc == 0
    return out


class GqaCache:
    """Per-sequence K/V cache [HK][LT][HD] (f32 holding f16-representable values when f16=1)."""

    def __init__(self, LT, HK=2, HD=256):
        self.K = np.zeros((HK, LT, HD), np.float32)
        self.V = np.zeros((HK, LT, HD), np.float32)
        self.P = 0


def gqa_forward(rows, params, cache, rope, HQ=8, HK=2, HD=256, RD=64, f16=True):
    """One sequence, one layer: rows [T][stride] (f16 or f32 values) -> out [T][HQ*HD] f32; appends to cache."""
    T, stride = rows.shape
    LT = cache.K.shape[1]
    out = np.zeros((T, HQ * HD), np.float32)
    rc = lib().orc_gqa_forward(T, cache.P, LT, HQ, HK, HD, RD, stride, np.ascontiguousarray(rows, np.float32),
                               np.ascontiguousarray(params["q_norm"], np.float32),
                               np.ascontiguousarray(params["k_norm"], np.float32), rope, cache.K, cache.V, out,
                               int(f16))
    assert rc == 0
    cache.P += T
    return out


def rel_err(a, b):
    """max |a - b| / max |b|, the measure the reference's engine test page uses (engine/test.html:13)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    m = np.abs(b).max()
    return float(np.abs(a - b).max() / (m if m > 0 else 1.0))
