"""Independent numpy restatement of the path's semantics, for tiny shapes. TEST INFRASTRUCTURE ONLY.

Written from the mathematics (and the reference's equations, web/public/engine/wgsl.js:124-187, 252-302,
348-417), not from the C oracle, so that a mistake in either one shows up as a mismatch. Loops over tokens;
dense numpy inside a token. fp64 throughout.
"""
import numpy as np


def silu(x):
    return x / (1.0 + np.exp(-x))


def softplus(x):
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def gdn(rows, conv, negA, dtb, gnorm, H, DK, DV, hist=None, S=None):
    """rows [T][stride] -> (out [T][H*DV], hist', S'); gnorm None gives the raw o."""
    rows = np.asarray(rows, np.float64)
    T = rows.shape[0]
    C = 2 * H * DK + H * DV
    KC = conv.shape[1]
    hist = np.zeros((KC - 1, C)) if hist is None else np.asarray(hist, np.float64)
    S = np.zeros((H, DK, DV)) if S is None else np.array(S, np.float64)
    x = np.concatenate([hist, rows[:, :C]], 0)  # [KC-1+T][C]
    # conv: tap j multiplies x[t - (KC-1) + j]; the last tap is the current row (F.conv1d(pad=KC-1)[:T])
    u = np.stack([sum(conv[:, j] * x[t + j] for j in range(KC)) for t in range(T)])
    u = silu(u)
    aoff, boff, zoff = C + H * DV, C + H * DV + H, C
    out = np.zeros((T, H * DV))
    for t in range(T):
        for h in range(H):
            q = u[t, h * DK:(h + 1) * DK]
            k = u[t, H * DK + h * DK:H * DK + (h + 1) * DK]
            v = u[t, 2 * H * DK + h * DV:2 * H * DK + (h + 1) * DV]
            q = q / np.sqrt(q @ q + 1e-6) / np.sqrt(DK)
            k = k / np.sqrt(k @ k + 1e-6)
            beta = 1.0 / (1.0 + np.exp(-rows[t, boff + h]))
            alpha = np.exp(negA[h] * softplus(rows[t, aoff + h] + dtb[h]))
            S[h] = alpha * S[h]
            delta = beta * (v - S[h].T @ k)
            S[h] = S[h] + np.outer(k, delta)
            o = S[h].T @ q
            if gnorm is not None:
                z = rows[t, zoff + h * DV:zoff + (h + 1) * DV]
                o = gnorm * o / np.sqrt(np.mean(o * o) + 1e-6) * silu(z)
            out[t, h * DV:(h + 1) * DV] = o
    return out, x[-(KC - 1):].copy(), S


def rope_rotate(x, pos, RD, theta):
    """rotate-half RoPE on dims [0, RD) of x [..., HD] at integer position pos."""
    y = x.copy()
    i = np.arange(RD // 2)
    ang = pos / theta ** (2.0 * i / RD)
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[..., :RD // 2], x[..., RD // 2:RD]
    y[..., :RD // 2] = a * c - b * s
    y[..., RD // 2:RD] = b * c + a * s
    return y


def gqa(rows, qw, kw, HQ, HK, HD, RD, theta, Kc=None, Vc=None, P=0):
    """rows [T][stride] -> (out [T][HQ*HD], K [HK][P+T][HD], V); Kc/Vc hold P cached rows (post-norm/rope)."""
    rows = np.asarray(rows, np.float64)
    T = rows.shape[0]
    G = HQ // HK
    K = np.zeros((HK, P + T, HD)) if Kc is None else np.concatenate([Kc[:, :P], np.zeros((HK, T, HD))], 1)
    V = np.zeros((HK, P + T, HD)) if Vc is None else np.concatenate([Vc[:, :P], np.zeros((HK, T, HD))], 1)

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x) + 1e-6) * w

    Q = np.zeros((HQ, T, HD))
    for t in range(T):
        r = rows[t]
        for h in range(HQ):
            Q[h, t] = rope_rotate(rms(r[h * 2 * HD:h * 2 * HD + HD], qw), P + t, RD, theta)
        for kh in range(HK):
            K[kh, P + t] = rope_rotate(rms(r[HQ * 2 * HD + kh * HD:HQ * 2 * HD + (kh + 1) * HD], kw), P + t, RD, theta)
            V[kh, P + t] = r[HQ * 2 * HD + HK * HD + kh * HD:HQ * 2 * HD + HK * HD + (kh + 1) * HD]
    out = np.zeros((T, HQ * HD))
    for h in range(HQ):
        kh = h // G
        s = Q[h] @ K[kh].T / np.sqrt(HD)  # [T][P+T]
        mask = np.arange(P + T)[None, :] > (P + np.arange(T))[:, None]
        s[mask] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        o = p @ V[kh]
        gate = rows[:, h * 2 * HD + HD:h * 2 * HD + 2 * HD]
        out[:, h * HD:(h + 1) * HD] = o / (1.0 + np.exp(-gate))
    return out, K, V
