"""Writes the golden fixtures tests/golden/{gdn_tiny,gqa_tiny}.npz from the numpy brute force (brute.py).

The reference holds no vectors for this path (its layer dumps are not shipped and its Python driver needs a
package and weights that are not available), so the fixtures are produced by this project's own independent
fp64 restatement at tiny shapes and then pin the C oracle (tests/test_oracle.py). Run:
    python tests/golden/make_golden.py
"""
import os

import numpy as np

import brute

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    g = np.random.Generator(np.random.PCG64(np.random.SeedSequence([20261201, 1])))
    # gated-delta, H=2, DK=DV=8, conv 4; a continuation call checks the carried hist / state
    H, DK, DV, KC = 2, 8, 8, 4
    C = 2 * H * DK + H * DV
    stride = C + H * DV + 2 * H + 3  # padded like the engine's 8256
    rows1 = g.standard_normal((7, stride)).astype(np.float32)
    rows2 = g.standard_normal((4, stride)).astype(np.float32)
    conv = (0.5 * g.standard_normal((C, KC))).astype(np.float32)
    negA = (-np.exp(g.standard_normal(H) * 0.5)).astype(np.float32)
    dtb = (0.3 * g.standard_normal(H)).astype(np.float32)
    gnorm = (1 + 0.1 * g.standard_normal(DV)).astype(np.float32)
    out1, hist1, S1 = brute.gdn(rows1, conv, negA, dtb, gnorm, H, DK, DV)
    out2, hist2, S2 = brute.gdn(rows2, conv, negA, dtb, gnorm, H, DK, DV, hist1, S1)
    raw1, _, _ = brute.gdn(rows1, conv, negA, dtb, None, H, DK, DV)
    np.savez(os.path.join(HERE, "gdn_tiny.npz"), H=H, DK=DK, DV=DV, rows1=rows1, rows2=rows2, conv=conv, negA=negA,
             dtb=dtb, gnorm=gnorm, out1=out1, out2=out2, raw1=raw1, hist2=hist2, S2=S2)
    # gated GQA, HQ=4, HK=2, HD=16, RD=8, theta 1e4; a continuation at P=6
    HQ, HK, HD, RD, theta = 4, 2, 16, 8, 1e4
    stride = HQ * 2 * HD + 2 * HK * HD + 5
    rows1 = g.standard_normal((6, stride)).astype(np.float32)
    rows2 = g.standard_normal((3, stride)).astype(np.float32)
    qw = (1 + 0.2 * g.standard_normal(HD)).astype(np.float32)
    kw = (1 + 0.2 * g.standard_normal(HD)).astype(np.float32)
    o1, K1, V1 = brute.gqa(rows1, qw, kw, HQ, HK, HD, RD, theta)
    o2, K2, V2 = brute.gqa(rows2, qw, kw, HQ, HK, HD, RD, theta, K1, V1, P=6)
    np.savez(os.path.join(HERE, "gqa_tiny.npz"), HQ=HQ, HK=HK, HD=HD, RD=RD, theta=theta, rows1=rows1, rows2=rows2,
             qw=qw, kw=kw, out1=o1, out2=o2, K=K2, V=V2)


if __name__ == "__main__":
    main()
