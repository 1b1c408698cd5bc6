"""PyTorch CPU fp32 restatement of the hybrid-attention path: the CPU baseline that bench.py times next to the GPU.

Test and benchmark infrastructure only (only tests/ and bench.py's CPU-baseline leg import it); no product path
uses it. It states the same semantics as the reference's fp32 path in plain torch ops on the CPU, batched over
sequences and heads, the way the Hugging Face CPU path runs a prefill:

  gated-delta layer (web/public/engine/wgsl.js:124-187 + 252-268; transformers qwen3_5 torch_causal_conv1d_update,
  torch_chunk_gated_delta_rule and the gated RMSNorm): depthwise causal conv1d (kernel 4, F.conv1d with
  groups = C) + SiLU over the q/k/v channels; q, k l2-normalised (eps 1e-6, q also by 1/sqrt(d_k)); beta =
  sigmoid(b); g = negA * softplus(a + dt_bias); the chunked WY form with chunk 64 (A strictly lower, T = (I + A)^-1
  by a triangular solve, W = T diag(beta e^gc) k, U = T diag(beta) v, then the chunk recurrence on the 128 x 128
  state); y = gnorm_w * o * rsqrt(mean(o^2) + 1e-6) * SiLU(z).

  GQA layer (wgsl.js:271-302, 348-417): q/k RMSNorm times the stored (1 + w), rotate-half RoPE on dims [0, 64)
  at base 1e7, causal softmax attention in fp32 with scale 1/sqrt(256) (explicit masked scores), four query
  heads per KV head, output times sigmoid(gate).

Row layouts are the engine's fused rows (engine.js:264-274): linear rows q | k | v | z | a | b, full rows
[q | gate] x HQ | k x HK | v x HK. tests/test_torch_baseline.py checks both layers against the fp64 C oracle.
"""
import math

import torch
import torch.nn.functional as F


def gdn_layer(rows, conv_w, negA, dt_bias, gnorm_w, H=16, DK=128, DV=128, chunk=64):
    """rows [B][T][stride] fp32 -> (y [B][T][H*DV], S [B][H][DK][DV]); a fresh context (zero state and history)."""
    B, T, _ = rows.shape
    C = 2 * H * DK + H * DV
    x = rows[..., :C].transpose(1, 2)  # [B][C][T]
    u = F.silu(F.conv1d(F.pad(x, (conv_w.shape[1] - 1, 0)), conv_w.unsqueeze(1), groups=C)).transpose(1, 2)
    q = u[..., :H * DK].reshape(B, T, H, DK)
    k = u[..., H * DK:2 * H * DK].reshape(B, T, H, DK)
    v = u[..., 2 * H * DK:C].reshape(B, T, H, DV)
    q = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6) * (1.0 / math.sqrt(DK))
    k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    z = rows[..., C:C + H * DV].reshape(B, T, H, DV)
    a = rows[..., C + H * DV:C + H * DV + H]
    b = rows[..., C + H * DV + H:C + H * DV + 2 * H]
    beta = torch.sigmoid(b)
    g = negA * F.softplus(a + dt_bias)  # threshold 20, as F.softplus and the reference

    # chunked form: [B][H][N][64][...], rows past T padded with zero contributions
    N = (T + chunk - 1) // chunk
    pad = N * chunk - T

    def chunks(t, d):
        t = t.permute(0, 2, 1, 3) if d else t.permute(0, 2, 1)
        t = F.pad(t, (0, 0, 0, pad) if d else (0, pad))
        return t.reshape(B, H, N, chunk, -1) if d else t.reshape(B, H, N, chunk)

    qc, kc, vc = chunks(q, 1), chunks(k, 1), chunks(v, 1)
    bc, gc = chunks(beta, 0), chunks(g, 0).cumsum(-1)
    dec = (gc.unsqueeze(-1) - gc.unsqueeze(-2))  # gc_t - gc_t'
    lower = torch.tril(torch.ones(chunk, chunk, dtype=torch.bool), -1)
    causal = torch.tril(torch.ones(chunk, chunk, dtype=torch.bool))
    A = torch.where(lower, (bc.unsqueeze(-1) * (kc @ kc.transpose(-1, -2))) * dec.clamp(max=0).exp(),
                    torch.zeros((), dtype=rows.dtype))
    eye = torch.eye(chunk, dtype=rows.dtype)
    Tm = torch.linalg.solve_triangular(eye + A, eye.expand_as(A), upper=False)
    eg = gc.exp()
    W = Tm @ (kc * (bc * eg).unsqueeze(-1))
    U = Tm @ (vc * bc.unsqueeze(-1))
    att = torch.where(causal, (qc @ kc.transpose(-1, -2)) * dec.clamp(max=0).exp(), torch.zeros((), dtype=rows.dtype))
    S = torch.zeros(B, H, DK, DV, dtype=rows.dtype)
    out = torch.empty(B, H, N, chunk, DV, dtype=rows.dtype)
    for n in range(N):
        vn = U[:, :, n] - W[:, :, n] @ S
        out[:, :, n] = (qc[:, :, n] * eg[:, :, n].unsqueeze(-1)) @ S + att[:, :, n] @ vn
        gl = gc[:, :, n, -1]
        kd = kc[:, :, n] * (gl.unsqueeze(-1) - gc[:, :, n]).exp().unsqueeze(-1)
        S = S * gl.exp()[..., None, None] + kd.transpose(-1, -2) @ vn
    o = out.reshape(B, H, N * chunk, DV)[:, :, :T].permute(0, 2, 1, 3)  # [B][T][H][DV]
    y = gnorm_w * o * torch.rsqrt((o * o).mean(-1, keepdim=True) + 1e-6) * F.silu(z)
    return y.reshape(B, T, H * DV), S


def rope_table(LT, RD=64, theta=1e7):
    """cos/sin [LT][RD/2], angles t / theta^(2i/RD) computed in f64 (engine.js:105-106)."""
    t = torch.arange(LT, dtype=torch.float64).unsqueeze(1)
    inv = theta ** (-torch.arange(0, RD, 2, dtype=torch.float64) / RD)
    ang = t * inv
    return ang.cos().float(), ang.sin().float()


def gqa_layer(rows, q_norm, k_norm, cos, sin, HQ=8, HK=2, HD=256, RD=64):
    """rows [B][T][stride] (any float dtype; computed in fp32) -> out [B][T][HQ*HD] fp32, positions 0..T-1."""
    rows = rows.float()
    B, T, _ = rows.shape
    qg = rows[..., :HQ * 2 * HD].reshape(B, T, HQ, 2, HD)
    q, gate = qg[..., 0, :], qg[..., 1, :]
    k = rows[..., HQ * 2 * HD:HQ * 2 * HD + HK * HD].reshape(B, T, HK, HD)
    v = rows[..., HQ * 2 * HD + HK * HD:HQ * 2 * HD + 2 * HK * HD].reshape(B, T, HK, HD)

    def norm_rope(x, w):
        x = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w
        c, s = cos[:T].view(1, T, 1, RD // 2), sin[:T].view(1, T, 1, RD // 2)
        x1, x2 = x[..., :RD // 2], x[..., RD // 2:RD]
        return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s, x[..., RD:]], -1)

    q = norm_rope(q, q_norm).permute(0, 2, 1, 3)  # [B][HQ][T][HD]
    k = norm_rope(k, k_norm).permute(0, 2, 1, 3)  # [B][HK][T][HD]
    v = v.permute(0, 2, 1, 3)
    rep = HQ // HK
    mask = torch.triu(torch.ones(T, T, dtype=torch.bool), 1)
    out = torch.empty(B, HQ, T, HD)
    for h in range(HQ):  # one query head at a time keeps the score matrix at B x T x T
        s = (q[:, h] @ k[:, h // rep].transpose(-1, -2)) * (1.0 / math.sqrt(HD))
        s = s.masked_fill(mask, float("-inf"))
        out[:, h] = torch.softmax(s, -1) @ v[:, h // rep]
    out = out.permute(0, 2, 1, 3) * torch.sigmoid(gate)
    return out.reshape(B, T, HQ * HD)
