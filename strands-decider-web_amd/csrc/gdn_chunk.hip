// Chunked gated-delta prefill (ha_recurrence HA_CHUNKED), gfx950.
//
// Same semantics as the sequential rule (reference web/public/engine/wgsl.js:124-187 + 252-268), evaluated in the
// chunked WY/UT form the reference's fp32 driver uses for prefill (transformers qwen3_5
// torch_chunk_gated_delta_rule; Yang et al. 2024, "Parallelizing Linear Transformers with the Delta Rule over
// Sequence Length"; Yang, Kautz & Hatamizadeh, "Gated Delta Networks"). For a chunk of 64 rows with cumulative
// log-decay gc (gc_t = sum_{s<=t} g_s inside the chunk) and the state S at the chunk start:
//   A   = strictly_lower(beta_t (k^_t . k^_t') exp(gc_t - gc_t'))      T = (I + A)^-1
//   U   = T diag(beta) v      V_new = U - T diag(beta e^gc) (k^ S)     (that is U - W S, W never formed)
//   o_t = exp(gc_t) q^_t S + sum_{t'<=t} (q^_t . k^_t') exp(gc_t - gc_t') V_new_t'
//   S  <- exp(gc_63) S + k^T diag(exp(gc_63 - gc)) V_new                 (complete chunks only)
//
// One workgroup of 8 waves per (sequence, head) walks the chunks in order, as a two-stage pipeline:
//   consumer waves 0..3 each own 32 value columns of the fp32 state, held in MFMA accumulator registers for the
//     whole call, and do chunk p's state-dependent work: q^ S, k^ S, V_new, o, the state update and the gated
//     RMSNorm epilogue (GNORM);
//   producer waves 4..7 meanwhile run chunk p+1's q/k conv (4 taps) + SiLU + l2 norm in registers from raw rows
//     fetched a chunk ahead, and one of them turns the a/b columns into the gate vectors.
// Per period p the workgroup passes five barriers:
//   A: consumers chunk p  |  producers conv(p+1), prefetch raw q/k rows of p+2
//   B: consumers store chunk p's output  |  producers write q^, k^, k^T of p+1 and the gate vectors to LDS
//   C: all waves: K K^T and Q K^T of p+1 on v_mfma_f32_16x16x32_f16 -> A (fp32) and the decay-masked scores
//   D: one producer solves the diagonal 16x16 blocks of T = (I + A)^-1  |  consumers: v conv(p+1), first half
//   E: three producers own one block column each of T's off-diagonal blocks (fp32 MFMA 16x16x4, no barrier
//      between block rows)  |  consumers: v conv(p+1), second half
// so the VALU-heavy conv overlaps the MFMA-heavy state work instead of following it. A tile is written only in a
// segment after its last reader of the previous chunk, so every LDS tile is single-buffered.
// Chunk boundaries sit at s0 + 64k, so a row is processed identically however a sequence is split into calls;
// only complete chunks advance the stored state.
//
// MFMA operand convention used below (16x16xK): lane l supplies row (l & 15) of A and column (l & 15) of B, and
// lane group l >> 4 supplies a block of the K index; any assignment of K indices to (lane group, element) works
// as long as A and B use the same one. The result D holds rows 4 (l >> 4) + e, e < 4, of column l & 15. That
// lets a D tile be reused as a B operand (K = its rows) without moving data between lanes: the matching A
// operand is read with the same "permuted" K order {32 kb + 4 grp + e} U {32 kb + 16 + 4 grp + e}.
#include "gdn_common.h"

namespace ha {
namespace {

constexpr int kNW = 8, kNT = 64 * kNW;
constexpr int kNC = 4;        // consumer waves (0..3), 32 value columns each; producers are waves 4..7
constexpr int kGW = kNW - 1;  // the producer that computes the gate vectors and the diagonal blocks of T
constexpr int kSP = 36;       // row pitch (floats) of a consumer's output staging area (16 rows x 32 columns)
constexpr int kRG = 8;        // rows per conv lane

struct Lds {
  _Float16 Qs[kCH * kQP];   // q^ / sqrt(DK), [t][i]
  _Float16 Ks[kCH * kQP];   // k^, [t][i]
  _Float16 KT[kDK * kTP];   // k^ transposed, [i][t], 8-column groups swizzled by kt16
  _Float16 VT[kDV * kTP];   // v transposed, [j][t], 8-column groups swizzled by vt16
  _Float16 Tb[kCH * kTP];   // T diag(beta), f16, [t][t']
  _Float16 Tw[kCH * kTP];   // T diag(beta e^gc), f16
  _Float16 Att[kCH * kTP];  // decay-masked causal q^ k^T, [t][t']
  float Tm[kCH * kAP];      // A, then T, fp32; the consumers' output staging area while the producers convolve
  // this head's conv taps, laid out so that the 32 conv lanes of a half wave read consecutive 16-byte entries:
  // q/k channel 8 g + c (g < 32: q then k) at cwq[c][g], v channel 4 g + c at cwv[c][g]
  float cwq[8][32][kKC];
  float cwv[4][32][kKC];
  float gc[kCH];            // cumulative log decay inside the chunk
  float eg[kCH];            // e^gc
  float bt[kCH];            // beta
  float ed[kCH];            // e^(gc_63 - gc)
  float rowf[kCH];          // e^(gc_t - gc_16(t/16)), in (0, 1]
  float brow[kCH];          // beta_t rowf_t
  float colf[3][kCH];       // colf[i-1][t'] = e^(gc_16i - gc_t') for t' < 16 i, in (0, 1]
  float red[kCH * kNC];     // gated-norm partial sums, [t][consumer]
  float inv[kNC][kCH];      // per-consumer copy of the row inverse norms
};
static_assert(sizeof(float) * kCH * kAP >= kNC * 16 * kSP * sizeof(float), "staging area");

template <typename T>
__global__ __launch_bounds__(512) void gdn_chunk_kernel(GdnArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  Lds& sm = *reinterpret_cast<Lds*>(lds_raw);
  const int b = blockIdx.x / a.H, h = blockIdx.x % a.H;
  const int tid0 = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  const bool consumer = w < kNC;
  const int end = a.P + a.L;
  const int nchunks = (a.L + (a.P - a.s0) + kCH - 1) / kCH;
  const float qscale = 0.08838834764831845f;  // 1/sqrt(128)
  const unsigned rowb = (unsigned)a.stride * sizeof(T);      // bytes per input row
  const unsigned orowb = (unsigned)(a.H * kDV) * sizeof(T);  // bytes per output row
  const char* const seq_in = (const char*)a.in + (size_t)b * a.L * rowb;  // row P of this sequence

  const size_t sbase = ((size_t)b * a.H + h) * kDK * kDV;

  // this head's conv taps: local channel q 0..127, k 128..255, v 256..383
  for (int i = tid0; i < 3 * 128 * kKC; i += kNT) {
    const int lc = i / kKC, j = i % kKC;
    const int ch = lc < 128 ? h * kDK + lc : lc < 256 ? a.H * kDK + h * kDK + (lc - 128) : 2 * a.H * kDK + h * kDV + (lc - 256);
    const float v = gp<float>(a.conv_w)[(size_t)ch * kKC + j];
    if (lc < 256)
      sm.cwq[lc & 7][lc >> 3][j] = v;
    else
      sm.cwv[(lc - 256) & 3][(lc - 256) >> 2][j] = v;
  }
  // blocks above the diagonal of the f16 T and score tiles are read by full 32-wide K blocks and never written
  for (int idx = tid0; idx < kCH * kCH; idx += kNT) {
    const int t = idx >> 6, tp = idx & 63;
    if ((tp >> 4) > (t >> 4)) {
      sm.Tb[t * kTP + tp] = (_Float16)0.0f;
      sm.Tw[t * kTP + tp] = (_Float16)0.0f;
      sm.Att[t * kTP + tp] = (_Float16)0.0f;
    }
  }
  const float na = gp<float>(a.negA)[h], db = gp<float>(a.dtb)[h];
  const int aoff = a.C + a.H * kDV + h, boff = aoff + a.H;

  // raw rows: producers hold q/k rows (11 rows x 8 channels) of the chunk they convolve next, consumers v rows
  // (11 rows x 4 channels); the gate producer also holds that chunk's a/b inputs
  float xq[kRG + kKC - 1][8], xv[kRG + kKC - 1][4], ga = 0.0f, gb = 0.0f;

  // Loads rows cs-3 .. cs+63 of the chunk starting at cs: lane rows 8 rg - 3 .. 8 rg + 7 of the chunk, at column
  // offset `col` (element) of the row, `n` channels. Uniform row bases and 32-bit lane offsets when no row is a
  // replay row or past the end; per-lane row pointers otherwise. Rows past the end repeat the last row: they only
  // feed conv outputs past the end, which are masked.
  const RowSrc src = row_src(a);
  auto fetch_rows = [&](int cs, int rg, int col, auto& x, auto nch) {
    constexpr int N = decltype(nch)::value;
    if (cs - (kKC - 1) >= a.P && cs + kCH <= end) {
      const char* base = seq_in + (ptrdiff_t)(cs - (kKC - 1) - a.P) * rowb;
      const unsigned off = (unsigned)(kRG * rg) * rowb + (unsigned)col * (unsigned)sizeof(T);
#pragma unroll
      for (int i = 0; i < kRG + kKC - 1; i++) {
        const char* rb = base + (size_t)i * rowb;
        if constexpr (N == 8)
          load8(gp<T>(rb + off), x[i]);
        else
          load4(gp<T>(rb + off), x[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kRG + kKC - 1; i++) {
        const int r = cs + kRG * rg - (kKC - 1) + i, rc = min(r, end - 1);
        const gptr<T> row = row_of<T>(a, src, b, rc) + col;
        if constexpr (N == 8)
          load8(row, x[i]);
        else
          load4(row, x[i]);
      }
    }
  };
  // producer lane pt = tid - 256: rows 8 (pt / 32) .., channels 8 (pt % 16) of q (pt % 32 < 16) or k
  auto fetch_qk = [&](int cs) {
    const int pt = opaque(tid0) - 64 * kNC, rg = pt >> 5, cgi = pt & 31, qk = cgi >> 4, cg = cgi & 15;
    fetch_rows(cs, rg, (qk ? a.H * kDK : 0) + h * kDK + 8 * cg, xq, Width<8>{});
    if (w == kGW) {
      const int lane = pt & 63;
      // rows past the end: their gates are never used (the gate lanes mask them)
      const gptr<T> grow = cs >= a.P && cs + kCH <= end ? gp<T>(seq_in + (size_t)(cs - a.P + lane) * rowb)
                                                         : row_of<T>(a, src, b, min(cs + lane, end - 1));
      ga = (float)grow[aoff];
      gb = (float)grow[boff];
    }
  };
  // consumer lane ct = tid: rows 8 (ct / 32) .., v channels 4 (ct % 32)
  auto fetch_v = [&](int cs) {
    const int ct = opaque(tid0), rg = ct >> 5, cvg = ct & 31;
    fetch_rows(cs, rg, 2 * a.H * kDK + h * kDV + 4 * cvg, xv, Width<4>{});
  };

  // producer: normalized conv outputs of the chunk being prepared, rows 8 rg + r, channels 8 cg + c
  float uq[kRG][8];
  float gcr = 0.0f, btr = 0.0f;
  auto produce_conv = [&](int cs) {
    const int pt = opaque(tid0) - 64 * kNC, rg = pt >> 5, cgi = pt & 31, qk = cgi >> 4;
    const int m = min(kCH, end - cs);
    float ss[kRG];
#pragma unroll
    for (int r = 0; r < kRG; r++) ss[r] = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const f4 wc = lds4(sm.cwq[c][cgi]);
#pragma unroll
      for (int r = 0; r < kRG; r++) {
        float sv = wc[0] * xq[r][c];
        sv = fmaf(wc[1], xq[r + 1][c], sv);
        sv = fmaf(wc[2], xq[r + 2][c], sv);
        sv = fmaf(wc[3], xq[r + 3][c], sv);
        uq[r][c] = kRG * rg + r < m ? silu(sv) : 0.0f;
        ss[r] = fmaf(uq[r][c], uq[r][c], ss[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < kRG; r++) {
      const float rs = rsqrtf(row_sum16(ss[r]) + 1e-6f) * (qk ? 1.0f : qscale);
#pragma unroll
      for (int c = 0; c < 8; c++) uq[r][c] *= rs;
    }
  };
  // gate producer: beta and the cumulative log decay of the chunk at cs from its a/b inputs (lane = row)
  auto produce_gates = [&](int cs) {
    const int lane = opaque(tid0) & 63;
    const int m = min(kCH, end - cs);
    gcr = 0.0f;
    btr = 0.0f;
    if (lane < m) {
      btr = __builtin_amdgcn_rcpf(1.0f + __expf(-gb));
      const float xs = ga + db;
      gcr = na * (xs > 20.0f ? xs : log1pf(__expf(xs)));
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float o = __shfl_up(gcr, d);
      if (lane >= d) gcr += o;
    }
  };
  auto produce_write = [&]() {
    const int pt = opaque(tid0) - 64 * kNC, rg = pt >> 5, cgi = pt & 31, qk = cgi >> 4, cg = cgi & 15;
#pragma unroll
    for (int r = 0; r < kRG; r++) {
      h8 hv;
#pragma unroll
      for (int c = 0; c < 8; c++) hv[c] = (_Float16)uq[r][c];
      *reinterpret_cast<h8*>((qk ? sm.Ks : sm.Qs) + (kRG * rg + r) * kQP + 8 * cg) = hv;
    }
    if (qk) {
#pragma unroll
      for (int c = 0; c < 8; c++) {
        h8 kt;
#pragma unroll
        for (int r = 0; r < kRG; r++) kt[r] = (_Float16)uq[r][c];
        *reinterpret_cast<h8*>(sm.KT + kt16(8 * cg + c, rg)) = kt;
      }
    }
    if (w == kGW) {
      const int lane = pt & 63;
      const float gl = __shfl(gcr, 63);
      const float rf = __expf(gcr - __shfl(gcr, lane & ~15));
      sm.gc[lane] = gcr;
      sm.eg[lane] = __expf(gcr);
      sm.bt[lane] = btr;
      sm.ed[lane] = __expf(gl - gcr);
      sm.rowf[lane] = rf;
      sm.brow[lane] = btr * rf;
#pragma unroll
      for (int i = 1; i < 4; i++) {
        const float gi = __shfl(gcr, 16 * i);
        sm.colf[i - 1][lane] = lane < 16 * i ? __expf(gi - gcr) : 0.0f;
      }
    }
  };
  // consumer: v conv of rows 8 rg + r0 .. r0 + 3 of the chunk at cs -> v^T (8 bytes per channel)
  auto consume_vconv = [&](int cs, int r0) {
    const int ct = opaque(tid0), rg = ct >> 5, cvg = ct & 31;
    const int m = min(kCH, end - cs);
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const f4 wc = lds4(sm.cwv[c][cvg]);
      h4 vt;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        float sv = wc[0] * xv[r0 + r][c];
        sv = fmaf(wc[1], xv[r0 + r + 1][c], sv);
        sv = fmaf(wc[2], xv[r0 + r + 2][c], sv);
        sv = fmaf(wc[3], xv[r0 + r + 3][c], sv);
        vt[r] = (_Float16)(kRG * rg + r0 + r < m ? silu(sv) : 0.0f);
      }
      *reinterpret_cast<h4*>(sm.VT + vt16(4 * cvg + c, rg) + r0) = vt;
    }
  };

  // One 16x16 tile of K K^T -> A (fp32) or Q K^T -> decay-masked scores (f16) of the chunk in Qs / Ks; tile jt of
  // the 10 on or below the diagonal (row block ti, column block tj)
  auto kkt_qkt_tile = [&](bool isq, int jt, int grp, int c16) {
    {
      const int ti = jt >= 6 ? 3 : jt >= 3 ? 2 : jt >= 1 ? 1 : 0;
      const int tj = jt - ti * (ti + 1) / 2;
      const _Float16* ab = (isq ? sm.Qs : sm.Ks) + (16 * ti + c16) * kQP + 8 * grp;
      const _Float16* bb = sm.Ks + (16 * tj + c16) * kQP + 8 * grp;
      f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 4; ks++)
        acc = mfma16(*reinterpret_cast<const h8*>(ab + 32 * ks), *reinterpret_cast<const h8*>(bb + 32 * ks), acc);
      const int tp = 16 * tj + c16, t0 = 16 * ti + 4 * grp;
      if (ti != tj) {
        // below the diagonal blocks gc_t <= gc_16ti <= gc_t', so e^(gc_t - gc_t') factors into two terms <= 1
        const float cf = sm.colf[ti - 1][tp];
        if (!isq) {
          const f4 bf = lds4(&sm.brow[t0]);
#pragma unroll
          for (int e = 0; e < 4; e++) sm.Tm[(t0 + e) * kAP + tp] = acc[e] * bf[e] * cf;
        } else {
          const f4 rf = lds4(&sm.rowf[t0]);
#pragma unroll
          for (int e = 0; e < 4; e++) sm.Att[(t0 + e) * kTP + tp] = (_Float16)(acc[e] * rf[e] * cf);
        }
      } else {
        const float gp_ = sm.gc[tp];
        const f4 gt = lds4(&sm.gc[t0]), bt = lds4(&sm.bt[t0]);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int t = t0 + e;
          const float dec = __expf(fminf(gt[e] - gp_, 0.0f));
          if (!isq)
            sm.Tm[t * kAP + tp] = tp < t ? bt[e] * acc[e] * dec : 0.0f;
          else
            sm.Att[t * kTP + tp] = (_Float16)(tp <= t ? acc[e] * dec : 0.0f);
        }
      }
    }
  };
  // The 16 tiles other than the diagonal blocks of A, over waves 0..6 (the gate producer does the diagonal blocks
  // of A itself, right before solving them)
  auto kkt_qkt = [&](int grp, int c16) {
    for (int j = w; j < 16; j += kNW - 1) {
      const int off[6] = {1, 3, 4, 6, 7, 8};  // below-diagonal tiles of A
      if (j < 6)
        kkt_qkt_tile(false, off[j], grp, c16);
      else
        kkt_qkt_tile(true, j - 6, grp, c16);
    }
  };

  __syncthreads();  // conv taps and zero blocks visible

  // The two roles run separate loops with the same barrier sequence (the role is uniform per wave, and every
  // condition that skips a barrier depends only on p and nchunks), so each loop keeps only its own registers live.
  if (consumer) {
    // ---- consumer state: S[ct][it][e] = S[16 it + 4 grp + e][32 w + 16 ct + c16] ----
    f4 S[2][8];
    {
      const int g0 = (tid0 & 63) >> 4, l16 = tid0 & 15;
#pragma unroll
      for (int ct = 0; ct < 2; ct++)
#pragma unroll
        for (int it = 0; it < 8; it++)
#pragma unroll
          for (int e = 0; e < 4; e++)
            S[ct][it][e] = a.S_in ? gp<float>(a.S_in)[sbase + (size_t)(16 * it + 4 * g0 + e) * kDV + 32 * w + 16 * ct + l16]
                                  : 0.0f;
    }
    // consumer epilogue layout: lane l holds rows 8 q + l / 8 (q < 8) of columns 32 w + 4 (l % 8) .. +3
    f4 gw = {1.0f, 1.0f, 1.0f, 1.0f};
    if (a.gnorm) gw = ld4(gp<float>(a.gnorm) + 32 * w + 4 * (tid0 & 7));
    // Drain these loads here: the compiler's wait counting merges the loop's entry state into every period, so a
    // state load still outstanding at the loop head would make each period's first use of S wait for every
    // global access issued before it (the previous chunk's output stores included).
    __builtin_amdgcn_s_waitcnt(0);
    f4 Y[8], zq[8];
    // period p: chunk p (p >= 0) here, chunk p + 1 (p + 1 < nchunks) on the producers
    for (int p = -1; p < nchunks; p++) {
      const int c0 = a.s0 + kCH * p, c1 = c0 + kCH;
      const int m = min(kCH, end - c0);
      const bool full = m == kCH;
      const bool plain = c0 >= a.P && full;  // no replay rows, no rows past the end
      const int tid = opaque(tid0), lane = tid & 63, grp = lane >> 4, c16 = lane & 15;
      const int er = lane >> 3, ec = 32 * w + 4 * (lane & 7);  // epilogue row (within 8) and column

      // ---- A: chunk p ----
      if (p >= 0) {
          // k^ S (K block outermost: only that block's f16 copy of S is live at a time); q^ S comes after V_new,
          // so the two never hold their accumulators at the same time
          f4 O[2][4], Vn[2][4];
          h8 KSb[2][2];
          {
            f4 KS[2][4];
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
              h8 S16[2];
#pragma unroll
              for (int ct = 0; ct < 2; ct++) S16[ct] = pack_b(S[ct][2 * kb], S[ct][2 * kb + 1]);
#pragma unroll
              for (int ti = 0; ti < 4; ti++) {
                const h8 ka = perm_a(sm.Ks, kQP, 16 * ti + c16, kb, grp);
#pragma unroll
                for (int ct = 0; ct < 2; ct++) {
                  const f4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};
                  KS[ct][ti] = mfma16(ka, S16[ct], kb ? KS[ct][ti] : z4);
                }
              }
            }
#pragma unroll
            for (int ct = 0; ct < 2; ct++) {
              KSb[ct][0] = pack_b(KS[ct][0], KS[ct][1]);
              KSb[ct][1] = pack_b(KS[ct][2], KS[ct][3]);
            }
          }
          // z of this chunk for the epilogue, in flight behind the rest of the chunk's MFMA work (one load site:
          // rows outside [P, P + L) are clamped, their outputs are not stored)
          if (plain) {
            const char* zb = seq_in + (size_t)(c0 - a.P) * rowb + (a.C + h * kDV) * sizeof(T);
            const unsigned oz = (unsigned)er * rowb + ec * (unsigned)sizeof(T);
#pragma unroll
            for (int q = 0; q < 8; q++) zq[q] = ld4(gp<T>(zb + (size_t)(8 * q) * rowb + oz));
          } else {
            const gptr<T> zb = gp<T>(seq_in) + a.C + h * kDV + ec;
#pragma unroll
            for (int q = 0; q < 8; q++) {
              const int rr = min(max(c0 + 8 * q + er - a.P, 0), a.L - 1);
              zq[q] = ld4(zb + (size_t)rr * a.stride);
            }
          }
          // V_new = T diag(beta) v - T diag(beta e^gc) (k^ S)
#pragma unroll
          for (int ti = 0; ti < 4; ti++) {
            f4 u[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}}, ws[2] = {u[0], u[0]};
#pragma unroll
            for (int kb = 0; kb <= (ti >> 1); kb++) {
              const h8 tb = *reinterpret_cast<const h8*>(sm.Tb + (16 * ti + c16) * kTP + 32 * kb + 8 * grp);
              const h8 tw = perm_a(sm.Tw, kTP, 16 * ti + c16, kb, grp);
#pragma unroll
              for (int ct = 0; ct < 2; ct++) {
                const int col = 32 * w + 16 * ct + c16;
                u[ct] = mfma16(tb, *reinterpret_cast<const h8*>(sm.VT + vt16(col, 4 * kb + grp)), u[ct]);
                ws[ct] = mfma16(tw, KSb[ct][kb], ws[ct]);
              }
            }
#pragma unroll
            for (int ct = 0; ct < 2; ct++) Vn[ct][ti] = u[ct] - ws[ct];
          }
          // q^ S
#pragma unroll
          for (int kb = 0; kb < 4; kb++) {
            h8 S16[2];
#pragma unroll
            for (int ct = 0; ct < 2; ct++) S16[ct] = pack_b(S[ct][2 * kb], S[ct][2 * kb + 1]);
#pragma unroll
            for (int ti = 0; ti < 4; ti++) {
              const h8 qa = perm_a(sm.Qs, kQP, 16 * ti + c16, kb, grp);
#pragma unroll
              for (int ct = 0; ct < 2; ct++) {
                const f4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};
                O[ct][ti] = mfma16(qa, S16[ct], kb ? O[ct][ti] : z4);
              }
            }
          }
          // o = e^gc (q^ S) + scores V_new
#pragma unroll
          for (int ti = 0; ti < 4; ti++) {
            const f4 eg = lds4(&sm.eg[16 * ti + 4 * grp]);
#pragma unroll
            for (int ct = 0; ct < 2; ct++) O[ct][ti] *= eg;
          }
          {
            h8 Vb[2][2];
#pragma unroll
            for (int ct = 0; ct < 2; ct++) {
              Vb[ct][0] = pack_b(Vn[ct][0], Vn[ct][1]);
              Vb[ct][1] = pack_b(Vn[ct][2], Vn[ct][3]);
            }
#pragma unroll
            for (int ti = 0; ti < 4; ti++) {
              const h8 a0 = perm_a(sm.Att, kTP, 16 * ti + c16, 0, grp);
#pragma unroll
              for (int ct = 0; ct < 2; ct++) O[ct][ti] = mfma16(a0, Vb[ct][0], O[ct][ti]);
              if (ti >= 2) {
                const h8 a1 = perm_a(sm.Att, kTP, 16 * ti + c16, 1, grp);
#pragma unroll
                for (int ct = 0; ct < 2; ct++) O[ct][ti] = mfma16(a1, Vb[ct][1], O[ct][ti]);
              }
            }
          }
          if (full) {
            // rows of V_new scaled by e^(gl - gc_t), then S <- e^gl S + k^T (scaled V_new)
            h8 Vd[2][2];
#pragma unroll
            for (int ti = 0; ti < 4; ti++) {
              const f4 ed = lds4(&sm.ed[16 * ti + 4 * grp]);
#pragma unroll
              for (int ct = 0; ct < 2; ct++) Vn[ct][ti] *= ed;
            }
#pragma unroll
            for (int ct = 0; ct < 2; ct++) {
              Vd[ct][0] = pack_b(Vn[ct][0], Vn[ct][1]);
              Vd[ct][1] = pack_b(Vn[ct][2], Vn[ct][3]);
            }
            const float el = sm.eg[kCH - 1];
#pragma unroll
            for (int it = 0; it < 8; it++) {
              const h8 k0 = perm_a_kt(sm.KT, 16 * it + c16, 0, grp), k1 = perm_a_kt(sm.KT, 16 * it + c16, 1, grp);
#pragma unroll
              for (int ct = 0; ct < 2; ct++) S[ct][it] = mfma16(k1, Vd[ct][1], mfma16(k0, Vd[ct][0], S[ct][it] * el));
            }
          }
          // O (D layout) -> epilogue layout through this consumer's slice of Tm, 16 rows at a time
          {
            float* stg = sm.Tm + w * (16 * kSP);
#pragma unroll
            for (int ti = 0; ti < 4; ti++) {
#pragma unroll
              for (int ct = 0; ct < 2; ct++)
#pragma unroll
                for (int e = 0; e < 4; e++) stg[(4 * grp + e) * kSP + 16 * ct + c16] = O[ct][ti][e];
              wave_sync();
#pragma unroll
              for (int s = 0; s < 2; s++) Y[2 * ti + s] = lds4(stg + (8 * s + er) * kSP + 4 * (lane & 7));
              wave_sync();
            }
          }
          if (a.gnorm) {
#pragma unroll
            for (int q = 0; q < 8; q++) {
              const float sq = sum8((Y[q][0] * Y[q][0] + Y[q][1] * Y[q][1]) + (Y[q][2] * Y[q][2] + Y[q][3] * Y[q][3]));
              if ((lane & 7) == 0) sm.red[(8 * q + er) * kNC + w] = sq;
            }
            // the gate factor w * silu(z) of the gated norm, here where the consumers have slack
#pragma unroll
            for (int q = 0; q < 8; q++)
#pragma unroll
              for (int c = 0; c < 4; c++) zq[q][c] = gw[c] * silu(zq[q][c]);
          }
      }
      __syncthreads();  // B

      // ---- B: chunk p's gated norm and store; the v rows of chunk p+1 ----
      if (p >= 0) {
        if (a.gnorm) {
          const f4 r = lds4(&sm.red[lane * kNC]);
          sm.inv[w][lane] = rsqrtf(((r[0] + r[1]) + (r[2] + r[3])) / kDV + 1e-6f);
          wave_sync();
#pragma unroll
          for (int q = 0; q < 8; q++) {
            const float iv = sm.inv[w][8 * q + er];
#pragma unroll
            for (int c = 0; c < 4; c++) Y[q][c] = Y[q][c] * iv * zq[q][c];
          }
        }
        if (plain) {
          char* ob = (char*)a.out + ((size_t)b * a.L + (c0 - a.P)) * (size_t)orowb + (size_t)h * kDV * sizeof(T);
          const unsigned oo = (unsigned)er * orowb + ec * (unsigned)sizeof(T);
#pragma unroll
          for (int q = 0; q < 8; q++) store4(gpw<T>(ob + (size_t)(8 * q) * orowb + oo), Y[q]);
        } else {
          __attribute__((address_space(1))) T* ob = gpw<T>(a.out) + (size_t)b * a.L * (a.H * kDV) + (size_t)h * kDV + ec;
#pragma unroll
          for (int q = 0; q < 8; q++) {
            const int t = 8 * q + er, r = c0 + t;
            if (t < m && r >= a.P) store4(ob + (size_t)(r - a.P) * (a.H * kDV), Y[q]);
          }
        }
      }
      if (p + 1 >= nchunks) break;
      fetch_v(c1);
      __syncthreads();  // C
      // ---- C: score / A tiles of chunk p+1, then the first half of its v conv ----
      kkt_qkt(grp, c16);
      consume_vconv(c1, 0);
      __syncthreads();  // E
      consume_vconv(c1, 4);
      __syncthreads();  // A
    }
    const int g0 = (tid0 & 63) >> 4, l16 = tid0 & 15;
#pragma unroll
    for (int ct = 0; ct < 2; ct++)
#pragma unroll
      for (int it = 0; it < 8; it++)
#pragma unroll
        for (int e = 0; e < 4; e++)
          gpw<float>(a.S_out)[sbase + (size_t)(16 * it + 4 * g0 + e) * kDV + 32 * w + 16 * ct + l16] = S[ct][it][e];
  } else {
    const int last_cs = a.s0 + kCH * (nchunks - 1);
    fetch_qk(a.s0);
    if (w == kGW) produce_gates(a.s0);
    for (int p = -1; p < nchunks; p++) {
      const int c1 = a.s0 + kCH * (p + 1);
      const int tid = opaque(tid0), lane = tid & 63, grp = lane >> 4, c16 = lane & 15;

      // ---- A: conv of chunk p+1 in registers; raw q/k rows (and a/b) of chunk p+2 ----
      // Wave priorities: each segment's longest wave (the gate producer in B and C, the block-column-0 wave in E) is
      // raised so the SIMD it shares with a consumer issues for it first; in A all run at the base priority.
      // Both run every period, past the last chunk on clamped rows whose results are never used: conditional
      // loads would make the loop-carried rows a merge of old and new values, which the compiler resolves with
      // copies that wait for the loads right after they are issued.
      __builtin_amdgcn_s_setprio(0);
      produce_conv(c1);
      fetch_qk(min(c1 + kCH, last_cs));
      __syncthreads();  // B

      // ---- B: q^, k^, k^T and the gate vectors of chunk p+1 to LDS ----
      if (p + 1 >= nchunks) break;
      if (w == kGW) __builtin_amdgcn_s_setprio(2);
      produce_write();
      __syncthreads();  // C

      // ---- C: score / A tiles; the gate producer makes the diagonal blocks of A and solves them ----
      if (w == kGW) {
#pragma unroll
        for (int d = 0; d < 4; d++) kkt_qkt_tile(false, d * (d + 3) / 2, grp, c16);
        wave_sync();
        // lane (grp, c16): column c16 of diagonal block grp, rows in order (left-looking); row r of A is read as a
        // broadcast shared by the 16 lanes of the block
        const int base = 16 * grp;
        float pc[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const float* ar = &sm.Tm[(base + r) * kAP + base];
          float acc = r == c16 ? 1.0f : 0.0f;
#pragma unroll
          for (int j = 0; j < r; j++) acc = fmaf(-ar[j], pc[j], acc);
          pc[r] = acc;
        }
        const float cb = sm.bt[base + c16], cbw = cb * sm.eg[base + c16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
          sm.Tm[(base + r) * kAP + base + c16] = pc[r];
          sm.Tb[(base + r) * kTP + base + c16] = (_Float16)(pc[r] * cb);
          sm.Tw[(base + r) * kTP + base + c16] = (_Float16)(pc[r] * cbw);
        }
      } else {
        kkt_qkt(grp, c16);
      }
      __syncthreads();  // E

      // ---- E: off-diagonal block columns of T; the gate vectors of chunk p+2 ----
      if (w == kNC)
        __builtin_amdgcn_s_setprio(2);
      else
        __builtin_amdgcn_s_setprio(0);
      if (w == kNC)
        t_column<0>(sm, grp, c16);
      else if (w == kNC + 1)
        t_column<1>(sm, grp, c16);
      else if (w == kNC + 2)
        t_column<2>(sm, grp, c16);
      else if (p + 2 < nchunks)
        produce_gates(c1 + kCH);
      __syncthreads();  // A
      (void)lane;
    }
  }
}

template <typename T>
hipError_t launch(const GdnArgs& a, hipStream_t s) {
  auto k = gdn_chunk_kernel<T>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)sizeof(Lds));
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k, dim3(a.B * a.H), dim3(kNT), sizeof(Lds), s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gdn_chunked(const GdnArgs& a, hipStream_t s) {
  if (a.DK != kDK || a.DV != kDV || a.KC != kKC) return hipErrorInvalidValue;
  if (a.P - a.s0 >= kCH || a.P < a.s0) return hipErrorInvalidValue;  // at most one open chunk is replayed
  return a.dtype == 0 ? launch<float>(a, s) : launch<_Float16>(a, s);
}

}  // namespace ha
