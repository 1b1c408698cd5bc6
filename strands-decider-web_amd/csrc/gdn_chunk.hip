// Chunked gated-delta prefill (ha_recurrence HA_CHUNKED), gfx950.
//
// Same semantics as the sequential rule (reference web/public/engine/wgsl.js:124-187 + 252-268), evaluated in the
// chunked WY/UT form the reference's fp32 driver uses for prefill (transformers qwen3_5
// torch_chunk_gated_delta_rule; Yang et al. 2024, "Parallelizing Linear Transformers with the Delta Rule over
// Sequence Length"; Yang, Kautz & Hatamizadeh, "Gated Delta Networks"). For a chunk of 64 rows with cumulative
// log-decay gc (gc_t = sum_{s<=t} g_s inside the chunk) and the state S at the chunk start:
//   A   = strictly_lower(beta_t (k^_t . k^_t') exp(gc_t - gc_t'))      T = (I + A)^-1
//   U   = T (beta v)      W = T (beta exp(gc) k^)      V_new = U - W S
//   o_t = exp(gc_t) q^_t S + sum_{t'<=t} (q^_t . k^_t') exp(gc_t - gc_t') V_new_t'
//   S  <- exp(gc_63) S + sum_t exp(gc_63 - gc_t) k^_t V_new_t^T          (complete chunks only)
//
// One workgroup of 8 waves per (sequence, head) walks the chunks in order; the fp32 state stays in MFMA
// accumulator registers for the whole call (wave w owns value columns 16w..16w+15). Per chunk:
//   1. conv (4 taps) + SiLU straight from the fused rows in HBM, l2 norms by 16-lane reductions, gates by a
//      64-lane scan; f16 tiles of q^, k^ and the pre-scaled transposes (beta e^gc k^)^T, (e^(gl-gc) k^)^T and
//      (beta v)^T land in LDS;
//   2. K K^T and Q K^T on v_mfma_f32_16x16x32_f16 -> A (fp32) and the decay-masked scores (f16);
//   3. T by fp32 forward substitution on the four 16x16 diagonal blocks and fp32 MFMA (16x16x4) for the
//      off-diagonal blocks, while the other waves compute q^ S;
//   4. U and W on f16 MFMA; 5. V_new, o and the state update on f16 MFMA with fp32 accumulation, with S as f16
//      B operands built in registers; 6. gated RMSNorm epilogue (GNORM) and the store.
// Chunk boundaries sit at s0 + 64k, so a row is processed identically however a sequence is split into calls;
// only complete chunks advance the stored state.
//
// MFMA operand convention used below (16x16xK): lane l supplies row (l & 15) of A and column (l & 15) of B, and
// lane group l >> 4 supplies a block of the K index; any assignment of K indices to (lane group, element) works
// as long as A and B use the same one. The result D holds rows 4 (l >> 4) + e, e < 4, of column l & 15. That
// lets a D tile be reused as a B operand (K = its rows) without moving data between lanes: the matching A
// operand is read with the same "permuted" K order {32 kb + 4 grp + e} U {32 kb + 16 + 4 grp + e}.
#include "ha_kernels.h"

namespace ha {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kDK = 128, kDV = 128, kCH = 64, kKC = 4, kNW = 8, kNT = 64 * kNW;
constexpr int kQP = kDK + 8;  // row pitch (halves) of [64][128] f16 tiles
constexpr int kTP = kCH + 8;  // row pitch (halves) of [*][64] f16 tiles
constexpr int kAP = kCH + 4;  // row pitch (floats) of the fp32 A / T tile

struct Lds {
  _Float16 Qs[kCH * kQP];   // q^ / sqrt(DK), [t][i]
  _Float16 Ks[kCH * kQP];   // k^, [t][i]
  _Float16 Ws[kCH * kQP];   // -W, [t][i]
  _Float16 KbT[kDK * kTP];  // (beta e^gc k^)^T, [i][t]
  _Float16 KdT[kDK * kTP];  // (e^(gl - gc) k^)^T, [i][t]
  _Float16 VbT[kDV * kTP];  // (beta v)^T, [j][t]
  _Float16 Tf[kCH * kTP];   // T in f16, [t][t']
  _Float16 Att[kCH * kTP];  // decay-masked causal q^ k^T, [t][t']
  float Tm[kCH * kAP];      // A, then T, fp32
  float Xs[3 * 256];        // off-diagonal solve scratch
  float cw[3 * 128][kKC];   // this head's conv taps (q, k, v channels)
  float red[kCH * kNW];     // gated-norm partial sums
  float inv[kCH];
};

__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }

template <typename T>
__device__ __forceinline__ const T* row_of(const GdnArgs& a, int b, int r) {
  if (r < a.P) return static_cast<const T*>(a.tail) + ((size_t)b * a.tail_cap + (r - (a.s0 - (kKC - 1)))) * a.stride;
  return static_cast<const T*>(a.in) + ((size_t)b * a.L + (r - a.P)) * a.stride;
}

__device__ __forceinline__ void load8(const float* p, float* o) {
  const f4 x = *reinterpret_cast<const f4*>(p), y = *reinterpret_cast<const f4*>(p + 4);
  o[0] = x[0]; o[1] = x[1]; o[2] = x[2]; o[3] = x[3]; o[4] = y[0]; o[5] = y[1]; o[6] = y[2]; o[7] = y[3];
}
__device__ __forceinline__ void load8(const _Float16* p, float* o) {
  const h8 x = *reinterpret_cast<const h8*>(p);
#pragma unroll
  for (int i = 0; i < 8; i++) o[i] = (float)x[i];
}
__device__ __forceinline__ void load4(const float* p, float* o) {
  const f4 x = *reinterpret_cast<const f4*>(p);
  o[0] = x[0]; o[1] = x[1]; o[2] = x[2]; o[3] = x[3];
}
__device__ __forceinline__ void load4(const _Float16* p, float* o) {
  const h4 x = *reinterpret_cast<const h4*>(p);
  o[0] = (float)x[0]; o[1] = (float)x[1]; o[2] = (float)x[2]; o[3] = (float)x[3];
}

// A operand read in the permuted K order matching a D tile pair used as B: row r of a [*][pitch] f16 tile,
// K block kb (32 wide), lane group grp.
__device__ __forceinline__ h8 perm_a(const _Float16* base, int pitch, int r, int kb, int grp) {
  const _Float16* p = base + r * pitch + 32 * kb + 4 * grp;
  const h4 lo = *reinterpret_cast<const h4*>(p), hi = *reinterpret_cast<const h4*>(p + 16);
  return h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Two D tiles (rows 32kb..32kb+15 and 32kb+16..+31 of a column) as one f16 B operand.
__device__ __forceinline__ h8 pack_b(const f4& x, const f4& y) {
  return h8{(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3],
            (_Float16)y[0], (_Float16)y[1], (_Float16)y[2], (_Float16)y[3]};
}

__device__ __forceinline__ f4 mfma16(const h8& a, const h8& b, const f4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <typename T>
__global__ __launch_bounds__(512) void gdn_chunk_kernel(GdnArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  Lds& sm = *reinterpret_cast<Lds*>(lds_raw);
  const int b = blockIdx.x / a.H, h = blockIdx.x % a.H;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, grp = lane >> 4, c16 = lane & 15;
  const int end = a.P + a.L;
  const float qscale = 0.08838834764831845f;  // 1/sqrt(128)

  // state: S[it][e] = S[16 it + 4 grp + e][16 w + c16]
  f4 S[8];
  const size_t sbase = ((size_t)b * a.H + h) * kDK * kDV;
#pragma unroll
  for (int it = 0; it < 8; it++)
#pragma unroll
    for (int e = 0; e < 4; e++)
      S[it][e] = a.S_in ? a.S_in[sbase + (size_t)(16 * it + 4 * grp + e) * kDV + 16 * w + c16] : 0.0f;

  // this head's conv taps: local channel q 0..127, k 128..255, v 256..383
  for (int i = tid; i < 3 * 128 * kKC; i += kNT) {
    const int lc = i / kKC, j = i % kKC;
    const int ch = lc < 128 ? h * kDK + lc : lc < 256 ? a.H * kDK + h * kDK + (lc - 128) : 2 * a.H * kDK + h * kDV + (lc - 256);
    sm.cw[lc][j] = a.conv_w[(size_t)ch * kKC + j];
  }
  __syncthreads();

  // conv tasks: rows 4 rg .. 4 rg + 3 of the chunk; 8 q-or-k channels and 4 v channels
  const int rg = tid >> 5, cgi = tid & 31, qk = cgi >> 4, cg = cgi & 15;
  const int chq = (qk ? a.H * kDK : 0) + h * kDK + 8 * cg, lq = qk * 128 + 8 * cg;
  const int chv = 2 * a.H * kDK + h * kDV + 4 * cgi, lv = 256 + 4 * cgi;
  const float na = a.negA[h], db = a.dtb[h];
  const int aoff = a.C + a.H * kDV + h, boff = aoff + a.H;

  for (int c0 = a.s0; c0 < end; c0 += kCH) {
    const int m = min(kCH, end - c0);
    const bool full = m == kCH;

    // ---- 1. gates: every wave computes all 64 rows (lane = row), kept in registers and read by lane shuffles
    float gcr = 0.0f, btr = 0.0f;
    if (lane < m) {
      const T* row = row_of<T>(a, b, c0 + lane);
      const float av = (float)row[aoff], bv = (float)row[boff];
      btr = 1.0f / (1.0f + __expf(-bv));
      const float xs = av + db;
      gcr = na * (xs > 20.0f ? xs : log1pf(__expf(xs)));
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float o = __shfl_up(gcr, d);
      if (lane >= d) gcr += o;
    }
    const float gl = __shfl(gcr, 63);

    // conv + SiLU + l2 norm of 8 q-or-k channels over 4 rows; f16 tiles (and k's scaled transposes) to LDS
    {
      float x[7][8];
#pragma unroll
      for (int i = 0; i < 7; i++) {
        const int r = c0 + 4 * rg - 3 + i;
        if (r < end) {
          load8(row_of<T>(a, b, r) + chq, x[i]);
        } else {
#pragma unroll
          for (int c = 0; c < 8; c++) x[i][c] = 0.0f;
        }
      }
      float u[4][8], rs[4];
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        const bool valid = 4 * rg + rr < m;
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) {
          const float* wc = sm.cw[lq + c];
          float s = wc[0] * x[rr][c];
          s = fmaf(wc[1], x[rr + 1][c], s);
          s = fmaf(wc[2], x[rr + 2][c], s);
          s = fmaf(wc[3], x[rr + 3][c], s);
          u[rr][c] = valid ? silu(s) : 0.0f;
          ss = fmaf(u[rr][c], u[rr][c], ss);
        }
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) ss += __shfl_xor(ss, d);
        rs[rr] = rsqrtf(ss + 1e-6f) * (qk ? 1.0f : qscale);
      }
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        h8 hv;
#pragma unroll
        for (int c = 0; c < 8; c++) hv[c] = (_Float16)(u[rr][c] * rs[rr]);
        *reinterpret_cast<h8*>((qk ? sm.Ks : sm.Qs) + (4 * rg + rr) * kQP + 8 * cg) = hv;
      }
      float fb[4], fd[4];
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        const int t = 4 * rg + rr;
        const float gt = __shfl(gcr, t), bt = __shfl(btr, t);
        fb[rr] = bt * __expf(gt) * rs[rr];
        fd[rr] = __expf(gl - gt) * rs[rr];
      }
      if (qk) {
#pragma unroll
        for (int c = 0; c < 8; c++) {
          h4 kb, kd;
#pragma unroll
          for (int rr = 0; rr < 4; rr++) {
            kb[rr] = (_Float16)(u[rr][c] * fb[rr]);
            kd[rr] = (_Float16)(u[rr][c] * fd[rr]);
          }
          *reinterpret_cast<h4*>(sm.KbT + (8 * cg + c) * kTP + 4 * rg) = kb;
          *reinterpret_cast<h4*>(sm.KdT + (8 * cg + c) * kTP + 4 * rg) = kd;
        }
      }
    }
    // conv + SiLU of 4 v channels over 4 rows -> (beta v)^T
    {
      float xv[7][4];
#pragma unroll
      for (int i = 0; i < 7; i++) {
        const int r = c0 + 4 * rg - 3 + i;
        if (r < end) {
          load4(row_of<T>(a, b, r) + chv, xv[i]);
        } else {
#pragma unroll
          for (int c = 0; c < 4; c++) xv[i][c] = 0.0f;
        }
      }
      float bt[4];
#pragma unroll
      for (int rr = 0; rr < 4; rr++) bt[rr] = __shfl(btr, 4 * rg + rr);
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float* wc = sm.cw[lv + c];
        h4 vb;
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
          float s = wc[0] * xv[rr][c];
          s = fmaf(wc[1], xv[rr + 1][c], s);
          s = fmaf(wc[2], xv[rr + 2][c], s);
          s = fmaf(wc[3], xv[rr + 3][c], s);
          vb[rr] = (_Float16)(4 * rg + rr < m ? bt[rr] * silu(s) : 0.0f);
        }
        *reinterpret_cast<h4*>(sm.VbT + (4 * cgi + c) * kTP + 4 * rg) = vb;
      }
    }
    // upper blocks of the f16 T and score tiles are read by full 32-wide K blocks: keep them zero
    for (int idx = tid; idx < kCH * kCH; idx += kNT) {
      const int t = idx >> 6, tp = idx & 63;
      if ((tp >> 4) > (t >> 4)) {
        sm.Tf[t * kTP + tp] = (_Float16)0.0f;
        sm.Att[t * kTP + tp] = (_Float16)0.0f;
      }
    }
    __syncthreads();

    // ---- 2. K K^T -> A (fp32), Q K^T -> decay-masked scores (f16); the 10 lower 16x16 tiles of each ----
    for (int job = w; job < 20; job += kNW) {
      const bool isq = job >= 10;
      const int jt = isq ? job - 10 : job;
      const int ti = jt >= 6 ? 3 : jt >= 3 ? 2 : jt >= 1 ? 1 : 0;
      const int tj = jt - ti * (ti + 1) / 2;
      const _Float16* ab = (isq ? sm.Qs : sm.Ks) + (16 * ti + c16) * kQP + 8 * grp;
      const _Float16* bb = sm.Ks + (16 * tj + c16) * kQP + 8 * grp;
      f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 4; ks++)
        acc = mfma16(*reinterpret_cast<const h8*>(ab + 32 * ks), *reinterpret_cast<const h8*>(bb + 32 * ks), acc);
      const int tp = 16 * tj + c16;
      const float gp = __shfl(gcr, tp);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int t = 16 * ti + 4 * grp + e;
        // lane shuffles stay outside the masks: a shuffle in divergent code reads inactive lanes
        const float dec = __expf(fminf(__shfl(gcr, t) - gp, 0.0f)), bt = __shfl(btr, t);
        if (!isq)
          sm.Tm[t * kAP + tp] = tp < t ? bt * acc[e] * dec : 0.0f;
        else
          sm.Att[t * kTP + tp] = (_Float16)(tp <= t ? acc[e] * dec : 0.0f);
      }
    }
    __syncthreads();

    // ---- 3a. diagonal 16x16 blocks of T (wave 0, fp32 forward substitution); q^ S on the other waves ----
    h8 S16[4];
#pragma unroll
    for (int kb = 0; kb < 4; kb++) S16[kb] = pack_b(S[2 * kb], S[2 * kb + 1]);
    f4 O[4];
    auto q_times_s = [&]() {
#pragma unroll
      for (int ti = 0; ti < 4; ti++) {
        f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < 4; kb++) acc = mfma16(perm_a(sm.Qs, kQP, 16 * ti + c16, kb, grp), S16[kb], acc);
        O[ti] = acc;
      }
    };
    if (w == 0) {
      // lane (grp, c16) solves column c16 of diagonal block grp: x_r = [r == c] - sum_{j<r} A_rj x_j
      const int base = 16 * grp;
      float xc[16];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        float s = r == c16 ? 1.0f : 0.0f;
        const float* arow = sm.Tm + (base + r) * kAP + base;
#pragma unroll
        for (int j = 0; j < r; j++) s = fmaf(-arow[j], xc[j], s);
        xc[r] = s;
      }
#pragma unroll
      for (int r = 0; r < 16; r++) {
        sm.Tm[(base + r) * kAP + base + c16] = xc[r];
        sm.Tf[(base + r) * kTP + base + c16] = (_Float16)xc[r];
      }
    } else {
      q_times_s();
    }
    __syncthreads();
    if (w == 0) q_times_s();

    // ---- 3b. off-diagonal blocks: T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj, block rows in order ----
    for (int bi = 1; bi < 4; bi++) {
      if (w < bi) {
        const int j = w;
        f4 X = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int k = j; k < bi; k++)
#pragma unroll
          for (int ks = 0; ks < 4; ks++) {
            const float av = sm.Tm[(16 * bi + c16) * kAP + 16 * k + 4 * ks + grp];
            const float bv = sm.Tm[(16 * k + 4 * ks + grp) * kAP + 16 * j + c16];
            X = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, X, 0, 0, 0);
          }
#pragma unroll
        for (int e = 0; e < 4; e++) sm.Xs[j * 256 + (4 * grp + e) * 16 + c16] = X[e];
      }
      __syncthreads();
      if (w < bi) {
        const int j = w;
        f4 Y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
          const float av = sm.Tm[(16 * bi + c16) * kAP + 16 * bi + 4 * ks + grp];
          const float bv = sm.Xs[j * 256 + (4 * ks + grp) * 16 + c16];
          Y = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, Y, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int t = 16 * bi + 4 * grp + e, tp = 16 * j + c16;
          sm.Tm[t * kAP + tp] = -Y[e];
          sm.Tf[t * kTP + tp] = (_Float16)(-Y[e]);
        }
      }
      __syncthreads();
    }

    // ---- 4. U = T (beta v) for this wave's columns (registers); W = T (beta e^gc k^) -> -W in LDS ----
    f4 U[4];
#pragma unroll
    for (int ti = 0; ti < 4; ti++) {
      f4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, wacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kb = 0; kb <= (ti >> 1); kb++) {
        const h8 ta = *reinterpret_cast<const h8*>(sm.Tf + (16 * ti + c16) * kTP + 32 * kb + 8 * grp);
        acc = mfma16(ta, *reinterpret_cast<const h8*>(sm.VbT + (16 * w + c16) * kTP + 32 * kb + 8 * grp), acc);
        wacc = mfma16(ta, *reinterpret_cast<const h8*>(sm.KbT + (16 * w + c16) * kTP + 32 * kb + 8 * grp), wacc);
      }
      U[ti] = acc;
#pragma unroll
      for (int e = 0; e < 4; e++) sm.Ws[(16 * ti + 4 * grp + e) * kQP + 16 * w + c16] = (_Float16)(-wacc[e]);
    }
    // row decay of the inter-chunk output term: o_t += e^gc_t (q^ S)_t
#pragma unroll
    for (int ti = 0; ti < 4; ti++)
#pragma unroll
      for (int e = 0; e < 4; e++) O[ti][e] *= __expf(__shfl(gcr, 16 * ti + 4 * grp + e));
    __syncthreads();

    // ---- 5. V_new = U - W S; o += scores V_new; S <- e^gl S + (e^(gl-gc) k^)^T V_new ----
    f4 Vn[4];
#pragma unroll
    for (int ti = 0; ti < 4; ti++) {
      f4 acc = U[ti];
#pragma unroll
      for (int kb = 0; kb < 4; kb++) acc = mfma16(perm_a(sm.Ws, kQP, 16 * ti + c16, kb, grp), S16[kb], acc);
      Vn[ti] = acc;
    }
    const h8 Vb0 = pack_b(Vn[0], Vn[1]), Vb1 = pack_b(Vn[2], Vn[3]);
#pragma unroll
    for (int ti = 0; ti < 4; ti++) {
      O[ti] = mfma16(perm_a(sm.Att, kTP, 16 * ti + c16, 0, grp), Vb0, O[ti]);
      if (ti >= 2) O[ti] = mfma16(perm_a(sm.Att, kTP, 16 * ti + c16, 1, grp), Vb1, O[ti]);
    }
    if (full) {
      const float el = __expf(gl);
#pragma unroll
      for (int it = 0; it < 8; it++) {
        f4 acc = S[it] * el;
        acc = mfma16(perm_a(sm.KdT, kTP, 16 * it + c16, 0, grp), Vb0, acc);
        acc = mfma16(perm_a(sm.KdT, kTP, 16 * it + c16, 1, grp), Vb1, acc);
        S[it] = acc;
      }
    }

    // ---- 6. gated RMSNorm over the head's 128 columns and the store ----
    if (a.gnorm) {
#pragma unroll
      for (int ti = 0; ti < 4; ti++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float s = O[ti][e] * O[ti][e];
#pragma unroll
          for (int d = 1; d < 16; d <<= 1) s += __shfl_xor(s, d);
          if (c16 == 0) sm.red[(16 * ti + 4 * grp + e) * kNW + w] = s;
        }
      __syncthreads();
      if (tid < kCH) {
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < kNW; k++) s += sm.red[tid * kNW + k];
        sm.inv[tid] = rsqrtf(s / kDV + 1e-6f);
      }
      __syncthreads();
    }
    const int j = 16 * w + c16;
    const float gw = a.gnorm ? a.gnorm[j] : 1.0f;
#pragma unroll
    for (int ti = 0; ti < 4; ti++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int t = 16 * ti + 4 * grp + e, r = c0 + t;
        if (t < m && r >= a.P) {
          const T* row = static_cast<const T*>(a.in) + ((size_t)b * a.L + (r - a.P)) * a.stride;
          float y = O[ti][e];
          if (a.gnorm) y = gw * y * sm.inv[t] * silu((float)row[a.C + h * kDV + j]);
          static_cast<T*>(a.out)[((size_t)b * a.L + (r - a.P)) * (size_t)(a.H * kDV) + (size_t)h * kDV + j] = (T)y;
        }
      }
    __syncthreads();  // every wave is done with this chunk's LDS tiles before the next chunk writes them
  }
#pragma unroll
  for (int it = 0; it < 8; it++)
#pragma unroll
    for (int e = 0; e < 4; e++)
      a.S_out[sbase + (size_t)(16 * it + 4 * grp + e) * kDV + 16 * w + c16] = S[it][e];
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
