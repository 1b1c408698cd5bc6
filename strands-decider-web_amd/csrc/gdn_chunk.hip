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
// One workgroup of 8 waves per (sequence, head) walks the chunks in order; the fp32 state stays in MFMA
// accumulator registers for the whole call (wave w owns value columns 16w..16w+15). Per chunk:
//   1. conv (4 taps) + SiLU of raw rows fetched one chunk ahead (their loads overlap the previous chunk's state
//      update), l2 norms by 16-lane reductions, gates by a 64-lane scan; f16 tiles of q^, k^, k^T and v^T in LDS
//      (the per-row gate factors are applied to T's columns and V_new's rows instead of to copies of k);
//   2. K K^T and Q K^T on v_mfma_f32_16x16x32_f16 -> A (fp32) and the decay-masked scores (f16);
//   3. T: right-looking fp32 substitution on the four 16x16 diagonal blocks (one wave) and fp32 MFMA (16x16x4) for
//      the off-diagonal blocks, while the other waves compute q^ S; T diag(beta), T diag(beta e^gc) stored f16;
//   4-5. U, k^ S, V_new, o and the state update on f16 MFMA with fp32 accumulation, S as f16 B operands built in
//      registers; 6. gated RMSNorm epilogue (GNORM) and the store.
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
  _Float16 KT[kDK * kTP];   // k^ transposed, [i][t]
  _Float16 VT[kDV * kTP];   // v transposed, [j][t]
  _Float16 Tb[kCH * kTP];   // T diag(beta), f16, [t][t']
  _Float16 Tw[kCH * kTP];   // T diag(beta e^gc), f16
  _Float16 Att[kCH * kTP];  // decay-masked causal q^ k^T, [t][t']
  float Tm[kCH * kAP];      // A, then T, fp32
  float Xs[3 * 256];        // off-diagonal solve scratch
  float cw[3 * 128][kKC];   // this head's conv taps (q, k, v channels)
  float red[kCH * kNW];     // gated-norm partial sums
  float inv[kCH];
};

// SiLU / sigmoid with the hardware reciprocal (v_rcp_f32, 1 ulp) instead of an IEEE division sequence
__device__ __forceinline__ float silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// Global (address space 1) pointers: loads through them are global_load_*, not flat_load_*, so they are not
// counted by the LDS wait counter and outstanding global loads do not stall LDS traffic.
template <typename T>
using gptr = const __attribute__((address_space(1))) T*;
template <typename T>
__device__ __forceinline__ gptr<T> gp(const void* p) { return (gptr<T>)(p); }
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gpw(void* p) { return (__attribute__((address_space(1))) T*)(p); }

template <typename T>
__device__ __forceinline__ gptr<T> row_of(const GdnArgs& a, int b, int r) {
  if (r < a.P) return gp<T>(a.tail) + ((size_t)b * a.tail_cap + (r - (a.s0 - (kKC - 1)))) * a.stride;
  return gp<T>(a.in) + ((size_t)b * a.L + (r - a.P)) * a.stride;
}

__device__ __forceinline__ void load8(gptr<float> p, float* o) {
  const f4 x = *(gptr<f4>)(p), y = *(gptr<f4>)(p + 4);
  o[0] = x[0]; o[1] = x[1]; o[2] = x[2]; o[3] = x[3]; o[4] = y[0]; o[5] = y[1]; o[6] = y[2]; o[7] = y[3];
}
__device__ __forceinline__ void load8(gptr<_Float16> p, float* o) {
  const h8 x = *(gptr<h8>)(p);
#pragma unroll
  for (int i = 0; i < 8; i++) o[i] = (float)x[i];
}
__device__ __forceinline__ void load4(gptr<float> p, float* o) {
  const f4 x = *(gptr<f4>)(p);
  o[0] = x[0]; o[1] = x[1]; o[2] = x[2]; o[3] = x[3];
}
__device__ __forceinline__ void load4(gptr<_Float16> p, float* o) {
  const h4 x = *(gptr<h4>)(p);
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

__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

template <typename T>
__global__ __launch_bounds__(512) void gdn_chunk_kernel(GdnArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  Lds& sm = *reinterpret_cast<Lds*>(lds_raw);
  const int b = blockIdx.x / a.H, h = blockIdx.x % a.H;
  const int tid0 = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  const int end = a.P + a.L;
  const float qscale = 0.08838834764831845f;  // 1/sqrt(128)

  // state: S[it][e] = S[16 it + 4 grp + e][16 w + c16]
  f4 S[8];
  const size_t sbase = ((size_t)b * a.H + h) * kDK * kDV;
#pragma unroll
  for (int it = 0; it < 8; it++)
#pragma unroll
    for (int e = 0; e < 4; e++)
      S[it][e] = a.S_in ? gp<float>(a.S_in)[sbase + (size_t)(16 * it + 4 * ((tid0 & 63) >> 4) + e) * kDV + 16 * w + (tid0 & 15)] : 0.0f;

  // this head's conv taps: local channel q 0..127, k 128..255, v 256..383
  for (int i = tid0; i < 3 * 128 * kKC; i += kNT) {
    const int lc = i / kKC, j = i % kKC;
    const int ch = lc < 128 ? h * kDK + lc : lc < 256 ? a.H * kDK + h * kDK + (lc - 128) : 2 * a.H * kDK + h * kDV + (lc - 256);
    sm.cw[lc][j] = gp<float>(a.conv_w)[(size_t)ch * kKC + j];
  }

  const float na = gp<float>(a.negA)[h], db = gp<float>(a.dtb)[h];
  const int aoff = a.C + a.H * kDV + h, boff = aoff + a.H;

  // raw rows of a chunk (and its a/b gate inputs), fetched one chunk ahead; rows past the end read as 0, so the
  // fetch is unconditional and the previous chunk's rows are dead once it is issued
  float x[7][8], xv[7][4], ga, gb;
  __syncthreads();  // conv taps visible

  for (int c0 = a.s0; c0 < end; c0 += kCH) {
    const int m = min(kCH, end - c0);
    const bool full = m == kCH;
    // per-lane indices re-derived every chunk through an opaque copy: address arithmetic built on them stays in
    // the loop instead of being hoisted out of it and spilled
    const int tid = opaque(tid0), lane = tid & 63, grp = lane >> 4, c16 = lane & 15;
    // conv tasks: rows 4 rg .. 4 rg + 3 of the chunk; 8 q-or-k channels and 4 v channels
    const int rg = tid >> 5, cgi = tid & 31, qk = cgi >> 4, cg = cgi & 15;
    const int chq = (qk ? a.H * kDK : 0) + h * kDK + 8 * cg, lq = qk * 128 + 8 * cg;
    const int chv = 2 * a.H * kDK + h * kDV + 4 * cgi, lv = 256 + 4 * cgi;

    // raw rows of a chunk (and its a/b gate inputs), fetched one chunk ahead; rows past the end read as 0, so the
    // fetch is unconditional and the previous chunk's rows are dead once it is issued
    auto fetch = [&](int cs) {
      const bool fresh = cs - (kKC - 1) >= a.P;  // no row of this chunk (incl. its conv history) is a replay row
      const gptr<T> base = gp<T>(a.in) + ((ptrdiff_t)b * a.L + (cs - a.P)) * a.stride;
  #pragma unroll
      for (int i = 0; i < 7; i++) {
        const int r = cs + 4 * rg - 3 + i, rc = min(r, end - 1);
        const gptr<T> row = fresh ? base + (ptrdiff_t)(rc - cs) * a.stride : row_of<T>(a, b, rc);
        load8(row + chq, x[i]);
        load4(row + chv, xv[i]);
        if (r >= end) {
  #pragma unroll
          for (int c = 0; c < 8; c++) x[i][c] = 0.0f;
  #pragma unroll
          for (int c = 0; c < 4; c++) xv[i][c] = 0.0f;
        }
      }
      const gptr<T> grow = row_of<T>(a, b, min(cs + lane, end - 1));
      ga = cs + lane < end ? (float)grow[aoff] : 0.0f;
      gb = cs + lane < end ? (float)grow[boff] : 0.0f;
    };
    if (c0 == a.s0) fetch(c0);

    // z of this chunk for the gated-norm epilogue, in flight during the whole chunk
    float zr[4][4];
    {
      const gptr<T> zb = gp<T>(a.in) + (size_t)b * a.L * a.stride + a.C + h * kDV + 16 * w + c16;
#pragma unroll
      for (int ti = 0; ti < 4; ti++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int t = 16 * ti + 4 * grp + e, r = c0 + t;
          const int rr = min(max(r - a.P, 0), a.L - 1);
          zr[ti][e] = (float)zb[(size_t)rr * a.stride];
        }
    }

    // ---- 1. gates: every wave holds all 64 rows (lane = row) in registers, read by lane shuffles ----
    float gcr = 0.0f, btr = 0.0f;
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
    const float gl = __shfl(gcr, 63);

    // conv + SiLU + l2 norm of 8 q-or-k channels over 4 rows -> q^ / k^ rows, k^ transposed
    {
      float u[4][8], rs[4];
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        const bool valid = 4 * rg + rr < m;
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) {
          const float* wc = sm.cw[lq + c];
          float sv = wc[0] * x[rr][c];
          sv = fmaf(wc[1], x[rr + 1][c], sv);
          sv = fmaf(wc[2], x[rr + 2][c], sv);
          sv = fmaf(wc[3], x[rr + 3][c], sv);
          u[rr][c] = valid ? silu(sv) : 0.0f;
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
      if (qk) {
#pragma unroll
        for (int c = 0; c < 8; c++) {
          h4 kt;
#pragma unroll
          for (int rr = 0; rr < 4; rr++) kt[rr] = (_Float16)(u[rr][c] * rs[rr]);
          *reinterpret_cast<h4*>(sm.KT + (8 * cg + c) * kTP + 4 * rg) = kt;
        }
      }
    }
    // conv + SiLU of 4 v channels over 4 rows -> v^T
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float* wc = sm.cw[lv + c];
      h4 vt;
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        float sv = wc[0] * xv[rr][c];
        sv = fmaf(wc[1], xv[rr + 1][c], sv);
        sv = fmaf(wc[2], xv[rr + 2][c], sv);
        sv = fmaf(wc[3], xv[rr + 3][c], sv);
        vt[rr] = (_Float16)(4 * rg + rr < m ? silu(sv) : 0.0f);
      }
      *reinterpret_cast<h4*>(sm.VT + (4 * cgi + c) * kTP + 4 * rg) = vt;
    }
    // upper blocks of the f16 T and score tiles are read by full 32-wide K blocks: keep them zero
    for (int idx = tid; idx < kCH * kCH; idx += kNT) {
      const int t = idx >> 6, tp = idx & 63;
      if ((tp >> 4) > (t >> 4)) {
        sm.Tb[t * kTP + tp] = (_Float16)0.0f;
        sm.Tw[t * kTP + tp] = (_Float16)0.0f;
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
      const float gp_ = __shfl(gcr, tp);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int t = 16 * ti + 4 * grp + e;
        // lane shuffles stay outside the masks: a shuffle in divergent code reads inactive lanes
        const float dec = __expf(fminf(__shfl(gcr, t) - gp_, 0.0f)), bt = __shfl(btr, t);
        if (!isq)
          sm.Tm[t * kAP + tp] = tp < t ? bt * acc[e] * dec : 0.0f;
        else
          sm.Att[t * kTP + tp] = (_Float16)(tp <= t ? acc[e] * dec : 0.0f);
      }
    }
    __syncthreads();

    // column factors of T diag(beta) and T diag(beta e^gc) for column c16 of block grp
    const int colc = 16 * grp + c16;
    const float cb = __shfl(btr, colc), cbw = cb * __expf(__shfl(gcr, colc));

    // ---- 3a. diagonal 16x16 blocks of T (wave 0); q^ S on the other waves ----
    h8 S16[4];
    f4 O[4];
    auto q_times_s = [&]() {
#pragma unroll
      for (int kb = 0; kb < 4; kb++) S16[kb] = pack_b(S[2 * kb], S[2 * kb + 1]);
#pragma unroll
      for (int ti = 0; ti < 4; ti++) {
        f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < 4; kb++) acc = mfma16(perm_a(sm.Qs, kQP, 16 * ti + c16, kb, grp), S16[kb], acc);
        O[ti] = acc;
      }
    };
    if (w == 0) {
      // lane (grp, c16) computes column c16 of diagonal block grp, right-looking: after x_j is final, every
      // later row r subtracts A_rj x_j (A's column j read from LDS as it is needed)
      const int base = 16 * grp;
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; r++) p[r] = r == c16 ? 1.0f : 0.0f;
#pragma unroll
      for (int j = 0; j < 15; j++) {
#pragma unroll
        for (int r = j + 1; r < 16; r++) p[r] = fmaf(-sm.Tm[(base + r) * kAP + base + j], p[j], p[r]);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int r = 0; r < 16; r++) {
        sm.Tm[(base + r) * kAP + base + c16] = p[r];
        sm.Tb[(base + r) * kTP + base + c16] = (_Float16)(p[r] * cb);
        sm.Tw[(base + r) * kTP + base + c16] = (_Float16)(p[r] * cbw);
      }
    } else {
      q_times_s();
    }
    __syncthreads();

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
        const int col = 16 * j + c16;
        const float fb = __shfl(btr, col), fw = fb * __expf(__shfl(gcr, col));
        f4 Y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
          const float av = sm.Tm[(16 * bi + c16) * kAP + 16 * bi + 4 * ks + grp];
          const float bv = sm.Xs[j * 256 + (4 * ks + grp) * 16 + c16];
          Y = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, Y, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int t = 16 * bi + 4 * grp + e;
          sm.Tm[t * kAP + col] = -Y[e];
          sm.Tb[t * kTP + col] = (_Float16)(-Y[e] * fb);
          sm.Tw[t * kTP + col] = (_Float16)(-Y[e] * fw);
        }
      }
      __syncthreads();
    }
    if (w == 0) q_times_s();

    // ---- 4-5. U = T diag(beta) v; V_new = U - T diag(beta e^gc) (k^ S); o += scores V_new; S update ----
    // the next chunk's raw rows and gates load from here on, behind the state update and the epilogue
    fetch(c0 + kCH);
    f4 Vn[4];
    {
      // k^ S for this wave's columns (S16 still holds S), as a B operand over t
      h8 KSb[2];
      f4 ksd[4];
#pragma unroll
      for (int ti = 0; ti < 4; ti++) {
        f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < 4; kb++) acc = mfma16(perm_a(sm.Ks, kQP, 16 * ti + c16, kb, grp), S16[kb], acc);
        ksd[ti] = acc;
      }
      KSb[0] = pack_b(ksd[0], ksd[1]);
      KSb[1] = pack_b(ksd[2], ksd[3]);
      const int col = 16 * w + c16;
#pragma unroll
      for (int ti = 0; ti < 4; ti++) {
        f4 u = {0.0f, 0.0f, 0.0f, 0.0f}, ws = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb <= (ti >> 1); kb++) {
          u = mfma16(*reinterpret_cast<const h8*>(sm.Tb + (16 * ti + c16) * kTP + 32 * kb + 8 * grp),
                     *reinterpret_cast<const h8*>(sm.VT + col * kTP + 32 * kb + 8 * grp), u);
          ws = mfma16(perm_a(sm.Tw, kTP, 16 * ti + c16, kb, grp), KSb[kb], ws);
        }
        Vn[ti] = u - ws;
      }
    }
    // o_t = e^gc_t (q^ S)_t + scores V_new
#pragma unroll
    for (int ti = 0; ti < 4; ti++)
#pragma unroll
      for (int e = 0; e < 4; e++) O[ti][e] *= __expf(__shfl(gcr, 16 * ti + 4 * grp + e));
    const h8 Vb0 = pack_b(Vn[0], Vn[1]), Vb1 = pack_b(Vn[2], Vn[3]);
#pragma unroll
    for (int ti = 0; ti < 4; ti++) {
      O[ti] = mfma16(perm_a(sm.Att, kTP, 16 * ti + c16, 0, grp), Vb0, O[ti]);
      if (ti >= 2) O[ti] = mfma16(perm_a(sm.Att, kTP, 16 * ti + c16, 1, grp), Vb1, O[ti]);
    }
    if (full) {
      // rows of V_new scaled by e^(gl - gc_t), then S <- e^gl S + k^T (scaled V_new)
      f4 Vd[4];
#pragma unroll
      for (int ti = 0; ti < 4; ti++)
#pragma unroll
        for (int e = 0; e < 4; e++) Vd[ti][e] = Vn[ti][e] * __expf(gl - __shfl(gcr, 16 * ti + 4 * grp + e));
      const h8 Vd0 = pack_b(Vd[0], Vd[1]), Vd1 = pack_b(Vd[2], Vd[3]);
      const float el = __expf(gl);
#pragma unroll
      for (int it = 0; it < 8; it++) {
        f4 acc = S[it] * el;
        acc = mfma16(perm_a(sm.KT, kTP, 16 * it + c16, 0, grp), Vd0, acc);
        acc = mfma16(perm_a(sm.KT, kTP, 16 * it + c16, 1, grp), Vd1, acc);
        S[it] = acc;
      }
    }

    // ---- 6. gated RMSNorm over the head's 128 columns and the store ----
    if (a.gnorm) {
#pragma unroll
      for (int ti = 0; ti < 4; ti++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float sq = O[ti][e] * O[ti][e];
#pragma unroll
          for (int d = 1; d < 16; d <<= 1) sq += __shfl_xor(sq, d);
          if (c16 == 0) sm.red[(16 * ti + 4 * grp + e) * kNW + w] = sq;
        }
      __syncthreads();
      if (tid < kCH) {
        float sq = 0.0f;
#pragma unroll
        for (int k = 0; k < kNW; k++) sq += sm.red[tid * kNW + k];
        sm.inv[tid] = rsqrtf(sq / kDV + 1e-6f);
      }
      __syncthreads();
    }
    const int j = 16 * w + c16;
    const float gw = a.gnorm ? gp<float>(a.gnorm)[j] : 1.0f;
    __attribute__((address_space(1))) T* ob = gpw<T>(a.out) + (size_t)b * a.L * (a.H * kDV) + (size_t)h * kDV + j;
#pragma unroll
    for (int ti = 0; ti < 4; ti++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int t = 16 * ti + 4 * grp + e, r = c0 + t;
        if (t < m && r >= a.P) {
          float y = O[ti][e];
          if (a.gnorm) y = gw * y * sm.inv[t] * silu(zr[ti][e]);
          ob[(size_t)(r - a.P) * (a.H * kDV)] = (T)y;
        }
      }
    __syncthreads();  // every wave is done with this chunk's LDS tiles before the next chunk writes them
  }
#pragma unroll
  for (int it = 0; it < 8; it++)
#pragma unroll
    for (int e = 0; e < 4; e++)
      gpw<float>(a.S_out)[sbase + (size_t)(16 * it + 4 * ((tid0 & 63) >> 4) + e) * kDV + 16 * w + (tid0 & 15)] = S[it][e];
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
