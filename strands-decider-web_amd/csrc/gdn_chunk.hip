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
// accumulator registers for the whole call (wave w owns value columns 16w..16w+15). Five workgroup barriers per
// chunk separate:
//   1. conv (4 taps) + SiLU of raw rows fetched one chunk ahead (their loads overlap the previous chunk's solve and
//      state update), l2 norms by 16-lane DPP reductions -> f16 tiles of q^, k^, k^T and v^T in LDS; one wave turns
//      the a/b columns into the chunk's gate vectors (cumulative log decay, e^gc, beta, e^(gc_63 - gc)) in LDS. The
//      per-row gate factors go onto T's columns and V_new's rows instead of onto copies of k;
//   2. K K^T and Q K^T on v_mfma_f32_16x16x32_f16 -> A (fp32) and the decay-masked scores (f16);
//   3. T = (I + A)^-1: one wave solves the four 16x16 diagonal blocks (left-looking, A rows read as LDS
//      broadcasts) while the others compute q^ S and k^ S; then waves 0..2 each own one block column of the
//      off-diagonal blocks (fp32 MFMA 16x16x4, the column kept in registers), with no barrier between block rows;
//      T diag(beta) and T diag(beta e^gc) are stored f16;
//   4. V_new = T diag(beta) v - T diag(beta e^gc) (k^ S), o and the state update on f16 MFMA with fp32
//      accumulation, S as f16 B operands built in registers; 5. gated RMSNorm epilogue (GNORM) and the store.
// Memory is addressed from wave-uniform (SGPR) row bases plus 32-bit lane offsets on the common path (chunks with
// no replay rows and no rows past the end); the first and last chunk of a call take a general path.
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
constexpr int kGW = kNW - 1;  // the wave that computes the gate vectors and the diagonal blocks of T

struct Lds {
  _Float16 Qs[kCH * kQP];   // q^ / sqrt(DK), [t][i]
  _Float16 Ks[kCH * kQP];   // k^, [t][i]
  _Float16 KT[kDK * kTP];   // k^ transposed, [i][t], 4-column groups swizzled by kt_at
  _Float16 VT[kDV * kTP];   // v transposed, [j][t], 4-column groups swizzled by vt_at
  _Float16 Tb[kCH * kTP];   // T diag(beta), f16, [t][t']
  _Float16 Tw[kCH * kTP];   // T diag(beta e^gc), f16
  _Float16 Att[kCH * kTP];  // decay-masked causal q^ k^T, [t][t']
  float Tm[kCH * kAP];      // A, then T, fp32
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
  float red[kCH * kNW];     // gated-norm partial sums, [t][wave]
  float inv[kNW][kCH];      // per-wave copy of the row inverse norms
};
// After the solve, Tm is free until the next chunk's K K^T: each wave stages 32 x 16 floats of its output there.
static_assert(sizeof(float) * kCH * kAP >= kNW * 32 * 16 * sizeof(float), "staging area");

// Row permutation of the staging area: rows 4 g + e (fixed e) of a D tile land in different quarters of the banks.
__device__ __forceinline__ int stage_row(int r) { return (r & ~3) | ((r + (r >> 2)) & 3); }

// Quad sums (lanes 4q..4q+3) with DPP quad permutations.
__device__ __forceinline__ float quad_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xf, 0xf, false));
  return v;
}

// SiLU / sigmoid with the hardware reciprocal (v_rcp_f32, 1 ulp) instead of an IEEE division sequence
__device__ __forceinline__ float silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// Sum over the 16 lanes of a DPP row (lanes 16r..16r+15) with row rotations; every lane gets the sum.
__device__ __forceinline__ float row_sum16(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x122, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x121, 0xf, 0xf, false));
  return v;
}

// Orders a wave's LDS writes before its later reads of other lanes' entries (no workgroup barrier).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// An identity the compiler cannot see through: per-lane indices re-derived from it every chunk keep the address
// arithmetic built on them inside the chunk loop instead of being hoisted out of it and spilled.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

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

__device__ __forceinline__ f4 ld4(gptr<float> p) { return *(gptr<f4>)(p); }
__device__ __forceinline__ f4 ld4(gptr<_Float16> p) {
  const h4 x = *(gptr<h4>)(p);
  return f4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
}
__device__ __forceinline__ void store4(__attribute__((address_space(1))) float* p, const f4& v) {
  *(__attribute__((address_space(1))) f4*)(p) = v;
}
__device__ __forceinline__ void store4(__attribute__((address_space(1))) _Float16* p, const f4& v) {
  *(__attribute__((address_space(1))) h4*)(p) = h4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
}

// A operand read in the permuted K order matching a D tile pair used as B: row r of a [*][pitch] f16 tile,
// K block kb (32 wide), lane group grp.
__device__ __forceinline__ h8 perm_a(const _Float16* base, int pitch, int r, int kb, int grp) {
  const _Float16* p = base + r * pitch + 32 * kb + 4 * grp;
  const h4 lo = *reinterpret_cast<const h4*>(p), hi = *reinterpret_cast<const h4*>(p + 16);
  return h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Transposed tiles are written one 4-row strip per lane (8 bytes) down the rows of the transpose, which would put
// the lanes of a write 8 (k^T) or 4 (v^T) rows apart and in the same banks; the 4-column group index is XORed
// with a function of the row so those writes spread over the banks. Element (row, col) lives at
// row * kTP + 4 * (col / 4 ^ f(row)) + col % 4. For v^T, f is even, so 8-column (16-byte) reads stay contiguous.
__device__ __forceinline__ int kt_at(int i, int g4) { return i * kTP + 4 * (g4 ^ ((i >> 3) & 15)); }
__device__ __forceinline__ int vt_at(int j, int g4) { return j * kTP + 4 * (g4 ^ (2 * ((j >> 4) & 7))); }

// perm_a for the swizzled k^T tile
__device__ __forceinline__ h8 perm_a_kt(const _Float16* kt, int r, int kb, int grp) {
  const h4 lo = *reinterpret_cast<const h4*>(kt + kt_at(r, 8 * kb + grp));
  const h4 hi = *reinterpret_cast<const h4*>(kt + kt_at(r, 8 * kb + 4 + grp));
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

__device__ __forceinline__ f4 lds4(const float* p) { return *reinterpret_cast<const f4*>(p); }

// Block column J of T below the diagonal: T_iJ = -T_ii sum_{k=J}^{i-1} A_ik T_kJ for block rows i = J+1..3, in
// order. The column's blocks stay in registers (D layout: rows 4 grp + e, column c16), so A is never overwritten
// and the three column waves need no barrier between block rows; only the f16 copies T diag(beta) and
// T diag(beta e^gc) are stored. The D layout is used directly as the B operand of v_mfma_f32_16x16x4f32 by giving
// step e the K index 4 grp + e, and the A operand is read in the same order.
template <int J>
__device__ __forceinline__ void t_column(Lds& sm, int grp, int c16) {
  const int cj = 16 * J + c16;
  const float fb = sm.bt[cj], fw = fb * sm.eg[cj];
  f4 Tc[4];
#pragma unroll
  for (int e = 0; e < 4; e++) Tc[J][e] = sm.Tm[(16 * J + 4 * grp + e) * kAP + cj];
#pragma unroll
  for (int bi = J + 1; bi < 4; bi++) {
    const float* arow = &sm.Tm[(16 * bi + c16) * kAP];
    f4 X = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = J; k < bi; k++) {
      const f4 av = lds4(arow + 16 * k + 4 * grp);
#pragma unroll
      for (int e = 0; e < 4; e++) X = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], Tc[k][e], X, 0, 0, 0);
    }
    const f4 tv = lds4(arow + 16 * bi + 4 * grp);
    f4 Y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int e = 0; e < 4; e++) Y = __builtin_amdgcn_mfma_f32_16x16x4f32(tv[e], X[e], Y, 0, 0, 0);
    Tc[bi] = -Y;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int t = 16 * bi + 4 * grp + e;
      sm.Tb[t * kTP + cj] = (_Float16)(Tc[bi][e] * fb);
      sm.Tw[t * kTP + cj] = (_Float16)(Tc[bi][e] * fw);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(512) void gdn_chunk_kernel(GdnArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  Lds& sm = *reinterpret_cast<Lds*>(lds_raw);
  const int b = blockIdx.x / a.H, h = blockIdx.x % a.H;
  const int tid0 = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  const int end = a.P + a.L;
  const float qscale = 0.08838834764831845f;  // 1/sqrt(128)
  const unsigned rowb = (unsigned)a.stride * sizeof(T);         // bytes per input row
  const unsigned orowb = (unsigned)(a.H * kDV) * sizeof(T);     // bytes per output row

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
  // epilogue layout: lane l holds rows 16 q + l / 4 (q < 4) of columns 16 w + 4 (l % 4) .. +3
  f4 gw = {1.0f, 1.0f, 1.0f, 1.0f};
  if (a.gnorm) gw = ld4(gp<float>(a.gnorm) + 16 * w + 4 * (tid0 & 3));

  // raw rows of a chunk (and, on the gate wave, its a/b inputs), fetched one chunk ahead
  float x[7][8], xv[7][4], ga = 0.0f, gb = 0.0f;
  __syncthreads();  // conv taps and zero blocks visible

  for (int c0 = a.s0; c0 < end; c0 += kCH) {
    const int m = min(kCH, end - c0);
    const bool full = m == kCH;
    const int tid = opaque(tid0), lane = tid & 63, grp = lane >> 4, c16 = lane & 15;
    // conv tasks: rows 4 rg .. 4 rg + 3 of the chunk; 8 q-or-k channels and 4 v channels
    const int rg = tid >> 5, cgi = tid & 31, qk = cgi >> 4, cg = cgi & 15;
    const int chq = (qk ? a.H * kDK : 0) + h * kDK + 8 * cg, chv = 2 * a.H * kDK + h * kDV + 4 * cgi;

    // rows i0..i1-1 of the 7 conv input rows of this lane (chunk rows cs-3 .. cs+63; rows past the end read as 0),
    // and with the first group the gate wave's a/b inputs. The groups are issued at different points of the
    // previous chunk so that the whole workgroup's loads do not reach the memory system in one burst.
    auto fetch = [&](int cs, int i0, int i1) {
      if (cs - (kKC - 1) >= a.P && cs + kCH <= end) {
        // common path: all 67 rows come from `in`; uniform row bases, 32-bit lane offsets
        const char* base = (const char*)a.in + ((size_t)b * a.L + (cs - (kKC - 1) - a.P)) * (size_t)rowb;
        const unsigned oq = 4u * rg * rowb + chq * (unsigned)sizeof(T), ov = 4u * rg * rowb + chv * (unsigned)sizeof(T);
#pragma unroll
        for (int i = i0; i < i1; i++) {
          const char* rb = base + (size_t)i * rowb;
          load8(gp<T>(rb + oq), x[i]);
          load4(gp<T>(rb + ov), xv[i]);
        }
        if (w == kGW && i0 == 0) {
          const char* gb0 = base + (size_t)(kKC - 1) * rowb;
          const unsigned og = (unsigned)lane * rowb;
          ga = (float)*gp<T>(gb0 + og + aoff * sizeof(T));
          gb = (float)*gp<T>(gb0 + og + boff * sizeof(T));
        }
      } else {
#pragma unroll
        for (int i = i0; i < i1; i++) {
          const int r = cs + 4 * rg - 3 + i, rc = min(r, end - 1);
          const gptr<T> row = row_of<T>(a, b, rc);
          load8(row + chq, x[i]);
          load4(row + chv, xv[i]);
          if (r >= end) {
#pragma unroll
            for (int c = 0; c < 8; c++) x[i][c] = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; c++) xv[i][c] = 0.0f;
          }
        }
        if (w == kGW && i0 == 0) {
          const gptr<T> grow = row_of<T>(a, b, min(cs + lane, end - 1));
          ga = cs + lane < end ? (float)grow[aoff] : 0.0f;
          gb = cs + lane < end ? (float)grow[boff] : 0.0f;
        }
      }
    };
    if (c0 == a.s0) fetch(c0, 0, 7);

    // ---- 1. gate vectors (one wave, lane = row), conv + SiLU + norms (all waves) ----
    if (w == kGW) {
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
      sm.gc[lane] = gcr;
      sm.eg[lane] = __expf(gcr);
      sm.bt[lane] = btr;
      sm.ed[lane] = __expf(gl - gcr);
      const float rf = __expf(gcr - __shfl(gcr, lane & ~15));
      sm.rowf[lane] = rf;
      sm.brow[lane] = btr * rf;
#pragma unroll
      for (int i = 1; i < 4; i++) {
        const float gi = __shfl(gcr, 16 * i);
        sm.colf[i - 1][lane] = lane < 16 * i ? __expf(gi - gcr) : 0.0f;
      }
    }
    {
      float u[4][8], ss[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < 8; c++) {
        const f4 wc = lds4(sm.cwq[c][cgi]);
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
          float sv = wc[0] * x[rr][c];
          sv = fmaf(wc[1], x[rr + 1][c], sv);
          sv = fmaf(wc[2], x[rr + 2][c], sv);
          sv = fmaf(wc[3], x[rr + 3][c], sv);
          u[rr][c] = 4 * rg + rr < m ? silu(sv) : 0.0f;
          ss[rr] = fmaf(u[rr][c], u[rr][c], ss[rr]);
        }
      }
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        const float rs = rsqrtf(row_sum16(ss[rr]) + 1e-6f) * (qk ? 1.0f : qscale);
#pragma unroll
        for (int c = 0; c < 8; c++) u[rr][c] *= rs;
        h8 hv;
#pragma unroll
        for (int c = 0; c < 8; c++) hv[c] = (_Float16)u[rr][c];
        *reinterpret_cast<h8*>((qk ? sm.Ks : sm.Qs) + (4 * rg + rr) * kQP + 8 * cg) = hv;
      }
      if (qk) {
#pragma unroll
        for (int c = 0; c < 8; c++) {
          h4 kt;
#pragma unroll
          for (int rr = 0; rr < 4; rr++) kt[rr] = (_Float16)u[rr][c];
          *reinterpret_cast<h4*>(sm.KT + kt_at(8 * cg + c, rg)) = kt;
        }
      }
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const f4 wc = lds4(sm.cwv[c][cgi]);
      h4 vt;
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        float sv = wc[0] * xv[rr][c];
        sv = fmaf(wc[1], xv[rr + 1][c], sv);
        sv = fmaf(wc[2], xv[rr + 2][c], sv);
        sv = fmaf(wc[3], xv[rr + 3][c], sv);
        vt[rr] = (_Float16)(4 * rg + rr < m ? silu(sv) : 0.0f);
      }
      *reinterpret_cast<h4*>(sm.VT + vt_at(4 * cgi + c, rg)) = vt;
    }
    __syncthreads();  // B1
    fetch(c0 + kCH, 0, 3);
    // z of this chunk for the gated-norm epilogue (epilogue layout), in flight from here to the epilogue
    const bool plain = c0 >= a.P && full;  // no replay rows, no rows past the end
    const int er = lane >> 2, ec = 16 * w + 4 * (lane & 3);  // epilogue row within a 16-row block, column
    f4 zq[4];
    if (plain) {
      const char* zb = (const char*)a.in + ((size_t)b * a.L + (c0 - a.P)) * (size_t)rowb + (a.C + h * kDV) * sizeof(T);
      const unsigned oz = (unsigned)er * rowb + ec * (unsigned)sizeof(T);
#pragma unroll
      for (int q = 0; q < 4; q++) zq[q] = ld4(gp<T>(zb + (size_t)(16 * q) * rowb + oz));
    } else {
      const gptr<T> zb = gp<T>(a.in) + (size_t)b * a.L * a.stride + a.C + h * kDV + ec;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int rr = min(max(c0 + 16 * q + er - a.P, 0), a.L - 1);
        zq[q] = ld4(zb + (size_t)rr * a.stride);
      }
    }


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
    __syncthreads();  // B2

    // ---- 3. T = (I + A)^-1; q^ S and k^ S ----
    h8 S16[4], KSb[2];
    f4 O[4];
    auto qk_times_s = [&]() {
#pragma unroll
      for (int kb = 0; kb < 4; kb++) S16[kb] = pack_b(S[2 * kb], S[2 * kb + 1]);
      f4 ksd[4];
#pragma unroll
      for (int ti = 0; ti < 4; ti++) {
        f4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, acck = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
          acc = mfma16(perm_a(sm.Qs, kQP, 16 * ti + c16, kb, grp), S16[kb], acc);
          acck = mfma16(perm_a(sm.Ks, kQP, 16 * ti + c16, kb, grp), S16[kb], acck);
        }
        O[ti] = acc;
        ksd[ti] = acck;
      }
      KSb[0] = pack_b(ksd[0], ksd[1]);
      KSb[1] = pack_b(ksd[2], ksd[3]);
    };
    if (w == kGW) {
      // lane (grp, c16): column c16 of diagonal block grp, rows in order (left-looking); row r of A is read as a
      // broadcast shared by the 16 lanes of the block
      const int base = 16 * grp;
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const float* ar = &sm.Tm[(base + r) * kAP + base];
        float acc = r == c16 ? 1.0f : 0.0f;
#pragma unroll
        for (int j = 0; j < r; j++) acc = fmaf(-ar[j], p[j], acc);
        p[r] = acc;
      }
      const float cb = sm.bt[base + c16], cbw = cb * sm.eg[base + c16];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        sm.Tm[(base + r) * kAP + base + c16] = p[r];
        sm.Tb[(base + r) * kTP + base + c16] = (_Float16)(p[r] * cb);
        sm.Tw[(base + r) * kTP + base + c16] = (_Float16)(p[r] * cbw);
      }
      fetch(c0 + kCH, 3, 5);
    } else {
      fetch(c0 + kCH, 3, 5);
      qk_times_s();
    }
    __syncthreads();  // B3
    if (w == 0)
      t_column<0>(sm, grp, c16);
    else if (w == 1)
      t_column<1>(sm, grp, c16);
    else if (w == 2)
      t_column<2>(sm, grp, c16);
    else if (w == kGW)
      qk_times_s();
    // the next chunk's raw rows load from here on, behind the state update and the epilogue (issued after the
    // solve on the waves that do it, so address-unit back-pressure from the other waves' loads does not delay it)
    fetch(c0 + kCH, 5, 7);
    __syncthreads();  // B4

    // ---- 4. V_new = T diag(beta) v - T diag(beta e^gc) (k^ S); o = e^gc (q^ S) + scores V_new; state ----
    f4 Vn[4];
    const int col = 16 * w + c16;
#pragma unroll
    for (int ti = 0; ti < 4; ti++) {
      f4 u = {0.0f, 0.0f, 0.0f, 0.0f}, ws = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kb = 0; kb <= (ti >> 1); kb++) {
        u = mfma16(*reinterpret_cast<const h8*>(sm.Tb + (16 * ti + c16) * kTP + 32 * kb + 8 * grp),
                   *reinterpret_cast<const h8*>(sm.VT + vt_at(col, 8 * kb + 2 * grp)), u);
        ws = mfma16(perm_a(sm.Tw, kTP, 16 * ti + c16, kb, grp), KSb[kb], ws);
      }
      Vn[ti] = u - ws;
    }
#pragma unroll
    for (int ti = 0; ti < 4; ti++) O[ti] *= lds4(&sm.eg[16 * ti + 4 * grp]);
    const h8 Vb0 = pack_b(Vn[0], Vn[1]), Vb1 = pack_b(Vn[2], Vn[3]);
#pragma unroll
    for (int ti = 0; ti < 4; ti++) {
      O[ti] = mfma16(perm_a(sm.Att, kTP, 16 * ti + c16, 0, grp), Vb0, O[ti]);
      if (ti >= 2) O[ti] = mfma16(perm_a(sm.Att, kTP, 16 * ti + c16, 1, grp), Vb1, O[ti]);
    }
    if (full) {
      // rows of V_new scaled by e^(gl - gc_t), then S <- e^gl S + k^T (scaled V_new)
#pragma unroll
      for (int ti = 0; ti < 4; ti++) Vn[ti] *= lds4(&sm.ed[16 * ti + 4 * grp]);
      const h8 Vd0 = pack_b(Vn[0], Vn[1]), Vd1 = pack_b(Vn[2], Vn[3]);
      const float el = sm.eg[kCH - 1];
#pragma unroll
      for (int it = 0; it < 8; it++) {
        f4 acc = S[it] * el;
        acc = mfma16(perm_a_kt(sm.KT, 16 * it + c16, 0, grp), Vd0, acc);
        acc = mfma16(perm_a_kt(sm.KT, 16 * it + c16, 1, grp), Vd1, acc);
        S[it] = acc;
      }
    }
    // O (D layout) -> epilogue layout (4 consecutive columns of a row per lane) through this wave's slice of Tm,
    // 32 rows at a time, so that the z loads and the output stores are 16-byte accesses
    f4 Y[4];
    {
      float* stg = sm.Tm + w * (32 * 16);
#pragma unroll
      for (int hf = 0; hf < 2; hf++) {
#pragma unroll
        for (int ti = 0; ti < 2; ti++)
#pragma unroll
          for (int e = 0; e < 4; e++) stg[stage_row(16 * ti + 4 * grp + e) * 16 + c16] = O[2 * hf + ti][e];
        wave_sync();
#pragma unroll
        for (int s = 0; s < 2; s++) Y[2 * hf + s] = lds4(stg + stage_row(16 * s + er) * 16 + 4 * (lane & 3));
        wave_sync();
      }
    }
    if (a.gnorm) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float sq = quad_sum((Y[q][0] * Y[q][0] + Y[q][1] * Y[q][1]) + (Y[q][2] * Y[q][2] + Y[q][3] * Y[q][3]));
        if ((lane & 3) == 0) sm.red[(16 * q + er) * kNW + w] = sq;
      }
    }
    __syncthreads();  // B5: every wave is done with this chunk's tiles; the next chunk may overwrite them

    // ---- 5. gated RMSNorm over the head's 128 columns and the store ----
    if (a.gnorm) {
      const f4 r0 = lds4(&sm.red[lane * kNW]), r1 = lds4(&sm.red[lane * kNW + 4]);
      const float sq = ((r0[0] + r0[1]) + (r0[2] + r0[3])) + ((r1[0] + r1[1]) + (r1[2] + r1[3]));
      sm.inv[w][lane] = rsqrtf(sq / kDV + 1e-6f);
      wave_sync();
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float iv = sm.inv[w][16 * q + er];
#pragma unroll
        for (int c = 0; c < 4; c++) Y[q][c] = gw[c] * Y[q][c] * iv * silu(zq[q][c]);
      }
    }
    if (plain) {
      char* ob = (char*)a.out + ((size_t)b * a.L + (c0 - a.P)) * (size_t)orowb + (size_t)h * kDV * sizeof(T);
      const unsigned oo = (unsigned)er * orowb + ec * (unsigned)sizeof(T);
#pragma unroll
      for (int q = 0; q < 4; q++) store4(gpw<T>(ob + (size_t)(16 * q) * orowb + oo), Y[q]);
    } else {
      __attribute__((address_space(1))) T* ob = gpw<T>(a.out) + (size_t)b * a.L * (a.H * kDV) + (size_t)h * kDV + ec;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int t = 16 * q + er, r = c0 + t;
        if (t < m && r >= a.P) store4(ob + (size_t)(r - a.P) * (a.H * kDV), Y[q]);
      }
    }
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
