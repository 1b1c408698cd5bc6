// MatMulNBits projections, the matmuls either side of the hybrid-attention path, gfx950.
//
// Reference: web/public/gemmbench/kernels.js:1-14 (weight formats) and 15-36 (block decode),
// convert/export_engine.py:17-26 (int4 RTN export), web/public/engine/engine.js:236-246 (matmul dispatch) and
// engine.js:17-33 (kernel choice by M), web/public/engine/wgsl.js:91-108 (FWHT input rotation).
//
//   y[M][N] (f16) = a[M][K] (f16) x W^T, fp32 accumulation, W[n][k] dequantised from blocks of 32 consecutive k
//   of one row n: 4 bits: 4 words per block, element e at bits 4(e%8) of word e/8 (MatMulNBits: element 2i in the
//   low nibble of byte i); 2 bits: 2 words, element e at bits 2(e%16) of word e/16; 3 bits: 3 words, words 0-1
//   hold the low two bits as in the 2-bit layout and bit e of word 2 is element e's high bit. One f16 scale per
//   `group` (32 or 64) values of a row; symmetric w = (q - 2^(bits-1)) * scale, asymmetric w = q * scale + bias.
//
// Three implementations, chosen by M (mnb_packed_path) as the reference chooses its kernels by M:
//   M <= 2   mnb_gemv_lanes_kernel: weight-bandwidth bound. A wave owns 4 output columns, its lanes run along K
//            over whole packed blocks, v_dot2_f32_f16 products, a cross-lane reduction.
//   M <= 16 (48 on small matrices)  mnb_gemv_kernel: a workgroup owns 16 output columns and its 8 waves split the
//            K blocks; each lane dequantises a whole packed block into the f16 B operands of
//            v_mfma_f32_16x16x32_f16 (no LDS), the a rows are the A operand (16 rows per tile, up to 4 tiles share
//            each dequantised operand), and the waves' partial sums meet in LDS.
//   above    compute bound: the weights are dequantised once (mnb_dequant_kernel) into an f16 copy the handle
//            keeps, and the product is a plain f16 GEMM with fp32 accumulation through hipBLASLt, on row slices of
//            at most 512 rows (the host side slices).
// All three dequantise with the same f16 arithmetic (dequant8_pk: each weight rounded to f16 once), accumulate in
// fp32 and round the output to f16.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <cmath>
#include <map>
#include <mutex>
#include <tuple>

#include "ha_kernels.h"

namespace ha {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

template <typename T>
using gptr = const __attribute__((address_space(1))) T*;
template <typename T>
__device__ __forceinline__ gptr<T> gp(const void* p) { return (gptr<T>)(p); }

constexpr int kBlk = 32;       // elements per packed block
constexpr int kLanesRows = 2;  // up to this many rows: mnb_gemv_lanes_kernel

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Elements 8 j .. 8 j + 7 of a packed block (its `BITS` words in registers), dequantised to f16 in the slot order
// (e0, e4, e1, e5, e2, e6, e3, e7) of the slice: each 32-bit pair holds elements i and i + 4, which one shift and
// mask extract from every bit width at once. A code q placed in the mantissa of 0x6400 (1024.0) is the f16 value
// 1024 + q exactly; subtracting 1024 + 2^(bits-1) leaves q - 2^(bits-1) exactly, and one f16 multiply by the scale
// (one f16 fma with the bias when asymmetric) rounds each weight once.
template <int BITS, bool ASYM>
__device__ __forceinline__ h8 dequant8_pk(const unsigned* wd, int j, h2 sc, h2 bi) {
  unsigned u, hb = 0;  // element i in the low half-word, element i + 4 in the high one, at bit (BITS==4 ? 4 : 2) i
  if constexpr (BITS == 4) {
    u = wd[j];
  } else {
    const unsigned lo = (wd[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
    u = (lo & 0xFFu) | ((lo & 0xFF00u) << 8);
    if constexpr (BITS == 3) {
      const unsigned hi = (wd[2] >> (8 * j)) & 0xFFu;
      hb = (hi & 0xFu) | ((hi & 0xF0u) << 12);
    }
  }
  constexpr unsigned kMask = BITS == 4 ? 0x000F000Fu : 0x00030003u;
  constexpr int kStep = BITS == 4 ? 4 : 2;
  const h2 off = ASYM ? h2{(_Float16)1024.0f, (_Float16)1024.0f}
                      : h2{(_Float16)(1024 + (1 << (BITS - 1))), (_Float16)(1024 + (1 << (BITS - 1)))};
  h8 r;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    unsigned c = (u >> (kStep * i)) & kMask;
    if constexpr (BITS == 3) c |= ((hb >> i) & 0x00010001u) << 2;
    const h2 q = __builtin_bit_cast(h2, c | 0x64006400u) - off;
    const h2 w = ASYM ? __builtin_elementwise_fma(q, sc, bi) : q * sc;
    r[2 * i] = w[0];
    r[2 * i + 1] = w[1];
  }
  return r;
}

// Eight consecutive f16 values of a row of a in the slot order dequant8_pk produces.
__device__ __forceinline__ h8 perm8(h8 x) {
  return h8{x[0], x[4], x[1], x[5], x[2], x[6], x[3], x[7]};
}

__device__ __forceinline__ h2 splat2(_Float16 v) { return h2{v, v}; }

// W16[n][k] = dequantised W, one 32-element block per thread.
template <int BITS, int GROUP, bool ASYM>
__global__ __launch_bounds__(256) void mnb_dequant_kernel(MnbArgs a, _Float16* w16) {
  const int nblk = a.K / kBlk;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)a.N * nblk) return;
  const long n = i / nblk;
  const int b = (int)(i % nblk);
  const long gi = n * (a.K / GROUP) + (long)b * kBlk / GROUP;
  const h2 sc = splat2(gp<_Float16>(a.s)[gi]);
  const h2 bi = splat2(ASYM ? gp<_Float16>(a.b)[gi] : (_Float16)0.0f);
  gptr<unsigned> wp = gp<unsigned>(a.q) + i * BITS;
  unsigned wd[BITS];
#pragma unroll
  for (int j = 0; j < BITS; j++) wd[j] = wp[j];
  __attribute__((address_space(1))) h8* dst = (__attribute__((address_space(1))) h8*)(w16 + n * a.K + (long)b * kBlk);
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const h8 v = dequant8_pk<BITS, ASYM>(wd, g, sc, bi);
    dst[g] = h8{v[0], v[2], v[4], v[6], v[1], v[3], v[5], v[7]};
  }
}

// y for M <= 16 MT rows. Workgroup: kGW waves, output columns 16 blockIdx.x .. +15; the K blocks go in groups of
// four, wave w taking groups w, w + kGW, ... Lane (g = lane / 16, c = lane % 16) loads the whole packed block b0 + g
// of column c (one 16-byte load for 4 bits) and the same 32 k of row 16 mt + c of a (four 16-byte loads; rows past M
// are not loaded and count as zero). The block's four 8-element slices are the B operands of four
// v_mfma_f32_16x16x32_f16, the matching slices of the a row their A operands: MFMA j sums, over the lane groups g,
// k = 32 (b0 + g) + 8 j .. + 7, so the four together cover the 128 k of the group (both operands carry their eight
// k in the slot order of dequant8_pk). The waves' partial sums meet in LDS.
constexpr int kGW = 8;
template <int BITS, int GROUP, bool ASYM, int MT, int U>
__global__ __launch_bounds__(64 * kGW) void mnb_gemv_kernel(MnbArgs a) {
  __shared__ f4 red[kGW][MT][64];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, c = lane & 15;
  const int nblk = a.K / kBlk, ngrp = (nblk + 3) >> 2;
  const int n = 16 * blockIdx.x + c;
  gptr<unsigned> wrow = gp<unsigned>(a.q) + (size_t)n * nblk * BITS;
  gptr<_Float16> srow = gp<_Float16>(a.s) + (size_t)n * (a.K / GROUP);
  gptr<_Float16> brow = ASYM ? gp<_Float16>(a.b) + (size_t)n * (a.K / GROUP) : srow;
  f4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) acc[mt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int g0 = w; g0 < ngrp; g0 += kGW * U) {
    unsigned wd[U][BITS];
    h2 sc[U], bi[U];
    h8 av[U][MT][4];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int b = 4 * (g0 + kGW * u) + g;
      ok[u] = b < nblk;
      const int bc = ok[u] ? b : nblk - 1;
      gptr<unsigned> wp = wrow + (size_t)bc * BITS;
#pragma unroll
      for (int j = 0; j < BITS; j++) wd[u][j] = wp[j];
      sc[u] = splat2(srow[bc * kBlk / GROUP]);
      bi[u] = splat2(ASYM ? brow[bc * kBlk / GROUP] : (_Float16)0.0f);
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        const int r = 16 * mt + c;
        if (ok[u] && r < a.M) {
          gptr<h8> ap = (gptr<h8>)(gp<_Float16>(a.a) + (size_t)r * a.K + (size_t)bc * kBlk);
#pragma unroll
          for (int j = 0; j < 4; j++) av[u][mt][j] = perm8(ap[j]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; j++) av[u][mt][j] = h8{};
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const h8 wv = ok[u] ? dequant8_pk<BITS, ASYM>(wd[u], j, sc[u], bi[u]) : h8{};
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
          acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[u][mt][j], wv, acc[mt], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; mt++) red[w][mt][lane] = acc[mt];
  __syncthreads();
  if (w < MT) {
    const int mt = w;
    f4 s = red[0][mt][lane];
#pragma unroll
    for (int j = 1; j < kGW; j++) s += red[j][mt][lane];
    // D layout: rows 4 g + e of the tile, column c
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int m = 16 * mt + 4 * g + e;
      if (m < a.M) ((_Float16*)a.y)[(size_t)m * a.N + n] = (_Float16)s[e];
    }
  }
}

// y for M = MR <= 2 rows: a wave owns kLW consecutive output columns and its lanes run along K. Lane l takes
// blocks l, l + 64, ... of each of its columns (one whole-block load per column, so a wave instruction reads a
// contiguous 1 KiB of one column's packed row), dequantises them to f16 pairs and multiplies them into the rows of a
// with v_dot2_f32_f16 (fp32 accumulation); the a values are loaded once per block for all the columns. The lanes'
// partial sums are reduced across the wave. Grid: N / (4 kLW) workgroups of 4 waves.
constexpr int kLW = 4;
template <int BITS, int GROUP, bool ASYM, int MR>
__global__ __launch_bounds__(256) void mnb_gemv_lanes_kernel(MnbArgs a) {
  const int lane = threadIdx.x & 63, n0 = kLW * (4 * blockIdx.x + (threadIdx.x >> 6));
  const int nblk = a.K / kBlk, ng = a.K / GROUP;
  float acc[kLW][MR];
#pragma unroll
  for (int c = 0; c < kLW; c++)
#pragma unroll
    for (int m = 0; m < MR; m++) acc[c][m] = 0.0f;
  for (int b = lane; b < nblk; b += 64) {
    unsigned wd[kLW][BITS];
    h2 sc[kLW], bi[kLW];
#pragma unroll
    for (int c = 0; c < kLW; c++) {
      gptr<unsigned> wp = gp<unsigned>(a.q) + ((size_t)(n0 + c) * nblk + b) * BITS;
#pragma unroll
      for (int j = 0; j < BITS; j++) wd[c][j] = wp[j];
      const size_t gi = (size_t)(n0 + c) * ng + b * kBlk / GROUP;
      sc[c] = splat2(gp<_Float16>(a.s)[gi]);
      bi[c] = splat2(ASYM ? gp<_Float16>(a.b)[gi] : (_Float16)0.0f);
    }
    h8 av[MR][4];
#pragma unroll
    for (int m = 0; m < MR; m++) {
      gptr<h8> ap = (gptr<h8>)(gp<_Float16>(a.a) + (size_t)min(m, a.M - 1) * a.K + (size_t)b * kBlk);
#pragma unroll
      for (int j = 0; j < 4; j++) av[m][j] = perm8(ap[j]);
    }
#pragma unroll
    for (int c = 0; c < kLW; c++) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const h8 wv = dequant8_pk<BITS, ASYM>(wd[c], j, sc[c], bi[c]);
#pragma unroll
        for (int m = 0; m < MR; m++)
#pragma unroll
          for (int p = 0; p < 4; p++)
            acc[c][m] = __builtin_amdgcn_fdot2(h2{av[m][j][2 * p], av[m][j][2 * p + 1]}, h2{wv[2 * p], wv[2 * p + 1]},
                                               acc[c][m], false);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < kLW; c++)
#pragma unroll
    for (int m = 0; m < MR; m++) {
      float v = acc[c][m];
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
      if (lane == 0 && m < a.M) ((_Float16*)a.y)[(size_t)m * a.N + n0 + c] = (_Float16)v;
    }
}

// In-place orthonormal Walsh-Hadamard transform (Sylvester order) of each contiguous n-block of an f16 row, one
// workgroup per block (wgsl.js:91-108): the online input rotation of a tensor exported with `had: n`.
__global__ __launch_bounds__(256) void fwht_kernel(_Float16* x, int n, float scale) {
  extern __shared__ float sh[];
  _Float16* o = x + (size_t)blockIdx.x * n;
  for (int e = threadIdx.x; e < n; e += 256) sh[e] = (float)o[e];
  __syncthreads();
  for (int h = 1; h < n; h *= 2) {
    for (int p = threadIdx.x; p < n / 2; p += 256) {
      const int i = (p / h) * 2 * h + p % h;
      const float u = sh[i], v = sh[i + h];
      sh[i] = u + v;
      sh[i + h] = u - v;
    }
    __syncthreads();
  }
  for (int e = threadIdx.x; e < n; e += 256) o[e] = (_Float16)(sh[e] * scale);
}

template <int BITS, int GROUP, bool ASYM>
hipError_t launch_gemv_lanes(const MnbArgs& a, hipStream_t s) {
  const dim3 grid(a.N / (4 * kLW)), block(256);
  if (a.M == 1) hipLaunchKernelGGL((mnb_gemv_lanes_kernel<BITS, GROUP, ASYM, 1>), grid, block, 0, s, a);
  else if (a.M == 2) hipLaunchKernelGGL((mnb_gemv_lanes_kernel<BITS, GROUP, ASYM, 2>), grid, block, 0, s, a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int BITS, int GROUP, bool ASYM>
hipError_t launch_gemv(const MnbArgs& a, hipStream_t s) {
  const dim3 grid(a.N / 16), block(64 * kGW);
  const int mt = (a.M + 15) / 16;
  if (mt == 1) hipLaunchKernelGGL((mnb_gemv_kernel<BITS, GROUP, ASYM, 1, 2>), grid, block, 0, s, a);
  else if (mt == 2) hipLaunchKernelGGL((mnb_gemv_kernel<BITS, GROUP, ASYM, 2, 2>), grid, block, 0, s, a);
  else if (mt == 3) hipLaunchKernelGGL((mnb_gemv_kernel<BITS, GROUP, ASYM, 3, 1>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((mnb_gemv_kernel<BITS, GROUP, ASYM, 4, 1>), grid, block, 0, s, a);
  return hipGetLastError();
}

template <int BITS, int GROUP, bool ASYM>
hipError_t launch_dequant(const MnbArgs& a, _Float16* w16, hipStream_t s) {
  const long n = (long)a.N * (a.K / kBlk);
  hipLaunchKernelGGL((mnb_dequant_kernel<BITS, GROUP, ASYM>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a, w16);
  return hipGetLastError();
}

// format dispatch: bits 2/3/4, group 32/64, symmetric or not
template <template <int, int, bool> class F, typename... Args>
hipError_t dispatch_fmt(const MnbArgs& a, Args... args) {
#define HA_MNB_CASE(B, G, S) \
  if (a.bits == B && a.group == G && a.asym == S) return F<B, G, S>::run(a, args...);
  HA_MNB_CASE(4, 32, false) HA_MNB_CASE(4, 32, true) HA_MNB_CASE(4, 64, false) HA_MNB_CASE(4, 64, true)
  HA_MNB_CASE(3, 32, false) HA_MNB_CASE(3, 32, true) HA_MNB_CASE(3, 64, false) HA_MNB_CASE(3, 64, true)
  HA_MNB_CASE(2, 32, false) HA_MNB_CASE(2, 32, true) HA_MNB_CASE(2, 64, false) HA_MNB_CASE(2, 64, true)
#undef HA_MNB_CASE
  return hipErrorInvalidValue;
}
template <int B, int G, bool S>
struct GemvLanesF {
  static hipError_t run(const MnbArgs& a, hipStream_t s) { return launch_gemv_lanes<B, G, S>(a, s); }
};
template <int B, int G, bool S>
struct GemvF {
  static hipError_t run(const MnbArgs& a, hipStream_t s) { return launch_gemv<B, G, S>(a, s); }
};
template <int B, int G, bool S>
struct DequantF {
  static hipError_t run(const MnbArgs& a, _Float16* w16, hipStream_t s) { return launch_dequant<B, G, S>(a, w16, s); }
};

}  // namespace

hipError_t mnb_check(const MnbArgs& a) {
  if (a.N <= 0 || a.K <= 0 || a.N % 16 || a.K % 32) return hipErrorInvalidValue;
  if (!(a.bits == 2 || a.bits == 3 || a.bits == 4) || !(a.group == 32 || a.group == 64) || a.K % a.group)
    return hipErrorInvalidValue;
  if (!a.q || !a.s || (a.asym && !a.b)) return hipErrorInvalidValue;
  return hipSuccess;
}

bool mnb_packed_path(int M, int N, int K) {
  // Measured on MI355X, back-to-back calls on the model's projection shapes (N x K from 2048 x 2048 to
  // 12288 x 2048): the library GEMM costs about 10 us at any M <= 64, the MFMA kernel 4-11 us up to 16 rows and
  // up to 48 rows on matrices of at most 2048 x 2048, more beyond.
  return M <= 16 || (M <= 48 && (long)N * K <= 2048L * 2048L);
}

hipError_t launch_mnb_gemv(const MnbArgs& a, hipStream_t s) {
  if (a.M < 1 || a.M > 64 || !a.a || !a.y) return hipErrorInvalidValue;
  return a.M <= kLanesRows ? dispatch_fmt<GemvLanesF>(a, s) : dispatch_fmt<GemvF>(a, s);
}

hipError_t launch_mnb_dequant(const MnbArgs& a, _Float16* w16, hipStream_t s) { return dispatch_fmt<DequantF>(a, w16, s); }

hipError_t launch_fwht(void* x, long rows_times_k, int n, hipStream_t s) {
  if (n < 2 || (n & (n - 1)) || n > 8192 || rows_times_k % n) return hipErrorInvalidValue;
  const float scale = (float)(1.0 / std::sqrt((double)n));  // the reference's constant 1 / sqrt(n), rounded to f32
  hipLaunchKernelGGL(fwht_kernel, dim3((unsigned)(rows_times_k / n)), dim3(256), sizeof(float) * n, s, (_Float16*)x, n,
                     scale);
  return hipGetLastError();
}

// ---- the hipBLASLt product above mnb_packed_path: y (col-major N x M, ld N) = W16^T (W16 col-major K x N, ld K, transposed)
// x a (col-major K x M, ld K) ----
struct LtPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};
struct LtGemm {
  hipblasLtHandle_t h = nullptr;
  void* ws = nullptr;
  size_t ws_bytes = 32u << 20;
  std::mutex mu;
  std::map<std::tuple<int, int, int>, LtPlan> plans;  // descriptors and algorithm per (M, N, K), kept for reuse
};

static LtGemm& lt_for_device(int dev) {
  static std::mutex m;
  static std::map<int, LtGemm*> per;
  std::lock_guard<std::mutex> g(m);
  LtGemm*& p = per[dev];
  if (!p) p = new LtGemm();  // one per device for the process lifetime
  return *p;
}

static bool make_plan(LtGemm& L, int M, int N, int K, LtPlan& p) {
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) return false;
  if (hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) != HIPBLAS_STATUS_SUCCESS)
    return false;
  if (hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16F, K, N, K) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16F, K, M, K) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_16F, N, M, N) != HIPBLAS_STATUS_SUCCESS)
    return false;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return false;
  const uint64_t wsb = L.ws_bytes;
  bool ok = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb)) ==
            HIPBLAS_STATUS_SUCCESS;
  hipblasLtMatmulHeuristicResult_t res[1];
  int got = 0;
  ok = ok && hipblasLtMatmulAlgoGetHeuristic(L.h, p.desc, p.la, p.lb, p.lc, p.lc, pref, 1, res, &got) ==
                 HIPBLAS_STATUS_SUCCESS &&
       got >= 1 && res[0].state == HIPBLAS_STATUS_SUCCESS && res[0].workspaceSize <= L.ws_bytes;
  hipblasLtMatmulPreferenceDestroy(pref);
  if (ok) p.algo = res[0].algo;
  return ok;
}

hipError_t lt_gemm_f16(int device, int M, int N, int K, const void* w16, const void* a, void* y, hipStream_t s) {
  LtGemm& L = lt_for_device(device);
  std::lock_guard<std::mutex> g(L.mu);
  if (!L.h) {
    if (hipblasLtCreate(&L.h) != HIPBLAS_STATUS_SUCCESS) return hipErrorUnknown;
    if (hipMalloc(&L.ws, L.ws_bytes) != hipSuccess) return hipErrorOutOfMemory;
  }
  auto key = std::make_tuple(M, N, K);
  auto it = L.plans.find(key);
  if (it == L.plans.end()) {
    LtPlan p;
    if (!make_plan(L, M, N, K, p)) {
      if (p.lc) hipblasLtMatrixLayoutDestroy(p.lc);
      if (p.lb) hipblasLtMatrixLayoutDestroy(p.lb);
      if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
      if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
      return hipErrorNotSupported;
    }
    it = L.plans.emplace(key, p).first;
  }
  const LtPlan& p = it->second;
  const float alpha = 1.0f, beta = 0.0f;
  if (hipblasLtMatmul(L.h, p.desc, &alpha, w16, p.la, a, p.lb, &beta, y, p.lc, y, p.lc, &p.algo, L.ws, L.ws_bytes, s) !=
      HIPBLAS_STATUS_SUCCESS)
    return hipErrorUnknown;
  return hipSuccess;
}

}  // namespace ha
