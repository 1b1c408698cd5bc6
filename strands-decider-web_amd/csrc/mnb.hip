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
// Two implementations, chosen by M as the reference chooses its kernels by M:
//   M <= 64  mnb_gemv_kernel: weight-bandwidth bound. A workgroup owns 16 output columns and its 8 waves split the
//            K blocks; each lane decodes 8 consecutive elements of one column's block straight into the f16 B
//            operand of v_mfma_f32_16x16x32_f16 (no LDS), the a rows are the A operand (16 rows per tile, up to 4
//            tiles share each decoded operand), and the waves' partial sums meet in LDS.
//   M > 64   compute bound: the weights are dequantised once (mnb_dequant_kernel) into an f16 copy the handle keeps,
//            and the product is a plain f16 GEMM with fp32 accumulation through hipBLASLt.
// Both round each dequantised weight to f16 once ((q - z) * scale is formed exactly, then rounded) and accumulate
// in fp32, and round the output to f16.
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

constexpr int kBlk = 32;  // elements per packed block

// The 8 quantised values of elements 8 g .. 8 g + 7 of packed block `blk` (its `BITS` u32 words start at wp).
template <int BITS>
__device__ __forceinline__ void decode8(gptr<unsigned> wp, int g, unsigned* q) {
  if constexpr (BITS == 4) {
    const unsigned w = wp[g];
#pragma unroll
    for (int i = 0; i < 8; i++) q[i] = (w >> (4 * i)) & 15u;
  } else {
    const unsigned lo = wp[g >> 1] >> (16 * (g & 1));
#pragma unroll
    for (int i = 0; i < 8; i++) q[i] = (lo >> (2 * i)) & 3u;
    if constexpr (BITS == 3) {
      const unsigned hi = wp[2] >> (8 * g);
#pragma unroll
      for (int i = 0; i < 8; i++) q[i] |= ((hi >> i) & 1u) << 2;
    }
  }
}

template <int BITS, bool ASYM>
__device__ __forceinline__ _Float16 dequant(unsigned q, float sc, float bi) {
  if constexpr (ASYM)
    return (_Float16)fmaf((float)q, sc, bi);
  else
    return (_Float16)((float)((int)q - (1 << (BITS - 1))) * sc);
}

// W16[n][k] = dequantised W, one 32-element block per thread.
template <int BITS, int GROUP, bool ASYM>
__global__ __launch_bounds__(256) void mnb_dequant_kernel(MnbArgs a, _Float16* w16) {
  const int nblk = a.K / kBlk;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)a.N * nblk) return;
  const long n = i / nblk;
  const int b = (int)(i % nblk);
  const long gi = n * (a.K / GROUP) + (long)b * kBlk / GROUP;
  const float sc = (float)gp<_Float16>(a.s)[gi];
  const float bi = ASYM ? (float)gp<_Float16>(a.b)[gi] : 0.0f;
  gptr<unsigned> wp = gp<unsigned>(a.q) + i * BITS;
  __attribute__((address_space(1))) h8* dst = (__attribute__((address_space(1))) h8*)(w16 + n * a.K + (long)b * kBlk);
#pragma unroll
  for (int g = 0; g < 4; g++) {
    unsigned q[8];
    decode8<BITS>(wp, g, q);
    h8 v;
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = dequant<BITS, ASYM>(q[e], sc, bi);
    dst[g] = v;
  }
}

// y for M <= 16 MT rows. Workgroup: 8 waves, output columns 16 blockIdx.x .. +15; wave w takes K blocks w, w + 8,
// ... Lane (g = lane / 16, c = lane % 16): B operand = elements 8 g .. 8 g + 7 of column c's block; A operand = row
// 16 mt + c, the same 8 k. Rows past M read row M - 1 and are not stored.
constexpr int kGW = 8;
template <int BITS, int GROUP, bool ASYM, int MT>
__global__ __launch_bounds__(64 * kGW) void mnb_gemv_kernel(MnbArgs a) {
  __shared__ f4 red[kGW][MT][64];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, c = lane & 15;
  const int nblk = a.K / kBlk;
  const int n = 16 * blockIdx.x + c;
  gptr<unsigned> wrow = gp<unsigned>(a.q) + (size_t)n * nblk * BITS;
  gptr<_Float16> srow = gp<_Float16>(a.s) + (size_t)n * (a.K / GROUP);
  gptr<_Float16> brow = ASYM ? gp<_Float16>(a.b) + (size_t)n * (a.K / GROUP) : srow;
  gptr<_Float16> arow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) arow[mt] = gp<_Float16>(a.a) + (size_t)min(16 * mt + c, a.M - 1) * a.K + 8 * g;
  f4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) acc[mt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int U = 4;  // blocks in flight per wave
  for (int b0 = w; b0 < nblk; b0 += kGW * U) {
    unsigned q[U][8];
    float sc[U], bi[U];
    h8 av[U][MT];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int b = min(b0 + kGW * u, nblk - 1);
      decode8<BITS>(wrow + (size_t)b * BITS, g, q[u]);
      sc[u] = (float)srow[b * kBlk / GROUP];
      bi[u] = ASYM ? (float)brow[b * kBlk / GROUP] : 0.0f;
#pragma unroll
      for (int mt = 0; mt < MT; mt++) av[u][mt] = *(gptr<h8>)(arow[mt] + (size_t)b * kBlk);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      if (b0 + kGW * u < nblk) {
        h8 wv;
#pragma unroll
        for (int e = 0; e < 8; e++) wv[e] = dequant<BITS, ASYM>(q[u][e], sc[u], bi[u]);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[u][mt], wv, acc[mt], 0, 0, 0);
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
hipError_t launch_gemv(const MnbArgs& a, hipStream_t s) {
  const dim3 grid(a.N / 16), block(64 * kGW);
  const int mt = (a.M + 15) / 16;
  if (mt == 1) hipLaunchKernelGGL((mnb_gemv_kernel<BITS, GROUP, ASYM, 1>), grid, block, 0, s, a);
  else if (mt == 2) hipLaunchKernelGGL((mnb_gemv_kernel<BITS, GROUP, ASYM, 2>), grid, block, 0, s, a);
  else if (mt == 3) hipLaunchKernelGGL((mnb_gemv_kernel<BITS, GROUP, ASYM, 3>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((mnb_gemv_kernel<BITS, GROUP, ASYM, 4>), grid, block, 0, s, a);
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

hipError_t launch_mnb_gemv(const MnbArgs& a, hipStream_t s) {
  if (a.M < 1 || a.M > 64 || !a.a || !a.y) return hipErrorInvalidValue;
  return dispatch_fmt<GemvF>(a, s);
}

hipError_t launch_mnb_dequant(const MnbArgs& a, _Float16* w16, hipStream_t s) { return dispatch_fmt<DequantF>(a, w16, s); }

hipError_t launch_fwht(void* x, long rows_times_k, int n, hipStream_t s) {
  if (n < 2 || (n & (n - 1)) || n > 8192 || rows_times_k % n) return hipErrorInvalidValue;
  const float scale = (float)(1.0 / std::sqrt((double)n));  // the reference's constant 1 / sqrt(n), rounded to f32
  hipLaunchKernelGGL(fwht_kernel, dim3((unsigned)(rows_times_k / n)), dim3(256), sizeof(float) * n, s, (_Float16*)x, n,
                     scale);
  return hipGetLastError();
}

// ---- the hipBLASLt product for M > 64: y (col-major N x M, ld N) = W16^T (W16 col-major K x N, ld K, transposed)
// x a (col-major K x M, ld K) ----
struct LtGemm {
  hipblasLtHandle_t h = nullptr;
  void* ws = nullptr;
  size_t ws_bytes = 32u << 20;
  std::mutex mu;
  std::map<std::tuple<int, int, int>, hipblasLtMatmulAlgo_t> algos;
};

static LtGemm& lt_for_device(int dev) {
  static std::mutex m;
  static std::map<int, LtGemm*> per;
  std::lock_guard<std::mutex> g(m);
  LtGemm*& p = per[dev];
  if (!p) p = new LtGemm();  // one per device for the process lifetime
  return *p;
}

hipError_t lt_gemm_f16(int device, int M, int N, int K, const void* w16, const void* a, void* y, hipStream_t s) {
  LtGemm& L = lt_for_device(device);
  std::lock_guard<std::mutex> g(L.mu);
  if (!L.h) {
    if (hipblasLtCreate(&L.h) != HIPBLAS_STATUS_SUCCESS) return hipErrorUnknown;
    if (hipMalloc(&L.ws, L.ws_bytes) != hipSuccess) return hipErrorOutOfMemory;
  }
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulPreference_t pref = nullptr;
  hipError_t ret = hipErrorUnknown;
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  const float alpha = 1.0f, beta = 0.0f;
  do {
    if (hipblasLtMatmulDescCreate(&desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) break;
    if (hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) != HIPBLAS_STATUS_SUCCESS)
      break;
    if (hipblasLtMatrixLayoutCreate(&la, HIP_R_16F, K, N, K) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&lb, HIP_R_16F, K, M, K) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&lc, HIP_R_16F, N, M, N) != HIPBLAS_STATUS_SUCCESS)
      break;
    auto key = std::make_tuple(M, N, K);
    auto it = L.algos.find(key);
    if (it == L.algos.end()) {
      if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) break;
      const uint64_t wsb = L.ws_bytes;
      hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb));
      hipblasLtMatmulHeuristicResult_t res[1];
      int got = 0;
      if (hipblasLtMatmulAlgoGetHeuristic(L.h, desc, la, lb, lc, lc, pref, 1, res, &got) != HIPBLAS_STATUS_SUCCESS ||
          got < 1)
        break;
      it = L.algos.emplace(key, res[0].algo).first;
    }
    if (hipblasLtMatmul(L.h, desc, &alpha, w16, la, a, lb, &beta, y, lc, y, lc, &it->second, L.ws, L.ws_bytes, s) !=
        HIPBLAS_STATUS_SUCCESS)
      break;
    ret = hipSuccess;
  } while (false);
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (lc) hipblasLtMatrixLayoutDestroy(lc);
  if (lb) hipblasLtMatrixLayoutDestroy(lb);
  if (la) hipblasLtMatrixLayoutDestroy(la);
  if (desc) hipblasLtMatmulDescDestroy(desc);
  return ret;
}

}  // namespace ha
