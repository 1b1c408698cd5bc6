// The rest of the torso's per-layer work around the token mixers and the projections, gfx950: the embedding
// gather, the residual add + RMSNorm before each projection, the MLP's SiLU gate and an adapter layer's bias.
//
// Reference: web/public/engine/wgsl.js:33-52 (EMBED), 55-78 (ADD_NORM), 81-90 (SILU_MUL), 113-121 (ADD_BIAS), and
// their dispatch in Engine.plan(), web/public/engine/engine.js:247-281 (final-norm row gather: engine.js:283-284,
// 342). All are HBM-bound: each element is read and written once, in 16-byte accesses.
#include <hip/hip_runtime.h>

#include "ha_kernels.h"

namespace ha {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// x[t][0..D) = dequantised row ids[t] of the quantised table (f32, the reference's arithmetic: (q - z) * scale or
// q * scale + bias in f32). One thread per 8 elements (a quarter block), D / 8 threads per row.
template <int BITS, int GROUP, bool ASYM>
__global__ __launch_bounds__(256) void embed_kernel(EmbedArgs a) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;  // (row, 8-element group)
  const int per_row = a.D / 8;
  if (i >= (long)a.L * per_row) return;
  const int t = (int)(i / per_row), g8 = (int)(i % per_row);
  const unsigned id = a.ids[t];
  f4* dst = reinterpret_cast<f4*>(a.x + (size_t)t * a.D + 8 * g8);
  if (id >= (unsigned)a.rows) {  // not a row of the table: a NaN row, not an out-of-bounds read
    dst[0] = dst[1] = f4{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
    return;
  }
  const int nblk = a.D / 32, blk = g8 / 4, j = g8 % 4;  // block of the row, quarter of the block
  const unsigned* wp = a.q + ((size_t)id * nblk + blk) * BITS;
  const size_t gi = (size_t)id * (a.D / GROUP) + blk * 32 / GROUP;
  const float sc = (float)a.s[gi];
  const float bi = ASYM ? (float)a.b[gi] : 0.0f;
  unsigned q[8];
  if constexpr (BITS == 4) {
    const unsigned w = wp[j];
#pragma unroll
    for (int e = 0; e < 8; e++) q[e] = (w >> (4 * e)) & 15u;
  } else {
    const unsigned lo = wp[j >> 1] >> (16 * (j & 1));
#pragma unroll
    for (int e = 0; e < 8; e++) q[e] = (lo >> (2 * e)) & 3u;
    if constexpr (BITS == 3) {
      const unsigned hi = wp[2] >> (8 * j);
#pragma unroll
      for (int e = 0; e < 8; e++) q[e] |= ((hi >> e) & 1u) << 2;
    }
  }
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; e++)
    v[e] = ASYM ? (float)q[e] * sc + bi : ((float)q[e] - (float)(1 << (BITS - 1))) * sc;
  dst[0] = f4{v[0], v[1], v[2], v[3]};
  dst[1] = f4{v[4], v[5], v[6], v[7]};
}

// Output row r of the norm reads source row rows[r] (identity when rows is NULL). With y, x[src] += y[src] first
// (written back, f32). Then h[r] = x[src] * rsqrt(mean(x[src]^2) + eps) * w, f16 or f32. One workgroup of 256
// threads per output row; a thread holds 8 consecutive elements per 2048-column pass.
template <bool ADD, bool OUT_F32>
__global__ __launch_bounds__(256) void add_norm_kernel(AddNormArgs a) {
  __shared__ float red[4];
  const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const unsigned srcu = a.rows ? a.rows[r] : (unsigned)r;
  if (srcu >= (unsigned)a.nx) {  // not a row of x: a NaN output row, not an out-of-bounds access
    for (int c = tid; c < a.D; c += 256) {
      if (OUT_F32) ((float*)a.h)[(size_t)r * a.D + c] = __builtin_nanf("");
      else ((_Float16*)a.h)[(size_t)r * a.D + c] = (_Float16)__builtin_nanf("");
    }
    return;
  }
  const int src = (int)srcu;
  float* xr = a.x + (size_t)src * a.D;
  const _Float16* yr = ADD ? a.y + (size_t)src * a.D : nullptr;
  constexpr int kMaxPass = 4;  // D <= 4 * 2048
  float v[kMaxPass][8];
  float ss = 0.0f;
#pragma unroll
  for (int p = 0; p < kMaxPass; p++) {
    const int c = 8 * (tid + 256 * p);
    if (c < a.D) {
      const f4 x0 = *reinterpret_cast<const f4*>(xr + c), x1 = *reinterpret_cast<const f4*>(xr + c + 4);
      float t[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
      if constexpr (ADD) {
        const h8 yv = *reinterpret_cast<const h8*>(yr + c);
#pragma unroll
        for (int e = 0; e < 8; e++) t[e] += (float)yv[e];
        *reinterpret_cast<f4*>(xr + c) = f4{t[0], t[1], t[2], t[3]};
        *reinterpret_cast<f4*>(xr + c + 4) = f4{t[4], t[5], t[6], t[7]};
      }
#pragma unroll
      for (int e = 0; e < 8; e++) {
        v[p][e] = t[e];
        ss = fmaf(t[e], t[e], ss);
      }
    }
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d);
  if (lane == 0) red[w] = ss;
  __syncthreads();
  const float inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)a.D + a.eps);
#pragma unroll
  for (int p = 0; p < kMaxPass; p++) {
    const int c = 8 * (tid + 256 * p);
    if (c < a.D) {
      const f4 w0 = *reinterpret_cast<const f4*>(a.w + c), w1 = *reinterpret_cast<const f4*>(a.w + c + 4);
      const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
      if constexpr (OUT_F32) {
        float* hr = (float*)a.h + (size_t)r * a.D + c;
        *reinterpret_cast<f4*>(hr) = f4{v[p][0] * inv * wv[0], v[p][1] * inv * wv[1], v[p][2] * inv * wv[2],
                                        v[p][3] * inv * wv[3]};
        *reinterpret_cast<f4*>(hr + 4) = f4{v[p][4] * inv * wv[4], v[p][5] * inv * wv[5], v[p][6] * inv * wv[6],
                                            v[p][7] * inv * wv[7]};
      } else {
        h8 o;
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = (_Float16)(v[p][e] * inv * wv[e]);
        *reinterpret_cast<h8*>((_Float16*)a.h + (size_t)r * a.D + c) = o;
      }
    }
  }
}

// mid[t][j] = silu(big[t][j]) * big[t][I + j], f16 in and out, f32 arithmetic. 8 elements per thread.
__global__ __launch_bounds__(256) void silu_mul_kernel(const _Float16* big, _Float16* mid, long n8, int I) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const int per_row = I / 8;
  const long t = i / per_row;
  const int j = (int)(i % per_row) * 8;
  const h8 g = *reinterpret_cast<const h8*>(big + (size_t)t * 2 * I + j);
  const h8 u = *reinterpret_cast<const h8*>(big + (size_t)t * 2 * I + I + j);
  h8 o;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const float gv = (float)g[e];
    o[e] = (_Float16)(gv / (1.0f + __expf(-gv)) * (float)u[e]);
  }
  *reinterpret_cast<h8*>(mid + (size_t)t * I + j) = o;
}

// y[t][j] = y[t][j] + c[j] (f16 y, f32 c). 8 elements per thread.
__global__ __launch_bounds__(256) void add_bias_kernel(_Float16* y, const float* c, long n8, int N) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const int j = (int)((i * 8) % N);
  h8 v = *reinterpret_cast<const h8*>(y + 8 * i);
  const f4 c0 = *reinterpret_cast<const f4*>(c + j), c1 = *reinterpret_cast<const f4*>(c + j + 4);
  const float cv[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
#pragma unroll
  for (int e = 0; e < 8; e++) v[e] = (_Float16)((float)v[e] + cv[e]);
  *reinterpret_cast<h8*>(y + 8 * i) = v;
}

unsigned blocks_for(long n) { return (unsigned)((n + 255) / 256); }

}  // namespace

hipError_t launch_embed(const EmbedArgs& a, hipStream_t s) {
  if (a.L < 1 || a.rows < 1 || a.D % 32 || a.D < 32 || !(a.bits == 2 || a.bits == 3 || a.bits == 4) ||
      !(a.group == 32 || a.group == 64) || a.D % a.group || (a.asym && !a.b))
    return hipErrorInvalidValue;
  const dim3 grid(blocks_for((long)a.L * a.D / 8)), block(256);
#define HA_EMBED_CASE(B, G, S)                                                       \
  if (a.bits == B && a.group == G && a.asym == S) {                                  \
    hipLaunchKernelGGL((embed_kernel<B, G, S>), grid, block, 0, s, a);               \
    return hipGetLastError();                                                        \
  }
  HA_EMBED_CASE(4, 32, false) HA_EMBED_CASE(4, 32, true) HA_EMBED_CASE(4, 64, false) HA_EMBED_CASE(4, 64, true)
  HA_EMBED_CASE(3, 32, false) HA_EMBED_CASE(3, 32, true) HA_EMBED_CASE(3, 64, false) HA_EMBED_CASE(3, 64, true)
  HA_EMBED_CASE(2, 32, false) HA_EMBED_CASE(2, 32, true) HA_EMBED_CASE(2, 64, false) HA_EMBED_CASE(2, 64, true)
#undef HA_EMBED_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_add_norm(const AddNormArgs& a, hipStream_t s) {
  if (a.R < 1 || a.nx < 1 || a.D < 8 || a.D % 8 || a.D > 4 * 2048) return hipErrorInvalidValue;
  const dim3 grid(a.R), block(256);
  if (a.y) {
    if (a.out_f32) hipLaunchKernelGGL((add_norm_kernel<true, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((add_norm_kernel<true, false>), grid, block, 0, s, a);
  } else {
    if (a.out_f32) hipLaunchKernelGGL((add_norm_kernel<false, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((add_norm_kernel<false, false>), grid, block, 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_silu_mul(const void* big, void* mid, int L, int I, hipStream_t s) {
  if (L < 1 || I < 8 || I % 8) return hipErrorInvalidValue;
  const long n8 = (long)L * I / 8;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks_for(n8)), dim3(256), 0, s, (const _Float16*)big, (_Float16*)mid,
                     n8, I);
  return hipGetLastError();
}

hipError_t launch_add_bias(void* y, const float* c, int L, int N, hipStream_t s) {
  if (L < 1 || N < 8 || N % 8) return hipErrorInvalidValue;
  const long n8 = (long)L * N / 8;
  hipLaunchKernelGGL(add_bias_kernel, dim3(blocks_for(n8)), dim3(256), 0, s, (_Float16*)y, c, n8, N);
  return hipGetLastError();
}

}  // namespace ha
