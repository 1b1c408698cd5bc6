// Sequential gated-delta rule for decode / resume (ha_recurrence HA_SEQUENTIAL), gfx950.
//
// Semantics: the engine's CONV + GDN + GNORM steps (reference web/public/engine/wgsl.js:124-139, 146-187, 252-268)
// with the third-party fp32 rule they restate (transformers qwen3_5 torch_recurrent_gated_delta_rule):
//   u = silu(conv4(x)); q^ = q rsqrt(|q|^2 + 1e-6) / sqrt(DK); k^ = k rsqrt(|k|^2 + 1e-6)
//   beta = sigmoid(b); alpha = exp(negA * softplus(a + dt_bias))
//   S <- alpha S; delta = beta (v - S^T k^); S <- S + k^ delta^T; o = S^T q^
//   y = gnorm * o * rsqrt(mean(o^2) + 1e-6) * silu(z)
//
// Layout: one workgroup of 4 waves per (sequence, head). Lane l of wave w owns value column j = 32w + (l & 31)
// and key rows [64 * (l >> 5), +64): its 64 state entries stay in VGPRs for the whole call. Each wave computes
// the conv, the norms (wave reductions, no barrier) and q^/k^ redundantly and broadcasts them through a
// wave-private LDS slot, so the token loop has no workgroup barrier; the two key halves of a column are combined
// with one cross-lane swap. Raw outputs go to an LDS ring that is normalised (GNORM) every 16 tokens.
#include "ha_kernels.h"

namespace ha {
namespace {

constexpr int kDK = 128, kDV = 128, kKC = 4, kRing = 16;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

__device__ __forceinline__ float silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

template <typename T>
__device__ __forceinline__ const T* row_of(const GdnArgs& a, int b, int r) {
  if (r < a.P) return static_cast<const T*>(a.tail) + ((size_t)b * a.tail_cap + (r - (a.s0 - (kKC - 1)))) * a.stride;
  return static_cast<const T*>(a.in) + ((size_t)b * a.L + (r - a.P)) * a.stride;
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <typename T>
__global__ __launch_bounds__(256) void gdn_seq_kernel(GdnArgs a) {
  const int b = blockIdx.x / a.H, h = blockIdx.x % a.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int j = wave * 32 + (lane & 31);
  const int half = lane >> 5;

  __shared__ float qk[4][2][kDK];     // wave-private q^ (0) and k^ (1)
  __shared__ float ring[kRing][kDV];  // raw outputs awaiting the gated norm

  const size_t sbase = ((size_t)b * a.H + h) * kDK * kDV;
  float S[64];
#pragma unroll
  for (int i = 0; i < 64; i++) S[i] = a.S_in ? a.S_in[sbase + (size_t)(64 * half + i) * kDV + j] : 0.0f;

  // channels handled by this lane: q dims lane, lane+64; k dims lane, lane+64; v column j
  const int cq0 = h * kDK + lane, cq1 = cq0 + 64;
  const int ck0 = a.H * kDK + h * kDK + lane, ck1 = ck0 + 64;
  const int cv = 2 * a.H * kDK + h * kDV + j;
  const int cidx[5] = {cq0, cq1, ck0, ck1, cv};
  float w[5][kKC], hx[5][kKC - 1];
#pragma unroll
  for (int c = 0; c < 5; c++)
#pragma unroll
    for (int t = 0; t < kKC; t++) w[c][t] = a.conv_w[(size_t)cidx[c] * kKC + t];
  // conv history: raw rows s0-3 .. s0-1
#pragma unroll
  for (int t = 0; t < kKC - 1; t++) {
    const T* row = row_of<T>(a, b, a.s0 - (kKC - 1) + t);
#pragma unroll
    for (int c = 0; c < 5; c++) hx[c][t] = (float)row[cidx[c]];
  }
  const float na = a.negA[h], db = a.dtb[h];
  const int aoff = a.C + a.H * a.DV + h, boff = aoff + a.H;
  const float qscale = 0.08838834764831845f;  // 1/sqrt(128)
  const int end = a.P + a.L;

  for (int r = a.s0; r < end; ++r) {
    const T* row = row_of<T>(a, b, r);
    float u[5];
#pragma unroll
    for (int c = 0; c < 5; c++) {
      const float x = (float)row[cidx[c]];
      float s = w[c][0] * hx[c][0];
      s = fmaf(w[c][1], hx[c][1], s);
      s = fmaf(w[c][2], hx[c][2], s);
      s = fmaf(w[c][3], x, s);
      hx[c][0] = hx[c][1];
      hx[c][1] = hx[c][2];
      hx[c][2] = x;
      u[c] = silu(s);
    }
    const float av = (float)row[aoff], bv = (float)row[boff];
    const float ssq = wave_sum(u[0] * u[0] + u[1] * u[1]);
    const float ssk = wave_sum(u[2] * u[2] + u[3] * u[3]);
    const float rq = rsqrtf(ssq + 1e-6f) * qscale, rk = rsqrtf(ssk + 1e-6f);
    qk[wave][0][lane] = u[0] * rq;
    qk[wave][0][lane + 64] = u[1] * rq;
    qk[wave][1][lane] = u[2] * rk;
    qk[wave][1][lane + 64] = u[3] * rk;
    wave_sync();
    const float beta = __builtin_amdgcn_rcpf(1.0f + __expf(-bv));
    const float xs = av + db;
    const float sp = xs > 20.0f ? xs : log1pf(__expf(xs));
    const float alpha = __expf(na * sp);

    const float4* kv4 = reinterpret_cast<const float4*>(&qk[wave][1][64 * half]);
    const float4* qv4 = reinterpret_cast<const float4*>(&qk[wave][0][64 * half]);
    float kr = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float4 k4 = kv4[i];
      S[4 * i + 0] *= alpha; S[4 * i + 1] *= alpha; S[4 * i + 2] *= alpha; S[4 * i + 3] *= alpha;
      kr = fmaf(S[4 * i + 0], k4.x, kr);
      kr = fmaf(S[4 * i + 1], k4.y, kr);
      kr = fmaf(S[4 * i + 2], k4.z, kr);
      kr = fmaf(S[4 * i + 3], k4.w, kr);
    }
    kr += __shfl_xor(kr, 32);
    const float delta = beta * (u[4] - kr);
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float4 k4 = kv4[i], q4 = qv4[i];
      S[4 * i + 0] = fmaf(k4.x, delta, S[4 * i + 0]);
      S[4 * i + 1] = fmaf(k4.y, delta, S[4 * i + 1]);
      S[4 * i + 2] = fmaf(k4.z, delta, S[4 * i + 2]);
      S[4 * i + 3] = fmaf(k4.w, delta, S[4 * i + 3]);
      o = fmaf(S[4 * i + 0], q4.x, o);
      o = fmaf(S[4 * i + 1], q4.y, o);
      o = fmaf(S[4 * i + 2], q4.z, o);
      o = fmaf(S[4 * i + 3], q4.w, o);
    }
    o += __shfl_xor(o, 32);
    wave_sync();

    if (r >= a.P) {
      const int t = r - a.P;
      if (half == 0) ring[t % kRing][j] = o;
      if (t % kRing == kRing - 1 || r == end - 1) {
        __syncthreads();
        // gated norm of the buffered rows: thread -> (row tid / 16, columns 8 * (tid % 16) .. +8)
        const int n = t % kRing + 1, rr = tid >> 4, c0 = (tid & 15) * 8;
        const int tt = t - (n - 1) + rr;
        float v[8], ss = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) { v[c] = ring[rr][c0 + c]; ss += v[c] * v[c]; }
#pragma unroll
        for (int m = 1; m < 16; m <<= 1) ss += __shfl_xor(ss, m);
        if (rr < n) {
          const size_t ob = ((size_t)b * a.L + tt) * (size_t)(a.H * kDV) + (size_t)h * kDV + c0;
          if (a.gnorm) {
            const float inv = rsqrtf(ss / kDV + 1e-6f);
            const T* zrow = static_cast<const T*>(a.in) + ((size_t)b * a.L + tt) * a.stride + a.C + h * kDV + c0;
#pragma unroll
            for (int c = 0; c < 8; c++) v[c] = a.gnorm[c0 + c] * v[c] * inv * silu((float)zrow[c]);
          }
          T* op = static_cast<T*>(a.out) + ob;
#pragma unroll
          for (int c = 0; c < 8; c++) op[c] = (T)v[c];
        }
        __syncthreads();
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 64; i++) a.S_out[sbase + (size_t)(64 * half + i) * kDV + j] = S[i];
}

}  // namespace

hipError_t launch_gdn_sequential(const GdnArgs& a, hipStream_t s) {
  if (a.DK != kDK || a.DV != kDV || a.KC != kKC) return hipErrorInvalidValue;
  dim3 grid(a.B * a.H), block(256);
  if (a.dtype == 0)
    hipLaunchKernelGGL(gdn_seq_kernel<float>, grid, block, 0, s, a);
  else
    hipLaunchKernelGGL(gdn_seq_kernel<_Float16>, grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace ha
