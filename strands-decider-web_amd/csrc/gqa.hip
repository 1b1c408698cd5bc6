// Gated causal GQA attention for the full_attention layers, gfx950.
//
// Semantics (reference web/public/engine/wgsl.js:271-302 QK_PREP and 348-417 ATTN2; third-party fp32 form:
// transformers qwen3_5 Qwen3_5RMSNorm, apply_rotary_pos_emb, eager_attention_forward, sigmoid(gate)):
//   q~ = q rsqrt(mean(q^2) + 1e-6) * qw,  k~ likewise with kw   (qw, kw are the stored 1 + w)
//   rotate-half RoPE on dims [0, RD) at absolute position P + t (engine.js:105-106 table)
//   K[kh][P+t] = f16(k~'), V[kh][P+t] = f16(v), Q = f16(f16(q~') / sqrt(HD))
//   out = softmax_j<=P+t(Q . K_j) V * sigmoid(gate)
//
// gqa_prep_kernel: one wave per (sequence, row, head slot); RMS via a wave reduction, the RoPE partner dim via a
//   lane swap (d <-> d +- RD/2), f16 stores into the Q scratch and the K/V cache.
// gqa_attn_kernel: one workgroup per (sequence, KV head, block of 32 query rows) with one wave per query head of
//   the KV group, so each 64-key K/V tile is staged once in LDS and consumed by all G heads. S^T = K Q^T and
//   O += P V run on v_mfma_f32_16x16x32_f16 with fp32 accumulation; Q stays in VGPRs; the online softmax
//   (max / exp2 / sum in fp32) works on the S^T accumulators directly, which already have the A-operand shape P
//   needs for P V. The next tile is fetched into registers while the current one is consumed.
#include "ha_kernels.h"

namespace ha {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kHD = 256, kBQ = 32, kBK = 64, kKPad = 8, kVPad = 8;
constexpr int kKRow = kHD + kKPad;  // halves per K row in LDS
constexpr int kVRow = kBK + kVPad;  // halves per transposed-V row in LDS
constexpr size_t kAttnLds = sizeof(_Float16) * (size_t)(kBK * kKRow + kHD * kVRow);

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

template <typename T>
__global__ __launch_bounds__(256) void gqa_prep_kernel(GqaArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int NS = a.HQ + a.HK;
  const long item = (long)blockIdx.x * 4 + wave;
  if (item >= (long)a.B * a.L * NS) return;
  const int s = (int)(item % NS);
  const long bt = item / NS;
  const int t = (int)(bt % a.L), b = (int)(bt / a.L);
  const int HD = a.HD, RD = a.RD, pos = a.P + t;
  const T* row = static_cast<const T*>(a.in) + ((size_t)b * a.L + t) * a.stride;
  const bool isq = s < a.HQ;
  const T* src = isq ? row + (size_t)s * 2 * HD : row + (size_t)a.HQ * 2 * HD + (size_t)(s - a.HQ) * HD;
  const int nper = HD / 64;  // dims lane + 64 i
  float v[8], ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++)
    if (i < nper) { v[i] = (float)src[lane + 64 * i]; ss += v[i] * v[i]; }
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / HD + 1e-6f);
  const float* w = isq ? a.qw : a.kw;
#pragma unroll
  for (int i = 0; i < 8; i++)
    if (i < nper) v[i] = v[i] * inv * w[lane + 64 * i];
  // rotate-half on dims [0, RD): dim d pairs with d + RD/2 (d < RD/2) or d - RD/2; all of them are in v[0]
  const float partner = __shfl_xor(v[0], RD / 2);
  if (lane < RD) {
    const int i = lane % (RD / 2);
    const float cs = a.rope[(size_t)pos * RD + 2 * i], sn = a.rope[(size_t)pos * RD + 2 * i + 1];
    v[0] = lane < RD / 2 ? v[0] * cs - partner * sn : v[0] * cs + partner * sn;
  }
  if (isq) {
    const float scale = rsqrtf((float)HD);
    _Float16* dst = a.Q + (((size_t)b * a.HQ + s) * a.L + t) * HD;
#pragma unroll
    for (int i = 0; i < 8; i++)
      if (i < nper) dst[lane + 64 * i] = (_Float16)((float)(_Float16)v[i] * scale);
  } else {
    const int kh = s - a.HQ;
    const size_t cb = (((size_t)b * a.HK + kh) * a.LT + pos) * HD;
    const T* vs = row + (size_t)a.HQ * 2 * HD + (size_t)a.HK * HD + (size_t)kh * HD;
#pragma unroll
    for (int i = 0; i < 8; i++)
      if (i < nper) {
        a.K[cb + lane + 64 * i] = (_Float16)v[i];
        a.V[cb + lane + 64 * i] = (_Float16)(float)vs[lane + 64 * i];
      }
  }
}

template <int G, typename T>
__global__ __launch_bounds__(64 * G) void gqa_attn_kernel(GqaArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  _Float16* Ks = reinterpret_cast<_Float16*>(lds_raw);  // [kBK][kKRow]
  _Float16* Vt = Ks + kBK * kKRow;                      // [kHD][kVRow], transposed V tile

  const int nqb = (a.L + kBQ - 1) / kBQ;
  const int qb = nqb - 1 - (int)blockIdx.x;  // longest causal rows first
  const int kh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h = kh * G + wave;
  const int g = lane >> 4, c16 = lane & 15;
  const int q0 = qb * kBQ;
  constexpr int NT = 64 * G;

  // Q rows as the B operand of S^T = K Q^T: qreg[rt][ks] = Q[q0 + 16 rt + c16][32 ks + 8 g .. +7]
  h8 qreg[2][8];
  const _Float16* Qh = a.Q + ((size_t)b * a.HQ + h) * a.L * kHD;
#pragma unroll
  for (int rt = 0; rt < 2; rt++) {
    const int t = q0 + 16 * rt + c16;
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
      h8 z = {};
      qreg[rt][ks] = t < a.L ? *reinterpret_cast<const h8*>(Qh + (size_t)t * kHD + 32 * ks + 8 * g) : z;
    }
  }

  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};
  f4 O[2][16];
#pragma unroll
  for (int rt = 0; rt < 2; rt++)
#pragma unroll
    for (int dt = 0; dt < 16; dt++) O[rt][dt] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  const int nvalid = a.P + a.L;
  const int last_key = min(a.P + q0 + kBQ - 1, nvalid - 1);
  const int ntiles = last_key / kBK + 1;
  const _Float16* Kg = a.K + ((size_t)b * a.HK + kh) * a.LT * kHD;
  const _Float16* Vg = a.V + ((size_t)b * a.HK + kh) * a.LT * kHD;
  constexpr int kChunks = kBK * kHD / 8;  // 16-byte chunks per tile
  constexpr int kPer = kChunks / NT;
  const float log2e = 1.4426950408889634f;

  h8 kbuf[kPer], vbuf[kPer];
  auto fetch = [&](int kt) {
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int c = tid + i * NT, kr = c / (kHD / 8), d8 = c % (kHD / 8), key = kt * kBK + kr;
      h8 z = {};
      kbuf[i] = key < nvalid ? *reinterpret_cast<const h8*>(Kg + (size_t)key * kHD + d8 * 8) : z;
      vbuf[i] = key < nvalid ? *reinterpret_cast<const h8*>(Vg + (size_t)key * kHD + d8 * 8) : z;
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int c = tid + i * NT, kr = c / (kHD / 8), d8 = c % (kHD / 8);
      *reinterpret_cast<h8*>(Ks + kr * kKRow + d8 * 8) = kbuf[i];
#pragma unroll
      for (int e = 0; e < 8; e++) Vt[(d8 * 8 + e) * kVRow + kr] = vbuf[i][e];
    }
  };

  fetch(0);
  for (int kt = 0; kt < ntiles; kt++) {
    __syncthreads();
    stash();
    __syncthreads();
    if (kt + 1 < ntiles) fetch(kt + 1);

    // S^T[key 16kk + 4g + e][row 16rt + c16]
    f4 st[4][2];
#pragma unroll
    for (int kk = 0; kk < 4; kk++)
#pragma unroll
      for (int rt = 0; rt < 2; rt++) {
        f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
          const h8 ka = *reinterpret_cast<const h8*>(Ks + (16 * kk + c16) * kKRow + 32 * ks + 8 * g);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qreg[rt][ks], acc, 0, 0, 0);
        }
        st[kk][rt] = acc;
      }

    h8 pa[2][2];
#pragma unroll
    for (int rt = 0; rt < 2; rt++) {
      const int rowpos = a.P + q0 + 16 * rt + c16;
      float mx = -INFINITY;
#pragma unroll
      for (int kk = 0; kk < 4; kk++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int key = kt * kBK + 16 * kk + 4 * g + e;
          const float s = key <= rowpos ? st[kk][rt][e] * log2e : -INFINITY;
          st[kk][rt][e] = s;
          mx = fmaxf(mx, s);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mnew = fmaxf(m[rt], mx);
      const float alpha = exp2f(m[rt] - mnew);
      float sum = 0.0f;
#pragma unroll
      for (int kk = 0; kk < 4; kk++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float p = exp2f(st[kk][rt][e] - mnew);
          st[kk][rt][e] = p;
          sum += p;
        }
      sum += __shfl_xor(sum, 16);
      sum += __shfl_xor(sum, 32);
      l[rt] = l[rt] * alpha + sum;
      m[rt] = mnew;
      // O rows of this lane are 16 rt + 4 g + e; their alpha lives in lane 4 g + e
      float al[4];
#pragma unroll
      for (int e = 0; e < 4; e++) al[e] = __shfl(alpha, 4 * g + e);
#pragma unroll
      for (int dt = 0; dt < 16; dt++)
#pragma unroll
        for (int e = 0; e < 4; e++) O[rt][dt][e] *= al[e];
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          pa[rt][kb][e] = (_Float16)st[2 * kb][rt][e];
          pa[rt][kb][4 + e] = (_Float16)st[2 * kb + 1][rt][e];
        }
    }

#pragma unroll
    for (int dt = 0; dt < 16; dt++)
#pragma unroll
      for (int kb = 0; kb < 2; kb++) {
        const _Float16* vr = Vt + (16 * dt + c16) * kVRow + 32 * kb + 4 * g;
        const h4 lo = *reinterpret_cast<const h4*>(vr);
        const h4 hi = *reinterpret_cast<const h4*>(vr + 16);
        const h8 vb = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
        for (int rt = 0; rt < 2; rt++) O[rt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[rt][kb], vb, O[rt][dt], 0, 0, 0);
      }
  }

  // epilogue: out[t][h][d] = O / l * sigmoid(gate)
#pragma unroll
  for (int rt = 0; rt < 2; rt++) {
    float linv[4];
#pragma unroll
    for (int e = 0; e < 4; e++) linv[e] = 1.0f / __shfl(l[rt], 4 * g + e);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int t = q0 + 16 * rt + 4 * g + e;
      if (t >= a.L) continue;
      const T* grow = static_cast<const T*>(a.in) + ((size_t)b * a.L + t) * a.stride + (size_t)h * 2 * kHD + kHD;
      T* orow = static_cast<T*>(a.out) + ((size_t)b * a.L + t) * (size_t)(a.HQ * kHD) + (size_t)h * kHD;
#pragma unroll
      for (int dt = 0; dt < 16; dt++) {
        const int d = 16 * dt + c16;
        const float gt = (float)grow[d];
        orow[d] = (T)(O[rt][dt][e] * linv[e] / (1.0f + __expf(-gt)));
      }
    }
  }
}

template <int G, typename T>
hipError_t launch_attn(const GqaArgs& a, hipStream_t s) {
  auto k = gqa_attn_kernel<G, T>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)kAttnLds);
  if (e != hipSuccess) return e;
  dim3 grid((a.L + kBQ - 1) / kBQ, a.HK, a.B), block(64 * G);
  hipLaunchKernelGGL(k, grid, block, kAttnLds, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gqa(const GqaArgs& a, hipStream_t s) {
  if (a.HD != kHD || a.RD <= 0 || a.RD > 64 || (a.RD & (a.RD - 1)) || a.HQ % a.HK) return hipErrorInvalidValue;
  const int G = a.HQ / a.HK;
  const long items = (long)a.B * a.L * (a.HQ + a.HK);
  dim3 pgrid((unsigned)((items + 3) / 4)), pblock(256);
  if (a.dtype == 0)
    hipLaunchKernelGGL(gqa_prep_kernel<float>, pgrid, pblock, 0, s, a);
  else
    hipLaunchKernelGGL(gqa_prep_kernel<_Float16>, pgrid, pblock, 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  switch (G) {
    case 4: return a.dtype == 0 ? launch_attn<4, float>(a, s) : launch_attn<4, _Float16>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ha
