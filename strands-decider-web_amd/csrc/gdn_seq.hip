// Sequential gated-delta rule for decode / resume (ha_recurrence HA_SEQUENTIAL), gfx950.
//
// Semantics: the engine's CONV + GDN + GNORM steps (reference web/public/engine/wgsl.js:124-139, 146-187, 252-268)
// with the third-party fp32 rule they restate (transformers qwen3_5 torch_recurrent_gated_delta_rule):
//   u = silu(conv4(x)); q^ = q rsqrt(|q|^2 + 1e-6) / sqrt(DK); k^ = k rsqrt(|k|^2 + 1e-6)
//   beta = sigmoid(b); alpha = exp(negA * softplus(a + dt_bias))
//   S <- alpha S; delta = beta (v - S^T k^); S <- S + k^ delta^T; o = S^T q^
//   y = gnorm * o * rsqrt(mean(o^2) + 1e-6) * silu(z)
//
// Layout: kGroups workgroups of 4 waves per (sequence, head), each owning 32 of the 128 value columns, so the 64 KiB
// of fp32 state per head is read and written by 4 CUs. Lane l of wave w owns value column 32 g + 8 w + (l & 7) and
// key rows 16 (l >> 3) .. + 15: its 16 state entries stay in VGPRs for the whole call. The sums over key rows run
// over the 8 lanes of one column, l & 7 fixed: DPP row_ror:8 (lanes l ^ 8 inside a 16-lane row), v_permlane16_swap
// (l ^ 16) and v_permlane32_swap (l ^ 32), no LDS and no barrier. Each wave computes the conv, the norms (the same
// DPP and permlane sums over all 64 lanes) and q^/k^ redundantly and hands them to its own lanes through a
// wave-private LDS slot, so the token loop has no workgroup barrier either.
//
// The gated norm needs all 128 columns of a row, which live in kGroups workgroups: each workgroup stores its raw
// outputs (fp32, device-scope stores) in a per-engine scratch, waits for its own stores, and bumps a per-head
// counter; the workgroup that arrives last reads the whole rows back (device-scope loads) and writes the normalised
// outputs. Nothing waits for another workgroup. One launch covers at most kSegRows output rows (the scratch holds
// that many per head); a longer call is several launches, the state carried between them in S_out.
#include "ha_kernels.h"

namespace ha {
namespace {

constexpr int kDK = 128, kDV = 128, kKC = 4;
constexpr int kGroups = 4;  // workgroups per (sequence, head)
constexpr int kCols = kDV / kGroups;

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}
__device__ __forceinline__ float swap16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v), false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}
__device__ __forceinline__ float swap32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v), false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}
// sum over the 8 lanes l ^ 8k (one value column); every lane gets the same bits (each step adds two values the
// paired lanes see in the other order)
__device__ __forceinline__ float col_sum8(float v) { return swap32_sum(swap16_sum(v + dpp<0x128>(v))); }
// sum over all 64 lanes
__device__ __forceinline__ float wave_sum64(float v) {
  v += dpp<0x128>(v);  // row_ror:8
  v += dpp<0x124>(v);  // row_ror:4
  v += dpp<0x122>(v);  // row_ror:2
  v += dpp<0x121>(v);  // row_ror:1
  return swap32_sum(swap16_sum(v));
}

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

// device-scope (sc1) 4-byte store and 16-byte load through a buffer resource: visible to and read from the level
// every workgroup of the device sees
__device__ __forceinline__ void st_dev(float* base, int off_bytes, float v) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v), r, off_bytes, 0, 16);
}
__device__ __forceinline__ f4 ld_dev4(const float* base, int off_bytes) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, 0x7fffffff, 0x00020000);
  return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off_bytes, 0, 16));
}

// rows [r0, r1) of the call (absolute positions; outputs for rows >= P), one launch
template <typename T>
__global__ __launch_bounds__(256) void gdn_seq_kernel(GdnArgs a, int r0, int r1) {
  const int bh = blockIdx.x / kGroups, g = blockIdx.x % kGroups;
  const int b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int jl = 8 * wave + (lane & 7);  // value column inside this workgroup's 32
  const int j = kCols * g + jl;
  const int rg = lane >> 3;              // key rows 16 rg .. + 15

  __shared__ float qk[4][2][kDK];  // wave-private q^ (0) and k^ (1)

  const size_t sbase = ((size_t)b * a.H + h) * kDK * kDV;
  const float* Sin = r0 == a.s0 ? a.S_in : a.S_out;  // later launches continue from the state the last one wrote
  float S[16];
  if (Sin) {
#pragma unroll
    for (int i = 0; i < 16; i++) S[i] = Sin[sbase + (size_t)(16 * rg + i) * kDV + j];
  } else {
#pragma unroll
    for (int i = 0; i < 16; i++) S[i] = 0.0f;
  }

  // channels of this lane: q dims lane, lane + 64; k dims lane, lane + 64; v column j
  const int cq0 = h * kDK + lane, cq1 = cq0 + 64;
  const int ck0 = a.H * kDK + h * kDK + lane, ck1 = ck0 + 64;
  const int cv = 2 * a.H * kDK + h * kDV + j;
  const int cidx[5] = {cq0, cq1, ck0, ck1, cv};
  float w[5][kKC], hx[5][kKC - 1];
#pragma unroll
  for (int c = 0; c < 5; c++)
#pragma unroll
    for (int t = 0; t < kKC; t++) w[c][t] = a.conv_w[(size_t)cidx[c] * kKC + t];
  // conv history: raw rows r0-3 .. r0-1
#pragma unroll
  for (int t = 0; t < kKC - 1; t++) {
    const T* row = row_of<T>(a, b, r0 - (kKC - 1) + t);
#pragma unroll
    for (int c = 0; c < 5; c++) hx[c][t] = (float)row[cidx[c]];
  }
  const float na = a.negA[h], db = a.dtb[h];
  const int aoff = a.C + a.H * a.DV + h, boff = aoff + a.H;
  const float qscale = 0.08838834764831845f;  // 1/sqrt(128)
  const int orow0 = max(r0, a.P);             // first output row of this launch
  // raw outputs: scratch [B][H][kSegRows][128] fp32 (gated norm) or the output rows directly (raw core output)
  float* const raw = a.seq_raw + (size_t)bh * kSegRows * kDV;

  // this lane's inputs of a row: the 5 channels and the a / b gates. Two register sets alternate (rows r and r + 1),
  // each refilled with the row two ahead as soon as its row is consumed, so a load has a whole token to land and no
  // register holding a load in flight is ever copied (a copy would wait for the load).
  float x0[5], a0, b0, x1[5], a1, b1;
  auto load_row = [&](int r, float* x, float& av, float& bv) {
    const T* row = row_of<T>(a, b, min(r, r1 - 1));
#pragma unroll
    for (int c = 0; c < 5; c++) x[c] = (float)row[cidx[c]];
    av = (float)row[aoff];
    bv = (float)row[boff];
  };
  // one token: row r with inputs x, av, bv (then refilled with row r + 2)
  auto step = [&](int r, float* x, float& av, float& bv) {
    float u[5];
#pragma unroll
    for (int c = 0; c < 5; c++) {
      float s = w[c][0] * hx[c][0];
      s = fmaf(w[c][1], hx[c][1], s);
      s = fmaf(w[c][2], hx[c][2], s);
      s = fmaf(w[c][3], x[c], s);
      hx[c][0] = hx[c][1];
      hx[c][1] = hx[c][2];
      hx[c][2] = x[c];
      u[c] = silu(s);
    }
    const float beta = __builtin_amdgcn_rcpf(1.0f + __expf(-bv));
    const float xs = av + db;
    const float sp = xs > 20.0f ? xs : log1pf(__expf(xs));
    const float alpha = __expf(na * sp);
    load_row(r + 2, x, av, bv);
    const float ssq = wave_sum64(u[0] * u[0] + u[1] * u[1]);
    const float ssk = wave_sum64(u[2] * u[2] + u[3] * u[3]);
    const float rq = rsqrtf(ssq + 1e-6f) * qscale, rk = rsqrtf(ssk + 1e-6f);
    qk[wave][0][lane] = u[0] * rq;
    qk[wave][0][lane + 64] = u[1] * rq;
    qk[wave][1][lane] = u[2] * rk;
    qk[wave][1][lane + 64] = u[3] * rk;
    wave_sync();
    const f4* kv4 = reinterpret_cast<const f4*>(&qk[wave][1][16 * rg]);
    const f4* qv4 = reinterpret_cast<const f4*>(&qk[wave][0][16 * rg]);
    f4 kk[4], qq[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      kk[i] = kv4[i];
      qq[i] = qv4[i];
    }
    float kr = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      S[i] *= alpha;
      kr = fmaf(S[i], kk[i >> 2][i & 3], kr);
    }
    kr = col_sum8(kr);
    const float delta = beta * (u[4] - kr);
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      S[i] = fmaf(kk[i >> 2][i & 3], delta, S[i]);
      o = fmaf(S[i], qq[i >> 2][i & 3], o);
    }
    o = col_sum8(o);
    wave_sync();
    if (r >= a.P && rg == 0) {
      if (a.gnorm) st_dev(raw, ((r - orow0) * kDV + j) * 4, o);
      else static_cast<T*>(a.out)[((size_t)b * a.L + (r - a.P)) * (size_t)(a.H * kDV) + (size_t)h * kDV + j] = (T)o;
    }
  };
  load_row(r0, x0, a0, b0);
  load_row(r0 + 1, x1, a1, b1);
  for (int r = r0; r < r1; r += 2) {
    step(r, x0, a0, b0);
    if (r + 1 < r1) step(r + 1, x1, a1, b1);
  }
#pragma unroll
  for (int i = 0; i < 16; i++) a.S_out[sbase + (size_t)(16 * rg + i) * kDV + j] = S[i];

  const int nrows = r1 - orow0;
  if (!a.gnorm || nrows <= 0) return;
  // every raw output of this workgroup has reached the device-wide level before the counter moves
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  __shared__ unsigned last;
  if (tid == 0) {
    const unsigned old = __hip_atomic_fetch_add(a.seq_cnt + bh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == kGroups - 1;
    if (last) __hip_atomic_store(a.seq_cnt + bh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next launch
  }
  __syncthreads();
  if (!last) return;
  // the gated norm of this head's rows: 4 threads per row, 32 columns each (8 loads of 4 columns)
  for (int t = tid >> 2; t < nrows; t += 64) {
    const int c0 = 32 * (tid & 3);
    f4 v[8];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      v[k] = ld_dev4(raw, (t * kDV + c0 + 4 * k) * 4);
      ss += v[k][0] * v[k][0] + v[k][1] * v[k][1] + v[k][2] * v[k][2] + v[k][3] * v[k][3];
    }
    ss += dpp<0xB1>(ss);  // quad_perm [1,0,3,2]
    ss += dpp<0x4E>(ss);  // quad_perm [2,3,0,1]
    const float inv = rsqrtf(ss / kDV + 1e-6f);
    const int rr = orow0 + t - a.P;
    const T* zrow = static_cast<const T*>(a.in) + ((size_t)b * a.L + rr) * a.stride + a.C + h * kDV + c0;
    T* op = static_cast<T*>(a.out) + ((size_t)b * a.L + rr) * (size_t)(a.H * kDV) + (size_t)h * kDV + c0;
    float z[32], gw[32];
#pragma unroll
    for (int c = 0; c < 32; c++) {
      z[c] = (float)zrow[c];
      gw[c] = a.gnorm[c0 + c];
    }
#pragma unroll
    for (int k = 0; k < 8; k++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int c = 4 * k + e;
        op[c] = (T)(gw[c] * v[k][e] * inv * silu(z[c]));
      }
  }
}

}  // namespace

hipError_t launch_gdn_sequential(const GdnArgs& a, hipStream_t s) {
  if (a.DK != kDK || a.DV != kDV || a.KC != kKC) return hipErrorInvalidValue;
  if (a.gnorm && (!a.seq_raw || !a.seq_cnt)) return hipErrorInvalidValue;
  const dim3 grid(a.B * a.H * kGroups), block(256);
  const int end = a.P + a.L;
  // launches of at most kSegRows output rows; the first also replays rows [s0, P)
  for (int r0 = a.s0; r0 < end;) {
    const int r1 = min(end, max(r0, a.P) + kSegRows);
    if (a.dtype == 0)
      hipLaunchKernelGGL(gdn_seq_kernel<float>, grid, block, 0, s, a, r0, r1);
    else
      hipLaunchKernelGGL(gdn_seq_kernel<_Float16>, grid, block, 0, s, a, r0, r1);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    r0 = r1;
  }
  return hipSuccess;
}

}  // namespace ha
