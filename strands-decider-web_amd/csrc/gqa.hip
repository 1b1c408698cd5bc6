// Gated causal GQA attention for the full_attention layers, gfx950.
//
// Semantics (reference web/public/engine/wgsl.js:271-302 QK_PREP and 348-417 ATTN2; third-party fp32 form:
// transformers qwen3_5 Qwen3_5RMSNorm, apply_rotary_pos_emb, eager_attention_forward, sigmoid(gate)):
//   q~ = q rsqrt(mean(q^2) + 1e-6) * qw,  k~ likewise with kw   (qw, kw are the stored 1 + w)
//   rotate-half RoPE on dims [0, RD) at absolute position P + t (engine.js:105-106 table)
//   K[P+t] = f16(k~'), V[P+t] = f16(v), q = f16(f16(q~') / sqrt(HD))
//   out = softmax_{j <= P+t}(q . K_j) V * sigmoid(gate)
//
// Cache layout in HBM (per sequence, per KV head): K row-major [LT][HD]; V transposed [HD][LT] (positions
// contiguous), so that the attention kernel stages both tiles with 16-byte copies and reads the P V operand
// without an LDS transpose.
//
// gqa_kv_kernel: one workgroup per (sequence, KV head, 64 rows): k RMSNorm + RoPE -> K rows; v through an LDS
//   transpose -> V^T columns.
// gqa_attn_kernel: one workgroup per (sequence, KV head, 64 query rows), one wave per (query head of the group,
//   32-row half), so each 64-key K/V tile is staged once in LDS and consumed by 8 waves. q's RMSNorm, RoPE (both halves
//   of a rotated pair sit in the same lane) and 1/sqrt(HD) scaling happen in registers as Q is loaded.
//   S^T = K Q^T and O += P V run on v_mfma_f32_32x32x16_f16 with fp32 accumulation; the S^T accumulators are
//   already the A operand P V needs. K/V tiles are double-buffered in LDS and arrive by global_load_lds_dwordx4
//   one tile ahead, so no registers hold the prefetch. Online softmax in fp32 with a per-row reference max that is raised only when
//   a score exceeds it by 2^8, so the 128 O accumulators are rarely rescaled; the decision is per row, which keeps
//   every row's arithmetic independent of the other rows in its block (prefix + suffix stays bit-identical).
#include <algorithm>
#include <type_traits>

#include "ha_kernels.h"

namespace ha {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

template <typename T>
using gptr = const __attribute__((address_space(1))) T*;
template <typename T>
__device__ __forceinline__ gptr<T> gp(const void* p) { return (gptr<T>)(p); }
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gpw(void* p) { return (__attribute__((address_space(1))) T*)(p); }

constexpr int kHD = 256, kBQ = 32, kBK = 64;
constexpr int kEP = 136;  // row pitch (floats) of the epilogue staging area: rows r and r + 4 sit 32 banks apart
// two K + V^T tile buffers; after the tile loop, each wave's 32 x 128 f32 epilogue staging area
constexpr int kTileBytes = kBK * kHD * 2;  // one K tile or one V^T tile (f16)
// LDS: two (K, V^T) tile buffers; after the tile loop, each wave's 32 x 128 f32 epilogue staging area
constexpr size_t kAttnLds = 4 * (size_t)kTileBytes > sizeof(float) * 8 * 32 * kEP ? 4 * (size_t)kTileBytes
                                                                                  : sizeof(float) * 8 * 32 * kEP;
constexpr float kRescale = 8.0f;    // log2 headroom before the reference max is raised

// An identity the compiler cannot see through: lane indices re-derived from it on every tile keep the address
// arithmetic built on them inside the loop instead of hoisted out of it (and spilled).
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
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

__device__ __forceinline__ f4 lds4(const float* p) { return *reinterpret_cast<const f4*>(p); }

// Orders a wave's LDS writes before its later reads of other lanes' entries (no workgroup barrier).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// max / sum of x over lanes l and l ^ 32: v_permlane32_swap hands every lane both values (in an order that depends
// on the half, which neither a max nor a two-term sum sees)
__device__ __forceinline__ void both_halves(float x, float& u, float& v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, x), false, false);
  u = __builtin_bit_cast(float, (unsigned)r[0]);
  v = __builtin_bit_cast(float, (unsigned)r[1]);
}
__device__ __forceinline__ float max_halves(float x) {
  float u, v;
  both_halves(x, u, v);
  return fmaxf(u, v);
}
__device__ __forceinline__ float sum_halves(float x) {
  float u, v;
  both_halves(x, u, v);
  return u + v;
}

__device__ __forceinline__ float sigmoid(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

template <typename T>
__device__ __forceinline__ void load8f(gptr<T> p, float* o);
template <>
__device__ __forceinline__ void load8f<float>(gptr<float> p, float* o) {
  const f4 x = *(gptr<f4>)(p), y = *(gptr<f4>)(p + 4);
  o[0] = x[0]; o[1] = x[1]; o[2] = x[2]; o[3] = x[3]; o[4] = y[0]; o[5] = y[1]; o[6] = y[2]; o[7] = y[3];
}
template <>
__device__ __forceinline__ void load8f<_Float16>(gptr<_Float16> p, float* o) {
  const h8 x = *(gptr<h8>)(p);
#pragma unroll
  for (int i = 0; i < 8; i++) o[i] = (float)x[i];
}

// Sum over the 64 lanes of a wave without LDS: row rotations inside each 16-lane row, then v_permlane16_swap
// (rows 2r <-> 2r+1) and v_permlane32_swap (halves). Every lane ends with the same bits (each step adds two values
// that the lanes it pairs see in the other order).
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum64(float v) {
  v += dpp<0x128>(v);  // row_ror:8
  v += dpp<0x124>(v);  // row_ror:4
  v += dpp<0x122>(v);  // row_ror:2
  v += dpp<0x121>(v);  // row_ror:1
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v), false, false);
  v = __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
  return sum_halves(v);
}

// K rows and V^T columns for rows [t0, t0 + 64) of one (sequence, KV head). Wave w takes rows kKvRows w ..
// kKvRows w + kKvRows - 1, lane l dims 4 l .. 4 l + 3: every row's k and v loads are issued before any is used. k:
// RMSNorm (wave-wide sum of squares), gain, rotate-half RoPE on dims [0, 64) (dim i < 32 pairs with i + 32, held by
// lane l ^ 8), f16. v: a lane holds its 4 dims of the wave's 8 rows, so it writes V^T straight from registers: per
// dim the 8 positions as one 16-byte store when all 8 rows are live and aligned, else position by position.
constexpr int kKvWaves = 8, kKvRows = 64 / kKvWaves;
template <typename T>
__global__ __launch_bounds__(64 * kKvWaves) void gqa_kv_kernel(GqaArgs a) {
  static_assert(kKvRows == 8, "a lane's 8 rows of one dim form one 16-byte V^T store");
  __shared__ f4 rope_l[64][16];  // the RoPE table rows (64 cos/sin floats) of the workgroup's 64 positions
  const int t0 = blockIdx.x * 64, kh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const size_t kvb = ((size_t)b * a.HK + kh) * a.LT * kHD;
  // the table rows go out first, so that staging them waits for them alone; the row loads below stay in flight
  // across the barrier that publishes them
  {
    const int pr = tid >> 3, c = 2 * (tid & 7);
    gptr<float> rp = gp<float>(a.rope) + (size_t)(a.P + min(t0 + pr, a.L - 1)) * a.RD + 4 * c;
    const f4 r0 = *(gptr<f4>)(rp), r1 = *(gptr<f4>)(rp + 4);
    rope_l[pr][c] = r0;
    rope_l[pr][c + 1] = r1;
  }
  const f4 kw = *(gptr<f4>)(gp<float>(a.kw) + 4 * lane);
  f4 x[kKvRows], vv[kKvRows];
#pragma unroll
  for (int r = 0; r < kKvRows; r++) {
    const int t = min(t0 + kKvRows * wave + r, a.L - 1);
    gptr<T> row = gp<T>(a.in) + ((size_t)b * a.L + t) * a.stride + (size_t)a.HQ * 2 * kHD;
    x[r] = ld4(row + (size_t)kh * kHD + 4 * lane);
    vv[r] = ld4(row + (size_t)a.HK * kHD + (size_t)kh * kHD + 4 * lane);
  }
  const bool rot = lane < 16;  // dims 0 .. 63 (RD = 64)
  const int ri = 4 * (lane & 7);
  __syncthreads();  // RoPE rows staged
#pragma unroll
  for (int r = 0; r < kKvRows; r++) {
    const int t = t0 + kKvRows * wave + r, pos = a.P + min(t, a.L - 1);
    const float ss = wave_sum64((x[r][0] * x[r][0] + x[r][1] * x[r][1]) + (x[r][2] * x[r][2] + x[r][3] * x[r][3]));
    const float inv = rsqrtf(ss / kHD + 1e-6f);
    f4 k = x[r] * inv * kw;
    f4 pk;
#pragma unroll
    for (int c = 0; c < 4; c++) pk[c] = dpp<0x128>(k[c]);  // lane l ^ 8: row_ror:8 within each 16-lane row
    if (rot) {
      const f4 cs0 = rope_l[kKvRows * wave + r][ri >> 1], cs1 = rope_l[kKvRows * wave + r][(ri >> 1) + 1];
      const float cs[4] = {cs0[0], cs0[2], cs1[0], cs1[2]}, sn[4] = {cs0[1], cs0[3], cs1[1], cs1[3]};
#pragma unroll
      for (int c = 0; c < 4; c++) k[c] = lane < 8 ? k[c] * cs[c] - pk[c] * sn[c] : k[c] * cs[c] + pk[c] * sn[c];
    }
    if (t < a.L)
      *(__attribute__((address_space(1))) h4*)(gpw<_Float16>(a.K) + kvb + (size_t)pos * kHD + 4 * lane) =
          h4{(_Float16)k[0], (_Float16)k[1], (_Float16)k[2], (_Float16)k[3]};
  }
  const int tw = t0 + kKvRows * wave;  // the wave's first row
  __attribute__((address_space(1))) _Float16* vt = gpw<_Float16>(a.V) + kvb + (size_t)(4 * lane) * a.LT + a.P + tw;
  if (tw + kKvRows <= a.L && ((a.P + tw) & 7) == 0) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
      h8 v8;
#pragma unroll
      for (int r = 0; r < kKvRows; r++) v8[r] = (_Float16)vv[r][c];
      *(__attribute__((address_space(1))) h8*)(vt + (size_t)c * a.LT) = v8;
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
      for (int r = 0; r < kKvRows; r++)
        if (tw + r < a.L) vt[(size_t)c * a.LT + r] = (_Float16)vv[r][c];
  }
}

// 64-key tiles that query block qb (rows P + 64 qb .. +63 of the call) reads under the causal mask
__device__ __forceinline__ int gqa_ntiles(const GqaArgs& a, int qb) {
  return min(a.P + qb * 64 + 63, a.P + a.L - 1) / kBK + 1;
}
inline int host_ntiles(const GqaArgs& a, int qb) { return std::min(a.P + qb * 64 + 63, a.P + a.L - 1) / kBK + 1; }

// Workgroup = 8 waves: wave w serves query head kh*4 + (w & 3) on rows q0 + 32 (w >> 2) .. +31 (a block of 64
// query rows for all 4 heads of the KV group), so each staged 64-key K/V tile feeds 8 waves, and two waves share
// every SIMD to hide each other's latency.
constexpr int kRows = 64;     // query rows per workgroup
constexpr int kWaves = 8;

// Split key ranges in one launch: a piece stores its partial results with device-coherent (sc1) stores, waits for
// them, and marks its slot with the launch's epoch (a device-scope atomic store); the merge workgroups, which come
// after every piece in the grid, wait for the marks of their block's pieces and read the partials with sc1 loads.
// Each XCD dispatches its blocks in order, so it starts merge workgroups only once all of its pieces are out:
// pieces never wait, so every mark is eventually written, and each wait is bounded besides.
constexpr int kCacheSc1 = 16;  // cache-policy operand of buffer instructions: device-coherent (sc1)
typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ unsigned* part_marks(const GqaArgs& a) {
  return reinterpret_cast<unsigned*>(a.part + (size_t)a.part_slots * 4 * kRows * (kHD + 2));
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(const float* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, 0x7fffffff, 0x00020000);
}


// Merge workgroup mi of a launch with split key ranges: query block qb (descending, as the pieces are ordered) of
// one (sequence, KV head) pair and query head hh. Once the block's pieces have marked their slots,
// out = (O / l) * sigmoid(gate) with O = sum_j 2^(m_j - M) O_j, l = sum_j 2^(m_j - M) l_j over the pieces in order,
// M = max_j m_j: the attention epilogue's arithmetic, and a piece that holds no key of a row adds exact zeros, so a
// row comes out the same whichever block and pieces it falls in. Thread t: row t / 8, dims 32 (t % 8) .. + 31.
constexpr int kMaxPieces = 16;
template <typename T>
__device__ __forceinline__ void merge_block(const GqaArgs& a, int per_pair, int mi) {
  const int npair = a.B * a.HK, nqb = (a.L + kRows - 1) / kRows;
  const int hh = mi & 3, pq = mi >> 2, pair = pq % npair, qb = nqb - 1 - pq / npair;
  const int np = (gqa_ntiles(a, qb) + a.split - 1) / a.split;
  if (np < 2) return;
  int cum = 0;
  for (int q = 0; q < qb; q++) cum += (gqa_ntiles(a, q) + a.split - 1) / a.split;
  const int slot0 = pair * per_pair + cum;
  const int tid = threadIdx.x;
  if (tid == 0) {
    // bounded; a wait that runs out is reported through the engine's error word (a test's skew makes every mark
    // this wait looks for one that no piece writes)
    const unsigned* marks = part_marks(a);
    const unsigned want = a.epoch + a.wait.skew;
    bool late = false;
    for (int j = 0; j < np; j++) {
      int i = 0;
      for (; i < a.wait.polls && __hip_atomic_load(marks + slot0 + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != want; i++)
        __builtin_amdgcn_s_sleep(2);
      late |= i == a.wait.polls;
    }
    if (late && a.wait.err) __hip_atomic_store(a.wait.err, kErrGqaMerge, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  __syncthreads();
  const int b = pair / a.HK, h = (pair % a.HK) * 4 + hh;
  const int row = tid >> 3, d0 = 32 * (tid & 7), t = qb * kRows + row;
  if (t >= a.L) return;  // a row past the call's end is not output
  const __amdgpu_buffer_rsrc_t rs = part_rsrc(a.part);
  const unsigned ml0 = (unsigned)((size_t)a.part_slots * 4 * kRows * kHD);  // first (max, sum) float
  auto rowidx = [&](int j) { return (unsigned)(((slot0 + j) * 4 + hh) * kRows + row); };
  auto ldf = [&](unsigned fidx) { return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, fidx * 4, 0, kCacheSc1)); };
  f4 g[8];
#pragma unroll
  for (int i = 0; i < 8; i++) g[i] = ld4(gp<T>(a.in) + ((size_t)b * a.L + t) * a.stride + (size_t)h * 2 * kHD + kHD + d0 + 4 * i);
  // the reference maxima of every piece in one round of loads, then the pieces four at a time
  float mj[kMaxPieces];
#pragma unroll
  for (int j = 0; j < kMaxPieces; j++)
    if (j < np) mj[j] = ldf(ml0 + rowidx(j) * 2);
  float M = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMaxPieces; j++)
    if (j < np) M = fmaxf(M, mj[j]);
  f4 o[8];
#pragma unroll
  for (int i = 0; i < 8; i++) o[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  float l = 0.0f;
#pragma unroll
  for (int j0 = 0; j0 < kMaxPieces; j0 += 4) {
    if (j0 >= np) break;
    f4 oj[4][8];
    float lj[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      if (j0 + k < np) {
        const unsigned r = rowidx(j0 + k);
        lj[k] = ldf(ml0 + r * 2 + 1);
#pragma unroll
        for (int i = 0; i < 8; i++)
          oj[k][i] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, (r * kHD + d0 + 4 * i) * 4, 0, kCacheSc1));
      }
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      if (j0 + k < np) {
        const int j = j0 + k;
        const float w = mj[j] == M ? 1.0f : __builtin_amdgcn_exp2f(mj[j] - M);
#pragma unroll
        for (int i = 0; i < 8; i++) o[i] = o[i] + w * oj[k][i];
        l = l + w * lj[k];
      }
    }
  }
  const float linv = 1.0f / l;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    f4 r;
#pragma unroll
    for (int c = 0; c < 4; c++) r[c] = (o[i][c] * linv) * sigmoid(g[i][c]);
    store4(gpw<T>(a.out) + ((size_t)b * a.L + t) * (size_t)(a.HQ * kHD) + (size_t)h * kHD + d0 + 4 * i, r);
  }
}

// Blocks [0, npair * per_pair) run query blocks (or, with split key ranges, pieces of them); the rest merge pieces.
template <typename T, bool kIdleHalf>
__global__ __launch_bounds__(64 * kWaves) void gqa_attn_kernel(GqaArgs a, int per_pair) {
  if ((int)blockIdx.x >= a.B * a.HK * per_pair) {
    merge_block<T>(a, per_pair, blockIdx.x - a.B * a.HK * per_pair);
    return;
  }
  // LDS: tile buffer i (i < 2) at i * 2 kTileBytes: K tile, then V^T tile.
  // K tile: key r at [r][32 chunks of 8 dims], chunk j stored in slot j ^ (r & 31); V^T tile: dim d at [d][8 chunks
  // of 8 positions], chunk c stored in slot c ^ ((d >> 1) & 7). A wave's global_load_lds_dwordx4 covers whole 512 B
  // K rows or 128 B V^T rows (coalesced), and the XOR swizzles make every MFMA operand read conflict-free.
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  constexpr int kTileHalves = kBK * kHD;
  _Float16* lds = reinterpret_cast<_Float16*>(lds_raw);

  // heavy-first order over all workgroups; the (sequence, KV head) pairs cycle fastest, so every workgroup of a
  // pair lands on the same XCD (round-robin dispatch over 8 XCDs) and its K/V stays in that XCD's L2
  const int npair = a.B * a.HK;
  const int nqb = (a.L + kRows - 1) / kRows;
  const int id = blockIdx.x;
  const int pair = id % npair;
  // this workgroup's query block qb and key tiles [kt0, kt1): the whole block, or with split key ranges piece
  // `piece` of the block's npieces (absolute tile boundaries, a multiple of a.split)
  int qb = nqb - 1 - id / npair, npieces = 1, piece = 0;
  if (a.split > 0) {
    qb = nqb - 1;
    int item = id / npair;
    while (qb > 0) {
      const int np = (gqa_ntiles(a, qb) + a.split - 1) / a.split;
      if (item < np) break;
      item -= np;
      qb--;
    }
    npieces = (gqa_ntiles(a, qb) + a.split - 1) / a.split;
    piece = min(item, npieces - 1);
  }
  const int kt0 = piece * (a.split > 0 ? a.split : 0);
  const int kt1 = a.split > 0 ? min(kt0 + a.split, gqa_ntiles(a, qb)) : gqa_ntiles(a, qb);
  const int b = pair / a.HK, kh = pair % a.HK;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int h = kh * 4 + (wave & 3);
  const int half = lane >> 5, c32 = lane & 31;
  const int q0 = qb * kRows + 32 * (wave >> 2);
  const int RD = a.RD;

  const size_t kvb = ((size_t)b * a.HK + kh) * a.LT * kHD;
  gptr<_Float16> Kg = gp<_Float16>(a.K) + kvb;
  gptr<_Float16> Vg = gp<_Float16>(a.V) + kvb;

  // A tile = 32 K instructions (2 keys each) + 32 V^T instructions (8 dims each), all issued by the four waves of
  // one half of the block (waves 0..3 in longer calls, waves 4..7 in calls of at most 32 rows): instructions
  // (wave & 3) + 4 i, 8 + 8 per wave. The lane's share of the addresses is re-derived from `ln` on every call (cheap
  // VALU) rather than kept live across the loop: spilled addresses would be reloaded through the same counter the
  // tile loads are waited on.
  auto issue_tile = [&](int kt, int ln) {
    _Float16* kb = lds + (size_t)(kt & 1) * 2 * kTileHalves;
    _Float16* vb = kb + kTileHalves;
    const char* kg = (const char*)(Kg + (size_t)kt * kBK * kHD);
    const char* vg = (const char*)(Vg + (size_t)kt * kBK);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int ins = (wave & 3) + 4 * i;  // 0..31
      const int r = 2 * ins + (ln >> 5), js = ln & 31;
      const int j = js ^ (r & 31);                   // global chunk that belongs in slot js
      const unsigned ko = (unsigned)(r * kHD + 8 * j) * 2u;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(kg + ko),
                                       (__attribute__((address_space(3))) void*)(kb + (size_t)ins * 512), 16, 0, 0);
      const int d = 8 * ins + (ln >> 3), cs = ln & 7;
      const int c = cs ^ ((d >> 1) & 7);
      const unsigned vo = ((unsigned)d * (unsigned)a.LT + 8u * c) * 2u;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(vg + vo),
                                       (__attribute__((address_space(3))) void*)(vb + (size_t)ins * 512), 16, 0, 0);
    }
  };
  // kIdleHalf (calls of at most 32 rows, as in a decode step, where every block's second half holds no row of the
  // call): that half's waves copy every tile and the first half's waves none, which takes the copies off the path of
  // the waves that compute
  // Longer calls: waves 0..3 (which always hold rows) copy every tile and waves 4..7 none, which staggers the two
  // waves of each SIMD a little (one starts a tile's MFMAs while the other still issues copies).
  auto issue = [&](int kt, int ln) {
    if constexpr (!kIdleHalf) {
      if (wave < 4) issue_tile(kt, ln);
    }
  };

  // Q as the B operand of S^T = K Q^T (32x32x16): qreg[ks] = q[q0 + c32][16 ks + 8 half .. +7], prepared here:
  // RMSNorm (the two halves of a row sit in lanes l and l + 32), RoPE (dim i < 32 in ks 0/1 pairs with i + 32 in
  // ks 2/3 of the same lane and element), then f16(f16(.) / sqrt(HD)). A row past the end (t >= L) repeats row
  // L - 1: rows are independent and such a row is never stored, so every load here is unconditional.
  // qw (the stored 1 + w) is staged in LDS, in the tile buffer the first tile does not use (nothing is loaded into it
  // before the loop): every lane needs 128 of the 256 weights, the same ones as every other lane of its half. Wave 0
  // (always one with rows) loads them first and writes them to LDS once its Q loads are out, so that it does not wait
  // for them before issuing those.
  // The first tile's K/V copy is issued once the lane's Q loads are out, so that those return first.
  float* qw_l = reinterpret_cast<float*>(lds_raw + (size_t)(((kt0 & 1) ^ 1) * 2) * kTileBytes);
  f4 qwv = {};
  if (tid < kHD / 4) qwv = *(gptr<f4>)(gp<float>(a.qw) + 4 * tid);
  // A wave whose 32 rows all lie past the call's end (the second half of a block with at most 32 rows) meets the
  // other waves' barriers (q's weights staged, first tile in, then one per tile), copying every tile in calls of at
  // most 32 rows (kIdleHalf: the first half's waves copy none) and nothing in longer ones (the first half's waves
  // copy every tile), then leaves: its rows are never stored (nor read from a piece's partial results), and no other
  // row depends on it. Barriers after that count only the waves still running.
  if (q0 >= a.L) {
    if constexpr (kIdleHalf) issue_tile(kt0, lane);
    __syncthreads();
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int kt = kt0; kt < kt1; kt++) {
      if constexpr (kIdleHalf) {
        if (kt + 1 < kt1) issue_tile(kt + 1, opaque(tid) & 63);
      }
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
    return;
  }
  h8 qreg[16];
  {
    const int tc = min(q0 + c32, a.L - 1);
    gptr<T> src = gp<T>(a.in) + ((size_t)b * a.L + tc) * a.stride + (size_t)h * 2 * kHD;
    // cos/sin pairs of dims i = 16 ks + 8 half + e (ks < 2): rz[ks] holds rope[pos][2 i], rope[pos][2 i + 1]
    gptr<float> rp = gp<float>(a.rope) + (size_t)(a.P + tc) * RD + 16 * half;
    f4 rz[2][4];
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
      for (int j = 0; j < 4; j++) rz[ks][j] = *(gptr<f4>)(rp + 32 * ks + 4 * j);
    // x 1/sqrt(HD) = 2^-4 on the f16 value: an exact power-of-two scale, so the f16 product (packed, two dims per
    // instruction) is the f16 rounding of the exact one
    static_assert(kHD == 256, "the q scale 1/sqrt(HD) is 2^-4");
    const h8 scale = h8{} + (_Float16)0.0625f;
    float ss = 0.0f;
    // n(ks, e) = q * inv * w for dim 16 ks + 8 half + e, from the raw value x
    auto finish = [&](int ks, const float* x, float inv) {
      const f4 w0 = lds4(qw_l + 16 * ks + 8 * half), w1 = lds4(qw_l + 16 * ks + 8 * half + 4);
      h8 n;
#pragma unroll
      for (int e = 0; e < 8; e++) n[e] = (_Float16)(x[e] * inv * (e < 4 ? w0[e] : w1[e - 4]));
      qreg[ks] = n * scale;
    };
    auto rotate = [&](int ks, const float* x1, const float* x2, float inv) {
      const f4 w10 = lds4(qw_l + 16 * ks + 8 * half), w11 = lds4(qw_l + 16 * ks + 8 * half + 4);
      const f4 w20 = lds4(qw_l + 16 * ks + 8 * half + 32), w21 = lds4(qw_l + 16 * ks + 8 * half + 36);
      h8 r1, r2;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float n1 = x1[e] * inv * (e < 4 ? w10[e] : w11[e - 4]), n2 = x2[e] * inv * (e < 4 ? w20[e] : w21[e - 4]);
        const f4 c = rz[ks][e >> 1];
        const float cs = c[2 * (e & 1)], sn = c[2 * (e & 1) + 1];
        r1[e] = (_Float16)(n1 * cs - n2 * sn);
        r2[e] = (_Float16)(n2 * cs + n1 * sn);
      }
      qreg[ks] = r1 * scale;
      qreg[ks + 2] = r2 * scale;
    };
    if constexpr (sizeof(T) == 2) {
      // f16 rows: the whole row slice (16 x 16 B) is loaded at once and converted in place
      h8 raw[16];
#pragma unroll
      for (int ks = 0; ks < 16; ks++) raw[ks] = *(gptr<h8>)(src + 16 * ks + 8 * half);
      // before the tile's DMA, after which the compiler would wait for every load (the DMA included) to write it
      if (tid < kHD / 4) *reinterpret_cast<f4*>(qw_l + 4 * tid) = qwv;
      issue(kt0, lane);
#pragma unroll
      for (int ks = 0; ks < 16; ks++)
#pragma unroll
        for (int e = 0; e < 8; e++) ss += (float)raw[ks][e] * (float)raw[ks][e];
      const float inv = rsqrtf(sum_halves(ss) / kHD + 1e-6f);
      __syncthreads();  // qw staged
      // dims 0..63 (slots ks 0..3): normalise, rotate pairs (ks, ks + 2), scale
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        float x1[8], x2[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
          x1[e] = (float)raw[ks][e];
          x2[e] = (float)raw[ks + 2][e];
        }
        rotate(ks, x1, x2, inv);
      }
#pragma unroll
      for (int ks = 4; ks < 16; ks++) {
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; e++) x[e] = (float)raw[ks][e];
        finish(ks, x, inv);
      }
    } else {
      // f32 rows: two passes over the row slice, eight 32-byte loads in flight at a time
#pragma unroll
      for (int bt = 0; bt < 2; bt++) {
        float qv[8][8];
#pragma unroll
        for (int k = 0; k < 8; k++) load8f<T>(src + 16 * (8 * bt + k) + 8 * half, qv[k]);
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
          for (int e = 0; e < 8; e++) ss += qv[k][e] * qv[k][e];
        asm volatile("" : "+v"(ss)::"memory");
        if (bt == 0) {
          if (tid < kHD / 4) *reinterpret_cast<f4*>(qw_l + 4 * tid) = qwv;  // before the tile's DMA (see f16 rows)
          issue(kt0, lane);
        }
      }
      const float inv = rsqrtf(sum_halves(ss) / kHD + 1e-6f);
      __syncthreads();  // qw staged
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        float x1[8], x2[8];
        load8f<T>(src + 16 * ks + 8 * half, x1);
        load8f<T>(src + 16 * (ks + 2) + 8 * half, x2);
        rotate(ks, x1, x2, inv);
      }
#pragma unroll
      for (int bt = 0; bt < 3; bt++) {
        float qv[4][8];
#pragma unroll
        for (int k = 0; k < 4; k++) load8f<T>(src + 16 * (4 + 4 * bt + k) + 8 * half, qv[k]);
#pragma unroll
        for (int k = 0; k < 4; k++) finish(4 + 4 * bt + k, qv[k], inv);
        asm volatile("" : "+v"(qreg[4 + 4 * bt]), "+v"(qreg[5 + 4 * bt]), "+v"(qreg[6 + 4 * bt]), "+v"(qreg[7 + 4 * bt])::"memory");
      }
    }
  }

  // row state: this lane's S^T columns are query row c32 (both halves hold it after the xor-32 reductions)
  float mref = -INFINITY, lsum = 0.0f;
  const int rowpos = a.P + q0 + c32;
  const float log2e = 1.4426950408889634f;

  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // O is zeroed from a value produced here, so its 128 registers are not claimed during the prologue's loads
  f16v O[8];  // O[dt][v] = out row 8 (v/4) + 4 half + v%4, dim 32 dt + c32
  {
    float z = 0.0f;
    asm volatile("" : "+v"(z));
#pragma unroll
    for (int dt = 0; dt < 8; dt++) O[dt] = f16v{} + z;
  }
  // the lowest query position of this wave: tiles whose keys all lie at or below it need no causal mask
  const int minpos = a.P + q0;

  // S^T row i of a 32-key half holds key pi(i) (bits 2 and 3 of i swapped): then the eight S^T values a lane holds
  // for one 16-key step of P V are eight consecutive keys, and that step's V^T operand is one 16-byte read.
  // K operand of k-step ks for key row r = pi(c32): chunk j = 2 ks + half sits in slot j ^ r, i.e. at byte
  // (16 (r ^ half)) ^ (32 ks) of the row. V^T operand of dim d = 32 dt + c32, keys 8 c .. 8 c + 7: slot
  // c ^ ((d >> 1) & 7) of the row.
  auto kbase_of = [&](int kt, int kk, int ln) {
    const int lc = ln & 31, lh = ln >> 5;
    const int pr = (lc & 19) | ((lc & 4) << 1) | ((lc & 8) >> 1);
    return (unsigned)((kt & 1) * 2 * kTileBytes + kk * 32 * kHD * 2) + (unsigned)pr * (kHD * 2) + 16u * (unsigned)(pr ^ lh);
  };
  auto vbase_of = [&](int kt, int ln) {
    const int lc = ln & 31;
    return (unsigned)(((kt & 1) * 2 + 1) * kTileBytes) + (unsigned)lc * (kBK * 2) + 16u * (unsigned)((lc >> 1) & 7);
  };
  // S^T = K Q^T for the 32-key half at kb (byte address of this lane's row in the K tile)
  auto qk = [&](unsigned kb) {
    f16v st = f16v{};
#pragma unroll
    for (int ks = 0; ks < 16; ks++) {
      const h8 ka = *reinterpret_cast<const h8*>(lds_raw + (kb ^ (32u * ks)));
      st = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qreg[ks], st, 0, 0, 0);
    }
    return st;
  };
  // online softmax of one 32-key half (keys kt * 64 + 32 kk + 16 (v/8) + 8 half + v%8 in st[v]) -> f16 P in pa
  auto softmax = [&](f16v& st, int kt, int kk, h8* pa) {
    if (kt * kBK + kBK - 1 > minpos) {
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int key = kt * kBK + 32 * kk + 16 * (v >> 3) + 8 * half + (v & 7);
        st[v] = key <= rowpos ? st[v] : -INFINITY;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; v++) mx = fmaxf(mx, st[v]);
    mx = max_halves(mx) * log2e;
    // raise the reference max only when a score would exceed it by 2^kRescale (decided per row)
    const float mnew = mx > mref + kRescale ? mx : mref;
    // 1 when unchanged (also while a row has seen no key: a piece of a split key range can start with tiles that
    // lie wholly after some of its rows), 0 on a row's first keys
    const float alpha = mnew == mref ? 1.0f : __builtin_amdgcn_exp2f(mref - mnew);
    const bool need = mnew != mref && mref != -INFINITY;
    mref = mnew;
    const float msub = mnew == -INFINITY ? 0.0f : mnew;  // masked scores give exp2(-inf) = 0, never NaN
    float sum = 0.0f;
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const float pv = __builtin_amdgcn_exp2f(fmaf(st[v], log2e, -msub));
      st[v] = pv;
      sum += pv;
    }
    lsum = lsum * alpha + sum_halves(sum);
    if (__any(need)) {
      // O rows 8 (v/4) + 4 half + v%4 take alpha from lane (row) in the low half
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const float al = __shfl(alpha, 8 * (v >> 2) + 4 * (opaque(lane) >> 5) + (v & 3));
#pragma unroll
        for (int dt = 0; dt < 8; dt++) O[dt][v] *= al;
      }
    }
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int e = 0; e < 8; e++) pa[kb][e] = (_Float16)st[8 * kb + e];
  };
  // O += P V for the 32-key half kk: k-step kb covers keys 32 kk + 16 kb + 8 half + e (vb = this lane's V^T row)
  auto pv = [&](const h8* pa, int kk, unsigned vb, int ln) {
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
      const unsigned vo = vb ^ (unsigned)(16 * (4 * kk + 2 * kb + (ln >> 5)));
#pragma unroll
      for (int dt = 0; dt < 8; dt++) {
        const h8 vv = *reinterpret_cast<const h8*>(lds_raw + vo + (unsigned)(dt * 32 * kBK * 2));
        O[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa[kb], vv, O[dt], 0, 0, 0);
      }
    }
  };

  for (int kt = kt0; kt < kt1; kt++) {
    const int ln = opaque(tid) & 63;
    if (kt + 1 < kt1) issue(kt + 1, ln);
    h8 pa[2];
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
      f16v st = qk(kbase_of(kt, kk, ln));
      softmax(st, kt, kk, pa);
      pv(pa, kk, vbase_of(kt, ln), ln);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's part of the next tile has landed
    __syncthreads();                // ... and every wave's; nobody reads the current buffer any more
  }

  float* ep = reinterpret_cast<float*>(lds_raw) + (size_t)wave * 32 * kEP;
  const int er = lane >> 5, ec = 4 * (lane & 31);
  if (npieces > 1) {
    // one piece of a split key range: unnormalised O and the row's (reference max, sum) to the partial slot
    // (slot = pair's first slot + pieces of the blocks below qb + piece), sc1 stores, then the slot's mark
    const int slot = pair * per_pair + (per_pair - (id / npair - piece) - npieces) + piece;
    const size_t rbase = ((size_t)slot * 4 + (wave & 3)) * kRows + 32 * (wave >> 2);
    const __amdgpu_buffer_rsrc_t po = part_rsrc(a.part + rbase * kHD);
    const __amdgpu_buffer_rsrc_t pml = part_rsrc(a.part + (size_t)a.part_slots * 4 * kRows * kHD + rbase * 2);
    if (half == 0) {
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, mref), pml, 8 * c32, 0, kCacheSc1);
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, lsum), pml, 8 * c32 + 4, 0, kCacheSc1);
    }
#pragma unroll
    for (int p = 0; p < 2; p++) {
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int v = 0; v < 16; v++) ep[(8 * (v >> 2) + 4 * half + (v & 3)) * kEP + 32 * j + c32] = O[4 * p + j][v];
      wave_sync();
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const f4 o = lds4(ep + (2 * i + er) * kEP + ec);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i4v, o), po, ((2 * i + er) * kHD + 128 * p + ec) * 4, 0,
                                               kCacheSc1);
      }
      wave_sync();
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's partials have reached the device-coherent level
    __syncthreads();                // ... and every wave's
    if (tid == 0) __hip_atomic_store(part_marks(a) + slot, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  // epilogue: out[t][h][d] = O / l * sigmoid(gate), through LDS (free after the loop's last barrier). Each wave
  // stages 32 rows x 128 dims of O / l at a time; then a lane handles 4 consecutive dims of a row (rows 2 i + er),
  // so gate loads and output stores are 8- or 16-byte accesses, all issued before they are needed.
  // The gate loads of f16 rows (both passes, 64 VGPRs once Q is dead) are all issued first; f32 rows load each pass's
  // at its start.
  // The sequence's input and output rows are buffer ranges: a row at or past the call's end lies past the range, so
  // its gate loads read zeros and its stores are dropped by the hardware (the range check covers the per-lane
  // offset, which carries the row). No row index is clamped or tested, and each row costs one offset add.
  typedef typename std::conditional<sizeof(T) == 2, h4, f4>::type G4;
  const __amdgpu_buffer_rsrc_t gin = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(reinterpret_cast<const char*>(a.in)) + (size_t)b * a.L * a.stride * sizeof(T), 0,
      (int)((size_t)a.L * a.stride * sizeof(T)), 0x00020000);
  const __amdgpu_buffer_rsrc_t gout = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<char*>(a.out) + (size_t)b * a.L * a.HQ * kHD * sizeof(T), 0,
      (int)((size_t)a.L * a.HQ * kHD * sizeof(T)), 0x00020000);
  const unsigned gv0 = ((unsigned)(q0 + er) * (unsigned)a.stride + (unsigned)(h * 2 * kHD + kHD + ec)) * sizeof(T);
  const unsigned ov0 = ((unsigned)(q0 + er) * (unsigned)(a.HQ * kHD) + (unsigned)(h * kHD + ec)) * sizeof(T);
  const unsigned gstep = 2u * (unsigned)a.stride * sizeof(T), ostep = 2u * (unsigned)(a.HQ * kHD) * sizeof(T);
  G4 graw[2][16];
  auto load_gates = [&](int p) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const unsigned off = gv0 + (unsigned)i * gstep + 128u * p * sizeof(T);
      if constexpr (sizeof(T) == 2)
        graw[p][i] = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(gin, off, 0, 0));
      else
        graw[p][i] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(gin, off, 0, 0));
    }
  };
  load_gates(0);
  if constexpr (sizeof(T) == 2) load_gates(1);
  // 1 / l: one division per lane for its own row (lane c32 holds row c32's sum), handed to the lanes that need it
  const float rinv = 1.0f / lsum;
  float linv[16];
#pragma unroll
  for (int v = 0; v < 16; v++) linv[v] = __shfl(rinv, 8 * (v >> 2) + 4 * half + (v & 3));
#pragma unroll
  for (int p = 0; p < 2; p++) {
    if constexpr (sizeof(T) == 4) {
      if (p == 1) load_gates(1);
    }
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) ep[(8 * (v >> 2) + 4 * half + (v & 3)) * kEP + 32 * j + c32] = O[4 * p + j][v] * linv[v];
    wave_sync();
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const f4 o = lds4(ep + (2 * i + er) * kEP + ec);
      f4 r;
#pragma unroll
      for (int c = 0; c < 4; c++) r[c] = o[c] * sigmoid((float)graw[p][i][c]);
      const unsigned off = ov0 + (unsigned)i * ostep + 128u * p * sizeof(T);
      if constexpr (sizeof(T) == 2)
        __builtin_amdgcn_raw_buffer_store_b64(
            __builtin_bit_cast(i2v, h4{(_Float16)r[0], (_Float16)r[1], (_Float16)r[2], (_Float16)r[3]}), gout, off, 0, 0);
      else
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i4v, r), gout, off, 0, 0);
    }
    wave_sync();
  }
}

template <typename T>
hipError_t launch_attn(const GqaArgs& a, hipStream_t s) {
  auto k = a.L <= 32 ? gqa_attn_kernel<T, true> : gqa_attn_kernel<T, false>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)kAttnLds);
  if (e != hipSuccess) return e;
  const int npair = a.B * a.HK, nqb = (a.L + kRows - 1) / kRows;
  int per_pair = nqb;
  bool any_split = false;
  if (a.split > 0) {
    per_pair = 0;
    for (int q = 0; q < nqb; q++) {
      const int np = (host_ntiles(a, q) + a.split - 1) / a.split;
      per_pair += np;
      any_split |= np > 1;
    }
    if (any_split && ((size_t)npair * per_pair > (size_t)a.part_slots || !a.part)) return hipErrorInvalidValue;
    if ((a.LT / kBK + a.split - 1) / a.split > kMaxPieces) return hipErrorInvalidValue;
  }
  if (any_split && a.epoch == 0) return hipErrorInvalidValue;
  const int nmerge = any_split ? npair * nqb * 4 : 0;
  hipLaunchKernelGGL(k, dim3(npair * per_pair + nmerge), dim3(64 * kWaves), kAttnLds, s, a, per_pair);
  return hipGetLastError();
}

}  // namespace

size_t gqa_part_slot_bytes() { return (size_t)4 * kRows * (kHD + 2) * sizeof(float) + sizeof(unsigned); }

// Per pair, a call with P + L <= max_ctx has at most sum_{k=2}^{N+1} ceil(k / split) pieces (N = max_ctx / 64):
// block qb reads at most P/64 + qb + 2 tiles and there are at most N - P/64 blocks.
size_t gqa_part_slots(int pairs, int max_ctx, int split) {
  if (split <= 0) return 0;
  const int N = (max_ctx + kBK - 1) / kBK;
  size_t per = 0;
  for (int k = 2; k <= N + 1; k++) per += (size_t)((k + split - 1) / split);
  return per * (size_t)pairs;
}

hipError_t launch_gqa(const GqaArgs& a, hipStream_t s) {
  // RD = 64 puts both halves of every rotated q pair in one lane of the fused q preparation
  if (a.HD != kHD || a.RD != 64 || a.HQ % a.HK || a.HQ / a.HK != 4) return hipErrorInvalidValue;
  if (a.LT % kBK) return hipErrorInvalidValue;  // V^T tiles are read 64 positions at a time, inside [0, LT)
  // the attention epilogue addresses a sequence's input and output rows by 32-bit byte offsets, rows past the call's
  // end (up to 64 on) included: they must not wrap
  const size_t esz = a.dtype == 0 ? 4 : 2, rows = (size_t)a.L + 64;
  if (rows * a.stride * esz > 0xFFFFFFFFull || rows * a.HQ * kHD * esz > 0xFFFFFFFFull) return hipErrorInvalidValue;
  dim3 kgrid((a.L + 63) / 64, a.HK, a.B), kblock(64 * kKvWaves);
  if (a.dtype == 0)
    hipLaunchKernelGGL(gqa_kv_kernel<float>, kgrid, kblock, 0, s, a);
  else
    hipLaunchKernelGGL(gqa_kv_kernel<_Float16>, kgrid, kblock, 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return a.dtype == 0 ? launch_attn<float>(a, s) : launch_attn<_Float16>(a, s);
}

}  // namespace ha
