// Helpers shared by the chunked gated-delta kernels (gdn_chunk.hip: one fused kernel; gdn_split.hip: the
// chunk-parallel preparation, state and output kernels). Chunk geometry, the swizzled LDS tile layouts,
// the DPP reductions, global-pointer loads/stores and the MFMA operand conventions are described where they are
// defined. Everything is in an anonymous namespace: each translation unit gets its own copy.
#pragma once
#include "ha_kernels.h"

namespace ha {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kDK = 128, kDV = 128, kCH = 64, kKC = 4;
constexpr int kQP = kDK + 8;  // row pitch (halves) of [64][128] f16 tiles
constexpr int kTP = kCH + 8;  // row pitch (halves) of [*][64] f16 tiles
constexpr int kAP = kCH + 4;  // row pitch (floats) of the fp32 A / T tile

// Transposed tiles are written 8 rows of one column (16 bytes) per lane; the 8-column group index is XORed with a
// function of the row so those writes spread over the banks. Element (row, col) lives at
// row * kTP + 8 * (col / 8 ^ f(row)) + col % 8; every 16-byte read stays contiguous.
__device__ __forceinline__ int kt16(int i, int g8) { return i * kTP + 8 * (g8 ^ ((i >> 3) & 7)); }
__device__ __forceinline__ int vt16(int j, int g8) { return j * kTP + 8 * (g8 ^ ((j >> 4) & 7)); }

// SiLU / sigmoid with the hardware reciprocal (v_rcp_f32, 1 ulp) instead of an IEEE division sequence
__device__ __forceinline__ float silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

#define DPP_F(v, ctrl) __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, (v)), (ctrl), 0xf, 0xf, false))

// Sum over the 16 lanes of a DPP row (lanes 16r..16r+15) with row rotations; every lane gets the sum.
__device__ __forceinline__ float row_sum16(float v) {
  v += DPP_F(v, 0x128);
  v += DPP_F(v, 0x124);
  v += DPP_F(v, 0x122);
  v += DPP_F(v, 0x121);
  return v;
}

// Sum over aligned groups of 8 lanes: quad permutations, then the half-row mirror (lane i <-> 7 - i).
__device__ __forceinline__ float sum8(float v) {
  v += DPP_F(v, 0xB1);
  v += DPP_F(v, 0x4E);
  v += DPP_F(v, 0x141);
  return v;
}

// Orders a wave's LDS writes before its later reads of other lanes' entries (no workgroup barrier).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// An identity the compiler cannot see through: per-lane indices re-derived from it every period keep the address
// arithmetic built on them inside the loop instead of being hoisted out of it and spilled.
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

// The two sources of input rows as opaque values: a per-lane choice between them stays a select of two registers.
// (Choosing between the argument block's own fields instead turns into a load through a selected address, which
// moves the argument block to scratch memory.)
struct RowSrc {
  const char* in;
  const char* tail;
};
__device__ __forceinline__ RowSrc row_src(const GdnArgs& a) {
  const char* in = (const char*)a.in;
  const char* tail = (const char*)a.tail;
  asm volatile("" : "+s"(in), "+s"(tail));
  return RowSrc{in, tail};
}

// Row r of sequence b: rows before P come from the tail buffer (its first row is s0 - 3), later ones from the input.
template <typename T>
__device__ __forceinline__ gptr<T> row_of(const GdnArgs& a, const RowSrc& src, int b, int r) {
  const bool tl = r < a.P;
  const char* base = tl ? src.tail : src.in;
  const size_t row = tl ? (size_t)b * a.tail_cap + (r - (a.s0 - (kKC - 1))) : (size_t)b * a.L + (r - a.P);
  return gp<T>(base) + row * a.stride;
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

// perm_a for the swizzled k^T tile
__device__ __forceinline__ h8 perm_a_kt(const _Float16* kt, int r, int kb, int grp) {
  const int sub = 4 * (grp & 1);
  const h4 lo = *reinterpret_cast<const h4*>(kt + kt16(r, 4 * kb + (grp >> 1)) + sub);
  const h4 hi = *reinterpret_cast<const h4*>(kt + kt16(r, 4 * kb + 2 + (grp >> 1)) + sub);
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

// A bounded wait that ran out: its bit into the engine's host-visible error word (one system-scope vector store;
// several such stores may race, and any non-zero value reports the failure).
__device__ __forceinline__ void report_wait(const WaitCheck& w, unsigned bit) {
  if (w.err) __hip_atomic_store(w.err, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

template <int N>
struct Width {
  static constexpr int value = N;
};

// Block column J of T below the diagonal: T_iJ = -T_ii sum_{k=J}^{i-1} A_ik T_kJ for block rows i = J+1..3, in
// order. The column's blocks stay in registers (D layout: rows 4 grp + e, column c16), so A is never overwritten
// and the three column waves need no barrier between block rows; only the f16 copies T diag(beta) and (with
// kWithTw) T diag(beta e^gc) are stored. The D layout is used directly as the B operand of v_mfma_f32_16x16x4f32 by giving
// step e the K index 4 grp + e, and the A operand is read in the same order.
template <int J, bool kWithTw = true, typename LdsT>
__device__ __forceinline__ void t_column(LdsT& sm, int grp, int c16) {
  const int cj = 16 * J + c16;
  const float fb = sm.bt[cj], fw = kWithTw ? fb * sm.eg[cj] : 0.0f;
  f4 Tc[4];
#pragma unroll
  for (int e = 0; e < 4; e++) Tc[J][e] = sm.Tm[(16 * J + 4 * grp + e) * kAP + cj];
  // X[bi] accumulates sum_k A_bi,k T_kJ. The terms with k = J only need the diagonal block, so they are all issued
  // first; after that each block row adds just the term of the block found last, so the dependent chain per block
  // row is one product plus the multiplication by T_ii.
  f4 X[4];
#pragma unroll
  for (int bi = J + 1; bi < 4; bi++) {
    const f4 av = lds4(&sm.Tm[(16 * bi + c16) * kAP + 16 * J + 4 * grp]);
    X[bi] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int e = 0; e < 4; e++) X[bi] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], Tc[J][e], X[bi], 0, 0, 0);
  }
#pragma unroll
  for (int bi = J + 1; bi < 4; bi++) {
    const float* arow = &sm.Tm[(16 * bi + c16) * kAP];
    if (bi > J + 1) {
      const f4 av = lds4(arow + 16 * (bi - 1) + 4 * grp);
#pragma unroll
      for (int e = 0; e < 4; e++) X[bi] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], Tc[bi - 1][e], X[bi], 0, 0, 0);
    }
    const f4 tv = lds4(arow + 16 * bi + 4 * grp);
    f4 Y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int e = 0; e < 4; e++) Y = __builtin_amdgcn_mfma_f32_16x16x4f32(tv[e], X[bi][e], Y, 0, 0, 0);
    Tc[bi] = -Y;
    // the middle terms A_b,bi T_bi,J of the rows below, now that T_bi,J is known
#pragma unroll
    for (int b2 = bi + 2; b2 < 4; b2++) {
      const f4 av = lds4(&sm.Tm[(16 * b2 + c16) * kAP + 16 * bi + 4 * grp]);
#pragma unroll
      for (int e = 0; e < 4; e++) X[b2] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], Tc[bi][e], X[b2], 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int t = 16 * bi + 4 * grp + e;
      sm.Tb[t * kTP + cj] = (_Float16)(Tc[bi][e] * fb);
      if constexpr (kWithTw) sm.Tw[t * kTP + cj] = (_Float16)(Tc[bi][e] * fw);
    }
  }
}

}  // namespace
}  // namespace ha
