// MatMulNBits projections, the matmuls either side of the hybrid-attention path, gfx950.
//
// Reference: web/public/gemmbench/kernels.js:1-14 (weight formats) and 15-36 (block decode),
// convert/export_engine.py:17-26 (int4 RTN export), web/public/engine/engine.js:236-246 (matmul dispatch) and
// engine.js:17-33 (kernel choice by M), web/public/engine/wgsl.js:94-110 (FWHT input rotation).
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
//   M <= 64  mnb_gemv_kernel: a workgroup owns 16 output columns and its 8 waves split the K blocks; each lane
//            dequantises a whole packed block into the f16 B operands of v_mfma_f32_16x16x32_f16 (no LDS), the a
//            rows are the A operand (16 rows per tile, up to 4 tiles share each dequantised operand), and the
//            waves' partial sums meet in LDS.
//   above    mnb_gemm_kernel: compute bound. A tiled MFMA GEMM (128 or 256 x 128 workgroup tiles) whose weight
//            tiles are dequantised on their way into LDS, so the weights stay packed in HBM. With few output tiles
//            the K range is split over workgroups and mnb_split_sum_kernel adds the fp32 partials in order.
// All three dequantise with the same f16 arithmetic (dequant8_pk: each weight rounded to f16 once), accumulate in
// fp32 and round the output to f16. Results are deterministic: a split K range is summed in a fixed order that
// depends only on the shape.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>

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

// y for larger M: a tiled f16 GEMM whose weight tiles are dequantised on the way into LDS, so the weights are read
// packed (0.5 byte per weight for 4 bits) and no f16 copy exists. Workgroup tile 128 or 256 rows (the larger when
// there are enough tiles: each dequantised weight then serves twice the rows) x 128 columns, k tiles of
// 64 (two packed blocks); 4 waves (8 for 256-row tiles), wave (wm, wn) = (w / 2, w % 2) owns rows 64 wm .. + 63 and
// columns 64 wn .. + 63
// as 2 x 2 tiles of v_mfma_f32_32x32x16_f16 (A operand lane l: row l % 32 of a, k 8 (l / 32) .. + 7 of the
// 16-step; B operand: column l % 32, the same k; D: column l % 32, rows 8 (v / 4) + 4 (l / 32) + v % 4).
// The a tile and the dequantised weight tile are double-buffered in LDS, 16-byte chunks XOR-swizzled by row. The a
// tiles arrive by DMA (global_load_lds_dwordx4), issued one tile ahead; the packed weights of the next two tiles
// sit in a register ring and are dequantised into the other stage while the current one is multiplied; one barrier
// per k tile. Rows past M and columns past N load clamped rows and are not stored; a k tile past the last
// block (K % 64 == 32) is zero in both operands. Tiles are numbered so that each XCD (workgroup id % 8) takes a
// contiguous range of them, n fastest, sharing a rows in its L2.
constexpr int kTN = 128, kTK = 64;
typedef float f16v __attribute__((ext_vector_type(16)));
// 16-byte chunk c (k 8 c .. 8 c + 7 of the tile) of row r sits in slot 8 r + (c ^ (r & 7)): the MFMA operand reads
// of 32 rows at one chunk then fall in distinct banks without padding
__device__ __forceinline__ int swz(int r, int c) { return 8 * r + (c ^ (r & 7)); }
template <int BITS, int GROUP, bool ASYM, int WMW>
__global__ __launch_bounds__(128 * WMW) void mnb_gemm_kernel(MnbArgs a) {
  constexpr int kTM = 64 * WMW;                 // WMW wave rows of 64 a rows, 2 wave columns of 64 weight columns
  constexpr int kSPT = 8 / WMW;                 // dequantised 8-element slices per thread and k tile
  constexpr int kTPB = 4 / kSPT;                // threads per packed block
  constexpr int kNB = ASYM ? 3 : 2;             // load instructions per thread for one tile's weights
  // two stages of each tile as separate objects, so that the compiler can tell the stage being read from the one
  // the DMA is filling and does not wait for the DMA before every read
  __shared__ h8 As0[kTM * 8], As1[kTM * 8];
  __shared__ h8 Bs0[kTN * 8], Bs1[kTN * 8];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), wm = w >> 1, wn = w & 1;
  const int ntn = (a.N + kTN - 1) / kTN, ntm = (a.M + kTM - 1) / kTM, ntiles = ntn * ntm;
  int id = blockIdx.x;
  if (ntiles % 8 == 0) id = (id % 8) * (ntiles / 8) + id / 8;
  const int tn = id % ntn, tm = id / ntn;
  const int nblk = a.K / kBlk, nkt = (nblk + 1) / 2, ng = a.K / GROUP;
  // this workgroup's K range: tiles kt0 .. kt1 - 1 (all of them unless the product is split)
  const int sp_idx = blockIdx.y, kt0 = sp_idx * nkt / a.split, kt1 = (sp_idx + 1) * nkt / a.split;
  // a tiles go global -> LDS directly: wave w's instruction i fills slots 64 (4 w + i) .. + 63 (rows 8 (4 w + i) ..
  // + 7); lane l takes slot 64 (4 w + i) + l, i.e. row 8 (4 w + i) + l / 8 and the chunk swizzled into slot l % 8
  const _Float16* arow_p[4];
  int achunk[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = 8 * (4 * w + i) + (lane >> 3);
    arow_p[i] = (const _Float16*)a.a + (size_t)min(tm * kTM + r, a.M - 1) * a.K;
    achunk[i] = (lane & 7) ^ (r & 7);
  }
  auto issue_a = [&](int kt, h8* stage) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      // past the last block (K % 64 == 32, or a tile past the end) read the row's last real block: the weights
      // there are zero, so finite activations add nothing
      int blk = 2 * kt + (achunk[i] >> 2);
      const int c = blk < nblk ? achunk[i] : (achunk[i] & 3);
      blk = min(blk, nblk - 1);
      const _Float16* src = arow_p[i] + (size_t)blk * kBlk + 8 * (c & 3);
      // global_load_lds_dwordx4 written out: the compiler would otherwise wait for every DMA in flight before any
      // LDS read; the k-loop's explicit waits order the DMAs instead. m0 (the DMA's LDS base) is a register the
      // compiler reserves and does not preserve across asm; this is sound because no compiler-generated code in
      // these kernels keeps a value in m0 (tests/test_asm_guards.py checks the assembly)
      const unsigned lds = __builtin_amdgcn_readfirstlane(
          (unsigned)(size_t)(__attribute__((address_space(3))) h8*)&stage[64 * (4 * w + i)]);
      asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(src) : "memory", "m0");
    }
  };
  // weights: column tn * 128 + bc, block half bh, slices s0 .. s0 + kSPT - 1, loaded into a 2-deep register ring
  const int bc = tid / (2 * kTPB), bh = (tid / kTPB) & 1, s0 = (tid % kTPB) * kSPT;
  const int wcol = min(tn * kTN + bc, a.N - 1);
  gptr<unsigned> wp = gp<unsigned>(a.q) + (size_t)wcol * nblk * BITS;
  gptr<unsigned short> sp = gp<unsigned short>(a.s) + (size_t)wcol * ng;
  gptr<unsigned short> bp = ASYM ? gp<unsigned short>(a.b) + (size_t)wcol * ng : sp;
  typedef unsigned uw __attribute__((ext_vector_type(BITS)));
  uw wr[2];
  unsigned short sr[2], br[2];  // f16 bits, loaded zero-extended into whole registers
  auto load_b = [&](int kt, int r) {
    const int bb = min(2 * kt + bh, nblk - 1);
    wr[r] = *(const __attribute__((address_space(1))) uw*)(wp + bb * BITS);
    sr[r] = sp[bb * kBlk / GROUP];
    if constexpr (ASYM) br[r] = bp[bb * kBlk / GROUP];
  };
  auto store_b = [&](int kt, int r, h8* buf) {
    const bool okb = kt < kt1 && 2 * kt + bh < nblk;
    const h2 sc = splat2(__builtin_bit_cast(_Float16, sr[r]));
    const h2 bi = splat2(ASYM ? __builtin_bit_cast(_Float16, br[r]) : (_Float16)0.0f);
    unsigned wd[BITS];
#pragma unroll
    for (int j = 0; j < BITS; j++) wd[j] = wr[r][j];
#pragma unroll
    for (int j = s0; j < s0 + kSPT; j++) {
      const h8 v = dequant8_pk<BITS, ASYM>(wd, j, sc, bi);
      buf[swz(bc, 4 * bh + j)] = okb ? h8{v[0], v[2], v[4], v[6], v[1], v[3], v[5], v[7]} : h8{};
    }
  };
  f16v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = f16v{};
  const int fr = lane & 31, fh = lane >> 5;
  auto compute = [&](const h8* stage, const h8* buf) {
#pragma unroll
    for (int ks = 0; ks < kTK / 16; ks++) {
      h8 af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        af[i] = stage[swz(64 * wm + 32 * i + fr, 2 * ks + fh)];
        bf[i] = buf[swz(64 * wn + 32 * i + fr, 2 * ks + fh)];
      }
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };
  // s_waitcnt on vmcnt <= n (expcnt untouched) and, with lgkm, on this wave's LDS writes
  auto wait_vm = [](auto n, bool lgkm = false) {
    constexpr int v = decltype(n)::value;
    if (lgkm)
      __builtin_amdgcn_s_waitcnt((v & 15) | ((v >> 4) << 14) | (7 << 4));
    else
      __builtin_amdgcn_s_waitcnt((v & 15) | ((v >> 4) << 14) | (7 << 4) | (15 << 8));
  };
  // The k-loop's barrier: every wave's weight stores and its a tile kt + 1 have landed, then s_barrier. Written
  // out because __syncthreads() carries a release fence, which waits for every load in flight (the a tiles arrive
  // by DMA into LDS) and so would empty the pipeline; the empty asm statements keep the compiler from moving LDS
  // accesses across.
  auto barrier_after = [&](auto n) {
    asm volatile("" ::: "memory");
    wait_vm(n, true);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // prologue: a tile kt0 and its weights in LDS stage 0, the weights of tile kt0 + 1 in the ring
  issue_a(kt0, As0);
  load_b(kt0, 0);
  load_b(kt0 + 1, 1);
  store_b(kt0, 0, Bs0);
  wait_vm(std::integral_constant<int, kNB>{}, true);  // all but the weights of tile 1
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  // iteration kt (stage r = kt % 2): issue a tile kt + 1 into the other stage; multiply tile kt; load tile kt + 2's
  // weights into the ring slot tile kt's left, dequantise tile kt + 1's into the other stage; wait for a tile kt + 1
  // (tile kt + 2's weights may stay in flight); one barrier. Run to an even tile count with no branch inside, so
  // every stage and ring index is a constant; tiles past the last block are zero in the weight operand.
  const int kt_end = kt0 + ((kt1 - kt0 + 1) & ~1);
  for (int k0 = kt0; k0 < kt_end; k0 += 2) {
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int kt = k0 + r;
      issue_a(kt + 1, r ? As0 : As1);
      compute(r ? As1 : As0, r ? Bs1 : Bs0);
      __builtin_amdgcn_sched_barrier(0);
      load_b(kt + 2, r);
      store_b(kt + 1, r ^ 1, r ? Bs0 : Bs1);
      barrier_after(std::integral_constant<int, kNB>{});
    }
  }
  // the last iterations issued a tiles past the end: let them land before the workgroup's LDS can be reused
  wait_vm(std::integral_constant<int, 0>{});
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int n = tn * kTN + 64 * wn + 32 * j + fr;
      if (n >= a.N) continue;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int m = tm * kTM + 64 * wm + 32 * i + 8 * (v >> 2) + 4 * fh + (v & 3);
        if (m >= a.M) continue;
        if (a.split > 1)
          a.ws[((size_t)sp_idx * a.M + m) * a.N + n] = acc[i][j][v];
        else
          ((_Float16*)a.y)[(size_t)m * a.N + n] = (_Float16)acc[i][j][v];
      }
    }
}

// y = the sum of the split GEMM's partial products, in split order (so the result depends only on the shape)
__global__ __launch_bounds__(256) void mnb_split_sum_kernel(const float* ws, _Float16* y, long mn4, int split) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= mn4) return;
  f4 t = reinterpret_cast<const f4*>(ws)[i];
  for (int s = 1; s < split; s++) t += reinterpret_cast<const f4*>(ws)[(size_t)s * mn4 + i];
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  reinterpret_cast<h4*>(y)[i] = h4{(_Float16)t[0], (_Float16)t[1], (_Float16)t[2], (_Float16)t[3]};
}



// In-place orthonormal Walsh-Hadamard transform (Sylvester order) of each contiguous n-block of an f16 row, one
// workgroup per block (wgsl.js:94-110): the online input rotation of a tensor exported with `had: n`.
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
hipError_t launch_gemm(const MnbArgs& a, hipStream_t s) {
  // 256-row tiles (8 waves) when they still give every CU a workgroup, else 128-row tiles (4 waves)
  const long ntn = (a.N + kTN - 1) / kTN, tiles256 = ntn * ((a.M + 255) / 256);
  if (tiles256 >= 256)
    hipLaunchKernelGGL((mnb_gemm_kernel<BITS, GROUP, ASYM, 4>), dim3((unsigned)tiles256, a.split), dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL((mnb_gemm_kernel<BITS, GROUP, ASYM, 2>), dim3((unsigned)(ntn * ((a.M + 127) / 128)), a.split),
                       dim3(256), 0, s, a);
  if (a.split > 1) {
    const long mn4 = (long)a.M * a.N / 4;
    hipLaunchKernelGGL(mnb_split_sum_kernel, dim3((unsigned)((mn4 + 255) / 256)), dim3(256), 0, s, a.ws,
                       (_Float16*)a.y, mn4, a.split);
  }
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
struct GemmF {
  static hipError_t run(const MnbArgs& a, hipStream_t s) { return launch_gemm<B, G, S>(a, s); }
};
}  // namespace

hipError_t mnb_check(const MnbArgs& a) {
  if (a.N <= 0 || a.K <= 0 || a.K % 32) return hipErrorInvalidValue;  // N % 16 is checked per matmul
  if (!(a.bits == 2 || a.bits == 3 || a.bits == 4) || !(a.group == 32 || a.group == 64) || a.K % a.group)
    return hipErrorInvalidValue;
  if (!a.q || !a.s || (a.asym && !a.b)) return hipErrorInvalidValue;
  return hipSuccess;
}

bool mnb_packed_path(int M, int N, int K) {
  // Measured on MI355X, back-to-back calls on the model's projection shapes (N x K from 2048 x 2048 to
  // 12288 x 2048): up to 64 rows the packed-weight kernels are at least as fast as the tiled GEMM on every shape
  // (at 64 rows 10-28 us against 27-71 us).
  return M <= 64;
}

hipError_t launch_mnb_gemv(const MnbArgs& a, hipStream_t s) {
  if (a.M < 1 || a.M > 64 || !a.a || !a.y) return hipErrorInvalidValue;
  return a.M <= kLanesRows ? dispatch_fmt<GemvLanesF>(a, s) : dispatch_fmt<GemvF>(a, s);
}

int mnb_gemm_split(int M, int N, int K) {
  // Fewer output tiles than CUs leave CUs idle behind one long K loop each (about 0.85 us per 64-deep k tile):
  // split K so that about 384 workgroups run, each over at least 4 k tiles, with at most 64 MiB of fp32 partials.
  const long ntn = (N + kTN - 1) / kTN, tiles256 = ntn * ((M + 255) / 256);
  const long tiles = tiles256 >= 256 ? tiles256 : ntn * ((M + 127) / 128);
  const int nkt = (K / kBlk + 1) / 2;
  if (tiles >= 256) return 1;
  long sp = std::min<long>((384 + tiles - 1) / tiles, nkt / 4);
  while (sp > 1 && sp * M * (long)N * 4 > (64L << 20)) sp--;
  return (int)std::max<long>(sp, 1);
}

hipError_t launch_mnb_gemm(const MnbArgs& a, hipStream_t s) {
  if (a.M < 1 || !a.a || !a.y || a.split < 1 || (a.split > 1 && !a.ws)) return hipErrorInvalidValue;
  return dispatch_fmt<GemmF>(a, s);
}

// Fixed scratch for the allocation-free GEMM entry point: the fp32 partial products of a split K range. One copy per
// GPU (a device global is instantiated on each device the code object is loaded on), held until the process ends.
// Host code never passes the array's name to a kernel: it is a host-side stand-in there, not a device address. The
// address is looked up once per device by mnb_scratch_setup (with that device current) and kept in g_scratch_ptr.
static __device__ __align__(256) float scratch[kMnbScratchBytes / sizeof(float)];
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

hipError_t mnb_scratch_setup(int device) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device]) return hipSuccess;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (!p) return hipErrorInvalidSymbol;
  g_scratch_ptr[device] = p;
  return hipSuccess;
}

float* mnb_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return static_cast<float*>(g_scratch_ptr[device]);
}

hipError_t launch_fwht(void* x, long rows_times_k, int n, hipStream_t s) {
  if (n < 2 || (n & (n - 1)) || n > 8192 || rows_times_k % n) return hipErrorInvalidValue;
  const float scale = (float)(1.0 / std::sqrt((double)n));  // the reference's constant 1 / sqrt(n), rounded to f32
  hipLaunchKernelGGL(fwht_kernel, dim3((unsigned)(rows_times_k / n)), dim3(256), sizeof(float) * n, s, (_Float16*)x, n,
                     scale);
  return hipGetLastError();
}

}  // namespace ha
