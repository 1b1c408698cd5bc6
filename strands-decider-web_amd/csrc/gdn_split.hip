// Chunked gated-delta prefill in three kernels, gfx950 (HA_CHUNKED_SPLIT; HA_CHUNKED for few sequence-heads).
//
// Same semantics and chunk geometry as gdn_chunk.hip (the sequential rule of reference
// web/public/engine/wgsl.js:124-187 + 252-268 in the chunked WY/UT form, chunk 64, chunk boundaries at s0 + 64 k),
// split along the one dependency that is sequential. For a chunk with state S at its start:
//   A = strictly_lower(beta_t (k^_t . k^_t') e^(gc_t - gc_t'))    T = (I + A)^-1
//   W = T diag(beta e^gc) k^      U = T diag(beta) v^      V_new = U - W S
//   o = diag(e^gc) q^ S + Att V_new,  Att = causal(q^ k^T e^(gc_t - gc_t'))   (t' <= t)
//   S <- e^(gc_63) S + (diag(e^(gc_63 - gc)) k^)^T V_new                       (complete chunks only)
// Everything except the products with S depends only on the chunk's own rows, and of those only the state update is
// sequential, so
//   gdn_prep_kernel  runs one workgroup per (chunk, sequence, head), all chunks at once over the whole chip, and
//                    writes each chunk's "image": the MFMA A operands q~ = diag(e^gc) q^, W, K~^T and Att and the
//                    matrix U, every operand block in lane order (64 lanes x 16 bytes), so that the later kernels read
//                    each with one conflict-free 16-byte LDS load and no lane moves;
//   gdn_scan_kernel  runs two roles in one launch. The state pass carries the state through the chunks in order
//                    (four workgroups per (sequence, head) on 32 value columns each, X = W S -> V_new ->
//                    S <- e^(gc_63) S + K~^T V_new per chunk) and leaves the packed state at every chunk's start in
//                    that chunk's scratch. The output pass, one workgroup per (chunk, sequence, head) on the other
//                    CUs, takes each chunk as soon as its packed state is published: o^T = S^T q~^T + V_new^T Att^T,
//                    the gated norm (GNORM), the stores.

#include <stddef.h>

#include "gdn_common.h"

namespace ha {
namespace {

// ---- chunk image layout (bytes) ----
constexpr int kBlk = 1024;            // one A-operand block: 64 lanes x 16 bytes (8 f16)
constexpr int kOffQ = 0;              // q~ blocks [tb 0..3][kb 0..3]: rows 16 tb + (l & 15), state rows as K
constexpr int kOffW = 16 * kBlk;      // W blocks [tb][kb], same arrangement
constexpr int kOffK = 32 * kBlk;      // K~^T blocks [ib 0..7][kb 0..1]: state rows 16 ib + (l & 15), chunk rows as K
constexpr int kOffA = 48 * kBlk;      // Att blocks [tb 0..3][kb 0..1] (blocks with kb > tb / 2 are zero, never read)
constexpr int kOffU = 56 * kBlk;      // U in the D layout: blocks [tb 0..3][jt 0..7] of 64 lanes x 4 f16
constexpr int kOffS = 72 * kBlk;      // e^(gc_63) as f32
constexpr int kImg = 73 * kBlk;       // whole 1 KiB DMA instructions
// After the image, the state at the chunk's start as the state pass leaves it, packed as the products with S read it (f16 B operands):
// the h8 Sb[kb][jj] of lane l of wave w (state rows {32 kb + 4 grp + e} U {32 kb + 16 + 4 grp + e} of value column
// 32 w + 16 jj + (l & 15)) at byte ((w * 4 + kb) * 2 + jj) * 1024 + 16 l.
constexpr int kOffSnap = kImg;
constexpr int kSnap = 32 * kBlk;
constexpr int kChunkScratch = kImg + kSnap;

typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i2v __attribute__((ext_vector_type(2)));

// Stores into one chunk's image through a buffer resource (raw 16 / 8-byte stores; offsets in bytes).
struct ImgOut {
  __amdgpu_buffer_rsrc_t r;
  __device__ explicit ImgOut(void* base) : r(__builtin_amdgcn_make_buffer_rsrc(base, 0, kImg, 0x00020000)) {}
  __device__ void st16(int off, const h8& v) const {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i4v, v), r, off, 0, 0);
  }
  __device__ void st8(int off, const h4& v) const {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i2v, v), r, off, 0, 0);
  }
  __device__ void st4(int off, float v) const { __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v), r, off, 0, 0); }
};

__device__ __forceinline__ h8 join(const f4& lo, const f4& hi) { return pack_b(lo, hi); }

// ------------------------------------------------------------------------------------------------------------------
// gdn_prep_kernel: 4 waves. Conv lane pt: rows 8 (pt / 32) .. + 7 of the chunk, channels 4 (pt % 32) .. + 3 of each
// of q, k and v; q^, k^, k^T and v^T go to LDS. Wave 3 forms the gates, the diagonal blocks of A and their forward
// substitution; waves 0..2 the six below-diagonal blocks of A and then one block column of T each. The products
// are then spread over the four waves and written to the image straight from registers.
constexpr int kPW = 4, kPT = 64 * kPW;
constexpr int kPRG = 8;  // rows per conv lane
constexpr int kPG = kPW - 1;

// 80,128 bytes, so that two workgroups share a CU (one's row loads overlap the other's arithmetic). The arrays share
// storage by lifetime: q^ until Att and q~ are written, then A and T (fp32); k^ and the conv taps until A is formed,
// then T diag(beta) and T diag(beta e^gc).
struct PrepLds {
  union {
    _Float16 Qs[kCH * kQP];   // q^ / sqrt(DK), [t][i]
    float Tm[kCH * kAP];      // A, then T (fp32)
  };
  union {
    struct {
      _Float16 Ks[kCH * kQP];   // k^, [t][i]
      float cw[12][32][kKC];    // conv taps: channel 4 g + c of q (c < 4), k (4 <= c < 8), v (c >= 8) at cw[c][g]
    };
    struct {
      _Float16 Tb[kCH * kTP];   // T diag(beta), [t][t'] (blocks above the diagonal zero)
      _Float16 Tw[kCH * kTP];   // T diag(beta e^gc)
    };
  };
  _Float16 KT[kDK * kTP];   // k^ transposed, [i][t], swizzled by kt16
  _Float16 VT[kDV * kTP];   // v^ transposed, [j][t], swizzled by vt16
  float eg[kCH], ed[kCH], gc[kCH], rowf[kCH], colf[3][kCH];
  float bt[kCH];            // beta
  float brow[kCH];          // beta_t rowf_t
};
static_assert(sizeof(PrepLds) <= 80 * 1024, "two preparation workgroups per CU");

template <typename T>
__global__ __launch_bounds__(kPT) void gdn_prep_kernel(GdnArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  PrepLds& sm = *reinterpret_cast<PrepLds*>(lds_raw);
  const int c = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.H, h = bh % a.H;
  const int tid0 = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  const int end = a.P + a.L;
  const int cs = a.s0 + kCH * c;
  const int m = min(kCH, end - cs);
  const float qscale = 0.08838834764831845f;  // 1/sqrt(128)
  const unsigned rowb = (unsigned)a.stride * sizeof(T);
  const char* const seq_in = (const char*)a.in + (size_t)b * a.L * rowb;
  char* const slot = (char*)a.img + ((size_t)bh * a.img_chunks + c) * kChunkScratch;
  const ImgOut img(slot);

  const float na = gp<float>(a.negA)[h], db = gp<float>(a.dtb)[h];
  const int aoff = a.C + a.H * kDV + h, boff = aoff + a.H;

  // raw rows cs-3 .. cs+63 of this lane's q, k and v channels (x[i][0..3] q, [4..7] k, [8..11] v): every load
  // instruction reads whole 512-byte row segments. Rows past the end repeat the last row (they only feed conv
  // outputs past the end, which are masked); rows before P come from the tail buffer.
  const int pt = tid0, rg = pt >> 5, cl = pt & 31;
  float x[kPRG + kKC - 1][12];
  const RowSrc src = row_src(a);
  {
    const int col = h * kDK + 4 * cl;
    const bool fast = cs - (kKC - 1) >= a.P && cs + kCH <= end;
    const char* base = seq_in + (ptrdiff_t)(cs - (kKC - 1) - a.P) * rowb;
    const unsigned off = (unsigned)(kPRG * rg) * rowb + (unsigned)col * (unsigned)sizeof(T);
#pragma unroll
    for (int i = 0; i < kPRG + kKC - 1; i++) {
      const int r = min(cs + kPRG * rg - (kKC - 1) + i, end - 1);
      const gptr<T> q = fast ? gp<T>(base + (size_t)i * rowb + off) : row_of<T>(a, src, b, r) + col;
      load4(q, x[i]);
      load4(q + a.H * kDK, x[i] + 4);
      load4(q + 2 * a.H * kDK, x[i] + 8);
    }
  }
  // the gate wave: a and b of row `lane` of the chunk (rows past the end are masked where the gates are formed)
  float ga = 0.0f, gb = 0.0f;
  if (w == kPG) {
    const int lane = tid0 & 63;
    const gptr<T> grow = row_of<T>(a, src, b, min(cs + lane, end - 1));
    ga = (float)grow[aoff];
    gb = (float)grow[boff];
  }
  // conv taps to LDS, behind the row loads
  for (int i = tid0; i < 3 * 128 * kKC; i += kPT) {
    const int lc = i / kKC, j = i % kKC, part = lc >> 7;
    const int ch = part * a.H * kDK + h * kDK + (lc & 127);
    sm.cw[(lc & 3) + 4 * part][(lc & 127) >> 2][j] = gp<float>(a.conv_w)[(size_t)ch * kKC + j];
  }
  __syncthreads();  // conv taps visible

  // conv + SiLU; q and k rows l2-normalised (q also scaled by 1/sqrt(DK); a row's 128 channels of q, of k, sit in
  // the 32 lanes of a half wave): q^ and k^ rows to LDS, k^ and v^ columns (8 rows each) to the transposed tiles
  {
    float u[kPRG][12], ssq[kPRG], ssk[kPRG];
#pragma unroll
    for (int r = 0; r < kPRG; r++) ssq[r] = ssk[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < 12; k++) {
      const f4 wc = lds4(sm.cw[k][cl]);
#pragma unroll
      for (int r = 0; r < kPRG; r++) {
        float sv = wc[0] * x[r][k];
        sv = fmaf(wc[1], x[r + 1][k], sv);
        sv = fmaf(wc[2], x[r + 2][k], sv);
        sv = fmaf(wc[3], x[r + 3][k], sv);
        u[r][k] = kPRG * rg + r < m ? silu(sv) : 0.0f;
        if (k < 4)
          ssq[r] = fmaf(u[r][k], u[r][k], ssq[r]);
        else if (k < 8)
          ssk[r] = fmaf(u[r][k], u[r][k], ssk[r]);
      }
    }
    float rkv[kPRG];
#pragma unroll
    for (int r = 0; r < kPRG; r++) {
      float sq = row_sum16(ssq[r]), sk = row_sum16(ssk[r]);
      sq += __shfl_xor(sq, 16);
      sk += __shfl_xor(sk, 16);
      const float rq = rsqrtf(sq + 1e-6f) * qscale, rk = rsqrtf(sk + 1e-6f);
      rkv[r] = rk;
      const int t = kPRG * rg + r;
      *reinterpret_cast<h4*>(sm.Qs + t * kQP + 4 * cl) =
          h4{(_Float16)(u[r][0] * rq), (_Float16)(u[r][1] * rq), (_Float16)(u[r][2] * rq), (_Float16)(u[r][3] * rq)};
      *reinterpret_cast<h4*>(sm.Ks + t * kQP + 4 * cl) =
          h4{(_Float16)(u[r][4] * rk), (_Float16)(u[r][5] * rk), (_Float16)(u[r][6] * rk), (_Float16)(u[r][7] * rk)};
    }
#pragma unroll
    for (int cc = 0; cc < 4; cc++) {
      h8 kt, vt;
#pragma unroll
      for (int r = 0; r < kPRG; r++) {
        kt[r] = (_Float16)(u[r][4 + cc] * rkv[r]);
        vt[r] = (_Float16)u[r][8 + cc];
      }
      *reinterpret_cast<h8*>(sm.KT + kt16(4 * cl + cc, rg)) = kt;
      *reinterpret_cast<h8*>(sm.VT + vt16(4 * cl + cc, rg)) = vt;
    }
  }
  // gates: beta, the cumulative log decay (lane = row) and the vectors derived from it
  if (w == kPG) {
    const int lane = tid0 & 63;
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
    const float rf = __expf(gcr - __shfl(gcr, lane & ~15));
    sm.gc[lane] = gcr;
    sm.eg[lane] = __expf(gcr);
    sm.bt[lane] = btr;
    sm.ed[lane] = __expf(gl - gcr);
    sm.rowf[lane] = rf;
    sm.brow[lane] = btr * rf;
#pragma unroll
    for (int i = 1; i < 4; i++) {
      const float gi = __shfl(gcr, 16 * i);
      sm.colf[i - 1][lane] = lane < 16 * i ? __expf(gi - gcr) : 0.0f;
    }
  }
  __syncthreads();  // q^, k^, k^T, v^T, gates

  const int lane = tid0 & 63, grp = lane >> 4, c16 = lane & 15;
  const int lo16 = 16 * lane;
  // Att^T = k^ q^T, decay-masked: tile (a, tb) holds Att[16 tb + c16][16 a + 4 grp + e]; Att block (tb, kb) is the
  // tile pair a = 2 kb, 2 kb + 1 (a tile above the diagonal, a > tb, is zero). The six blocks that are read:
  // wave 0: (0,0) and (2,1); wave 1: (1,0); wave 2: (2,0); wave 3: (3,0) and (3,1).
  {
    auto att_tile = [&](int ta, int tb) {
      const _Float16* ab = sm.Ks + (16 * ta + c16) * kQP + 8 * grp;
      const _Float16* bb = sm.Qs + (16 * tb + c16) * kQP + 8 * grp;
      f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 4; ks++)
        acc = mfma16(*reinterpret_cast<const h8*>(ab + 32 * ks), *reinterpret_cast<const h8*>(bb + 32 * ks), acc);
      const int t = 16 * tb + c16, tp0 = 16 * ta + 4 * grp;
      const float gt = sm.gc[t];
      const f4 gp4 = lds4(&sm.gc[tp0]);
#pragma unroll
      for (int e = 0; e < 4; e++) acc[e] = tp0 + e <= t ? acc[e] * __expf(fminf(gt - gp4[e], 0.0f)) : 0.0f;
      return acc;
    };
    const f4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};
    auto att_block = [&](int tb, int kb) {
      const f4 lo = att_tile(2 * kb, tb);
      const f4 hi = 2 * kb + 1 <= tb ? att_tile(2 * kb + 1, tb) : z4;
      img.st16(kOffA + (tb * 2 + kb) * kBlk + lo16, join(lo, hi));
    };
    if (w == 0) {
      att_block(0, 0);
      att_block(2, 1);
    } else if (w == 1) {
      att_block(1, 0);
    } else if (w == 2) {
      att_block(2, 0);
    } else {
      att_block(3, 0);
      att_block(3, 1);
    }
  }
  // q~ blocks (tb = w, kb 0..3): q^ rows scaled by e^gc, K in the permuted order
  {
    const int t = 16 * w + c16;
    const float eg = sm.eg[t];
#pragma unroll
    for (int kb = 0; kb < 4; kb++) {
      const h8 q = perm_a(sm.Qs, kQP, t, kb, grp);
      h8 o;
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] = (_Float16)((float)q[e] * eg);
      img.st16(kOffQ + (w * 4 + kb) * kBlk + lo16, o);
    }
  }
  __syncthreads();  // q^ is dead: A and T reuse its storage
  if (w == kPG) {
    // the four diagonal blocks of A: k^ k^T (A and B operands are the same rows), beta and decay, strictly lower
    f4 dg[4];
#pragma unroll
    for (int d = 0; d < 4; d++) {
      const _Float16* kr = sm.Ks + (16 * d + c16) * kQP + 8 * grp;
      dg[d] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 4; ks++) {
        const h8 kv = *reinterpret_cast<const h8*>(kr + 32 * ks);
        dg[d] = mfma16(kv, kv, dg[d]);
      }
    }
#pragma unroll
    for (int d = 0; d < 4; d++) {
      const int tp = 16 * d + c16, t0 = 16 * d + 4 * grp;
      const float gp_ = sm.gc[tp];
      const f4 gt = lds4(&sm.gc[t0]), bv = lds4(&sm.bt[t0]);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int t = t0 + e;
        const float dec = __expf(fminf(gt[e] - gp_, 0.0f));
        sm.Tm[t * kAP + tp] = tp < t ? bv[e] * dg[d][e] * dec : 0.0f;
      }
    }
  } else {
    // below-diagonal blocks of A: tiles 1,3,4,6,7,8 of the 10 on or below the diagonal, two per wave
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int jt = w == 0 ? (k ? 3 : 1) : w == 1 ? (k ? 6 : 4) : (k ? 8 : 7);
      const int ti = jt >= 6 ? 3 : jt >= 3 ? 2 : 1, tj = jt - ti * (ti + 1) / 2;
      const _Float16* ab = sm.Ks + (16 * ti + c16) * kQP + 8 * grp;
      const _Float16* bb = sm.Ks + (16 * tj + c16) * kQP + 8 * grp;
      f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 4; ks++)
        acc = mfma16(*reinterpret_cast<const h8*>(ab + 32 * ks), *reinterpret_cast<const h8*>(bb + 32 * ks), acc);
      // e^(gc_t - gc_t') factors into two terms <= 1 below the diagonal blocks
      const int tp = 16 * tj + c16, t0 = 16 * ti + 4 * grp;
      const float cf = sm.colf[ti - 1][tp];
      const f4 bf = lds4(&sm.brow[t0]);
#pragma unroll
      for (int e = 0; e < 4; e++) sm.Tm[(t0 + e) * kAP + tp] = acc[e] * bf[e] * cf;
    }
  }
  __syncthreads();  // A complete; k^ and the taps are dead: T diag(beta), T diag(beta e^gc) reuse their storage
  // blocks above the diagonal of T diag(beta) and T diag(beta e^gc) are read by full 32-wide K blocks and never
  // written otherwise: row block rb (< 3) has 6 - 2 rb such 8-column groups per row, from column 16 (rb + 1)
  if (tid0 < 192) {
    const int k = tid0, rb = k < 96 ? 0 : k < 160 ? 1 : 2, k2 = k - (rb == 0 ? 0 : rb == 1 ? 96 : 160);
    const int ng = 6 - 2 * rb, t = 16 * rb + k2 / ng, g = k2 % ng + 2 * (rb + 1);
    *reinterpret_cast<h8*>(sm.Tb + t * kTP + 8 * g) = h8{};
    *reinterpret_cast<h8*>(sm.Tw + t * kTP + 8 * g) = h8{};
  }
  if (w == kPG) {
    // lane (grp, c16): column c16 of diagonal block grp, rows in order (left-looking)
    const int base = 16 * grp;
    float pc[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const float* ar = &sm.Tm[(base + r) * kAP + base];
      float acc = r == c16 ? 1.0f : 0.0f;
#pragma unroll
      for (int j = 0; j < r; j++) acc = fmaf(-ar[j], pc[j], acc);
      pc[r] = acc;
    }
    const float cb = sm.bt[base + c16], cw = cb * sm.eg[base + c16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      sm.Tm[(base + r) * kAP + base + c16] = pc[r];
      sm.Tb[(base + r) * kTP + base + c16] = (_Float16)(pc[r] * cb);
      sm.Tw[(base + r) * kTP + base + c16] = (_Float16)(pc[r] * cw);
    }
  }
  __syncthreads();
  if (w == 0)
    t_column<0, true>(sm, grp, c16);
  else if (w == 1)
    t_column<1, true>(sm, grp, c16);
  else if (w == 2)
    t_column<2, true>(sm, grp, c16);
  __syncthreads();  // T diag(beta), T diag(beta e^gc) complete

  // W^T = k^T (T diag(beta e^gc))^T: tiles (ib, tb), ib in {2w, 2w+1}: lane holds W[16 tb + c16][16 ib + 4 grp + e],
  // so the tile pair (2w, 2w+1) of one tb is W's A-operand block (tb, kb = w). T is lower triangular: the second
  // K block (chunk rows 32..63) only contributes to tb >= 2.
#pragma unroll
  for (int tb = 0; tb < 4; tb++) {
    f4 d[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int i = 16 * (2 * w + k) + c16;
      f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kb = 0; kb < 2; kb++) {
        if (kb == 1 && tb < 2) continue;
        const h8 av = *reinterpret_cast<const h8*>(sm.KT + kt16(i, 4 * kb + grp));
        const h8 bv = *reinterpret_cast<const h8*>(sm.Tw + (16 * tb + c16) * kTP + 32 * kb + 8 * grp);
        acc = mfma16(av, bv, acc);
      }
      d[k] = acc;
    }
    img.st16(kOffW + (tb * 4 + w) * kBlk + lo16, join(d[0], d[1]));
  }
  // U = T diag(beta) v^: tiles (tb, jt), jt in {2w, 2w+1}, in the D layout
#pragma unroll
  for (int tb = 0; tb < 4; tb++) {
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int jt = 2 * w + k;
      f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kb = 0; kb < 2; kb++) {
        if (kb == 1 && tb < 2) continue;
        const h8 av = *reinterpret_cast<const h8*>(sm.Tb + (16 * tb + c16) * kTP + 32 * kb + 8 * grp);
        const h8 bv = *reinterpret_cast<const h8*>(sm.VT + vt16(16 * jt + c16, 4 * kb + grp));
        acc = mfma16(av, bv, acc);
      }
      img.st8(kOffU + (tb * 8 + jt) * 512 + 8 * lane,
              h4{(_Float16)acc[0], (_Float16)acc[1], (_Float16)acc[2], (_Float16)acc[3]});
    }
  }
  // K~^T blocks (ib in {2w, 2w+1}, kb 0..1): k^ columns with chunk row t scaled by e^(gc_63 - gc_t)
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int i = 16 * (2 * w + k) + c16;
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
      const h8 kv = perm_a_kt(sm.KT, i, kb, grp);
      const f4 dlo = lds4(&sm.ed[32 * kb + 4 * grp]), dhi = lds4(&sm.ed[32 * kb + 16 + 4 * grp]);
      h8 o;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        o[e] = (_Float16)((float)kv[e] * dlo[e]);
        o[4 + e] = (_Float16)((float)kv[4 + e] * dhi[e]);
      }
      img.st16(kOffK + ((2 * w + k) * 2 + kb) * kBlk + lo16, o);
    }
  }
  if (tid0 == 0) img.st4(kOffS, sm.eg[kCH - 1]);
}

// ------------------------------------------------------------------------------------------------------------------
constexpr int kCW = 4, kCT = 64 * kCW;  // output pass: 4 waves, wave w on value columns 32 w .. + 31

__device__ __forceinline__ h8 lds16(const unsigned char* p) { return *reinterpret_cast<const h8*>(p); }

// sum of x over the four lanes c16, c16 + 16, c16 + 32, c16 + 48 (v_permlane16_swap pairs rows 2r and 2r + 1,
// v_permlane32_swap the two halves); every lane gets the same bits
__device__ __forceinline__ float sum_col4(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, x), false, false);
  x = __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
  const auto q = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, x), false, false);
  return __builtin_bit_cast(float, (unsigned)q[0]) + __builtin_bit_cast(float, (unsigned)q[1]);
}

// The sequential part is the state pass alone: per chunk four K blocks of MFMA products per wave, spread over four
// CUs per (sequence, head). The output work runs on every other CU in the same launch (gdn_scan_kernel), each chunk
// as soon as the state pass has published the packed state at its start.
//
// Publication: the state pass stores the packed states with device-coherent (sc1) stores; its period-end wait, which
// counts in issue order, proves a period's stores complete kStBufs - 2 periods later, and the workgroup then stores
// its progress counter (epoch << kDuoEpochShift | chunks published) with a device-scope atomic store. An output
// workgroup waits for the four counters of its (sequence, head) and reads the packed state with sc1 loads. State
// workgroups come first in the grid, so the dispatcher places every one of them before any output workgroup of its
// XCD: an output workgroup only ever waits for state workgroups that are resident or done, and every wait is bounded.
__device__ __forceinline__ unsigned ld_counter(const unsigned* c) {
  return __hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_counter(unsigned* c, unsigned v) {
  __hip_atomic_store(c, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
constexpr int kCacheSc1 = 16;  // cache-policy operand of buffer and LDS-DMA instructions: device-coherent (sc1)

// The state pass: kSG workgroups per (sequence, head), workgroup g on value columns 32 g .. + 31, its two waves on
// 16 columns each (wave v: columns 32 g + 16 v + c16), so that a head's products spread over kSG CUs; each wave
// reads the whole of W and K~^T every chunk, which with more waves per CU would make LDS reads the bound. Each chunk's
// W and K~^T (image blocks 16..47), the workgroup's 32 columns of U (one 1 KiB block per row block) and e^(gc_63),
// plus one block of padding so that both waves issue the same number of DMA instructions, arrive in one of four LDS
// buffers three chunks ahead.
constexpr int kSG = 4, kSV = 2, kSVT = 64 * kSV;
constexpr int kStBlocks = 38;
constexpr int kStBufs = 4;
constexpr int kStDma = kStBlocks / kSV;  // DMA instructions per wave per chunk
constexpr int kStW = 0, kStK = 16 * kBlk, kStU = 32 * kBlk, kStS = 36 * kBlk;  // LDS offsets in a buffer
static_assert(kStBlocks % kSV == 0 && kOffS / kBlk + 1 < kChunkScratch / kBlk, "state-pass DMA blocks");
// Vector memory instructions a wave issues after the DMA of chunk p + 1 (issued kStBufs - 1 periods before the end of
// period p) up to that end: the four stores of the packed state of its own period, then kStBufs - 2 periods of a DMA
// and four stores. s_waitcnt with that vmcnt and lgkmcnt 0 (expcnt not waited for) covers that DMA and this wave's
// LDS reads.
constexpr int kStAfter = 4 + (kStBufs - 2) * (kStDma + 4);
constexpr int kStWait = (kStAfter & 15) | ((kStAfter >> 4) << 14) | (7 << 4);

struct StateLds {
  unsigned char buf[kStBufs][kStBlocks * kBlk];  // chunk p in buf[p % kStBufs]
};

template <typename T>
__device__ __forceinline__ void state_pass(const GdnArgs& a, unsigned char* lds_raw, int g, int bh) {
  StateLds& sm = *reinterpret_cast<StateLds*>(lds_raw);
  const int b = bh / a.H, h = bh % a.H;
  const int tid0 = threadIdx.x, v = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  unsigned* const progress = a.sync_flags + (size_t)bh * 64 + 16 * g;
  const unsigned ep = a.sync_epoch << kDuoEpochShift;
  const int end = a.P + a.L;
  const int nchunks = (a.L + (a.P - a.s0) + kCH - 1) / kCH;
  char* const imgs = (char*)a.img + (size_t)bh * a.img_chunks * kChunkScratch;
  const size_t sbase = ((size_t)b * a.H + h) * kDK * kDV;
  const int col0 = 32 * g + 16 * v;  // this wave's first value column

  // chunk q's blocks into buf[d]: DMA instructions v, v + 2, ... (16 bytes per lane, whole 1 KiB blocks)
  auto issue = [&](int q, int d) {
    const char* src = imgs + (size_t)q * kChunkScratch;
    unsigned char* dst = sm.buf[d];
    const int ln = opaque(tid0) & 63;
#pragma unroll
    for (int k = 0; k < kStDma; k++) {
      const int i = v + kSV * k;
      const int sb = i < 32 ? kOffW / kBlk + i : i < 36 ? kOffU / kBlk + 4 * (i - 32) + g : kOffS / kBlk + (i - 36);
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + kBlk * (size_t)sb + 16 * ln),
                                       (__attribute__((address_space(3))) void*)(dst + kBlk * i), 16, 0, 0);
    }
  };

  const int lane0 = tid0 & 63, grp0 = lane0 >> 4, c160 = lane0 & 15;
  f4 S[8];
#pragma unroll
  for (int ib = 0; ib < 8; ib++)
#pragma unroll
    for (int e = 0; e < 4; e++)
      S[ib][e] = a.S_in ? gp<float>(a.S_in)[sbase + (size_t)(16 * ib + 4 * grp0 + e) * kDV + col0 + c160] : 0.0f;
#pragma unroll
  for (int q = 0; q < kStBufs - 1; q++) issue(min(q, nchunks - 1), q);
  __builtin_amdgcn_s_waitcnt(0);  // the prologue's loads drained (else every period's first use would wait for them)
  __syncthreads();
  // W of the period's chunk, read during the previous period (the first from the prologue)
  h8 wa[4][4];
  auto read_w = [&](int q) {
    const unsigned char* im = sm.buf[q % kStBufs];
    const int lo16 = 16 * (opaque(tid0) & 63);
#pragma unroll
    for (int kb = 0; kb < 4; kb++)
#pragma unroll
      for (int tb = 0; tb < 4; tb++) wa[kb][tb] = lds16(im + kStW + (tb * 4 + kb) * kBlk + lo16);
  };
  read_w(0);

  // Period p: the DMA of chunk p + kStBufs - 1; the packed state and its snapshot; K~^T of chunk p into registers
  // while X = W S runs; the wait for chunk p + 1 and the barrier; W of chunk p + 1 into registers while V_new and the
  // state update run. Every LDS read of a period's chunk thus has a stretch of MFMA work to land behind.
  for (int p = 0; p < nchunks; p++) {
    const int c0 = a.s0 + kCH * p;
    const bool full = end - c0 >= kCH;
    const int tid = opaque(tid0), lane = tid & 63;
    const int lo16 = 16 * lane;
    // every period (the last chunk again past the end, into a buffer nobody reads): the wait below counts a fixed
    // number of instructions
    issue(min(p + kStBufs - 1, nchunks - 1), (p + kStBufs - 1) % kStBufs);
    const unsigned char* im = sm.buf[p % kStBufs];
    h8 Sb[4];
#pragma unroll
    for (int kb = 0; kb < 4; kb++) Sb[kb] = pack_b(S[2 * kb], S[2 * kb + 1]);
    {
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc(imgs + (size_t)p * kChunkScratch + kOffSnap, 0, kSnap, 0x00020000);
#pragma unroll
      for (int kb = 0; kb < 4; kb++)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i4v, Sb[kb]), rs, (((g * 4 + kb) * 2 + v) * 64 + lane) * 16,
                                               0, kCacheSc1);
    }
    h8 kt[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int ib = 0; ib < 8; ib++) kt[kb][ib] = lds16(im + kStK + (ib * 2 + kb) * kBlk + lo16);
    f4 X[4];
    const f4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < 4; kb++)
#pragma unroll
      for (int tb = 0; tb < 4; tb++) X[tb] = mfma16(wa[kb][tb], Sb[kb], kb ? X[tb] : z4);
    h4 u[4];
#pragma unroll
    for (int tb = 0; tb < 4; tb++) u[tb] = *reinterpret_cast<const h4*>(im + kStU + tb * kBlk + v * 512 + 8 * lane);
    const float eL = *reinterpret_cast<const float*>(im + kStS);
    // This wave's part of chunk p + 1 has landed and its reads of chunk p are done; after the barrier both waves'
    // parts have, and no wave reads chunk p's buffer again before the next period's DMA into it. A bare s_barrier:
    // __syncthreads() would also wait for the DMAs just issued for later chunks (a workgroup-scope fence waits for every
    // LDS DMA in flight). The empty asm statements keep the compiler from moving memory accesses across it.
    __builtin_amdgcn_s_waitcnt(kStWait);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // the wait also covered both waves' packed-state stores of periods up to p - (kStBufs - 1)
    if (tid0 == 0 && p >= kStBufs - 1) st_counter(progress, ep + (unsigned)(p - (kStBufs - 2)));
    // every period (a conditional read would make wa a merge that waits at once), issued here: the empty asm keeps
    // the compiler from sinking the reads below the state update
    read_w(min(p + 1, nchunks - 1));
    asm volatile("" ::: "memory");
    if (full) {
      h8 Vb[2];
      {
        f4 Vn[4];
#pragma unroll
        for (int tb = 0; tb < 4; tb++) Vn[tb] = f4{(float)u[tb][0], (float)u[tb][1], (float)u[tb][2], (float)u[tb][3]} - X[tb];
#pragma unroll
        for (int kb = 0; kb < 2; kb++) Vb[kb] = pack_b(Vn[2 * kb], Vn[2 * kb + 1]);
      }
#pragma unroll
      for (int ib = 0; ib < 8; ib++) S[ib] = mfma16(kt[0][ib], Vb[0], S[ib] * eL);
#pragma unroll
      for (int ib = 0; ib < 8; ib++) S[ib] = mfma16(kt[1][ib], Vb[1], S[ib]);
    }
  }
  // every packed state stored: publish them all
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  if (tid0 == 0) st_counter(progress, ep + (unsigned)nchunks);
#pragma unroll
  for (int ib = 0; ib < 8; ib++)
#pragma unroll
    for (int e = 0; e < 4; e++)
      gpw<float>(a.S_out)[sbase + (size_t)(16 * ib + 4 * grp0 + e) * kDV + col0 + c160] = S[ib][e];
}

// The output pass: one 4-wave workgroup per (chunk, sequence, head), wave w on value columns 32 w .. + 31: the chunk's
// image in LDS and the packed state at its start from the state pass; X = W S and the first half of o^T = S^T q~^T
// from the packed state, V_new = U - X, o^T += V_new^T Att^T, the gated norm and the stores. o is computed transposed
// (the packed state and V_new serve as A operands with the same permuted K order in which they serve as B operands,
// and the image blocks of q~ and Att as B operands), so a lane holds 4 consecutive value columns of one row: the gate
// factors arrive and the outputs leave as 16-byte accesses. The state pass computes X from the same operands in the
// same order, so V_new here is bit for bit the one the state update used.
struct OutLds {
  unsigned char img[kImg];
  float red[kCH * kCW];  // gated-norm partial sums, [t][wave]
};

template <typename T>
__device__ __forceinline__ void out_pass(const GdnArgs& a, unsigned char* lds_raw, int p, int bh) {
  OutLds& sm = *reinterpret_cast<OutLds*>(lds_raw);
  const int b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, grp = lane >> 4, c16 = lane & 15, lo16 = 16 * lane;
  const int end = a.P + a.L;
  const int c0 = a.s0 + kCH * p;
  const int m = min(kCH, end - c0);
  const char* const src = (const char*)a.img + ((size_t)bh * a.img_chunks + p) * kChunkScratch;
  for (int i = w; i < kImg / kBlk; i += kCW)
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + kBlk * (size_t)i + 16 * lane),
                                     (__attribute__((address_space(3))) void*)(sm.img + kBlk * i), 16, 0, 0);
  // z at this lane's (transposed) output positions, row 16 tb + c16 (rows outside [P, P + L) clamped: their outputs
  // are never stored), columns 32 w + 16 jj + 4 grp .. + 3; the gate factors gnorm_w SiLU(z) are formed at their use
  f4 zq[4][2], gw[2];
  if (a.gnorm) {
    gw[0] = ld4(gp<float>(a.gnorm) + 32 * w + 4 * grp);
    gw[1] = ld4(gp<float>(a.gnorm) + 32 * w + 16 + 4 * grp);
    const gptr<T> zb = gp<T>((const char*)a.in + (size_t)b * a.L * ((unsigned)a.stride * sizeof(T))) + a.C + h * kDV + 32 * w + 4 * grp;
#pragma unroll
    for (int tb = 0; tb < 4; tb++) {
      const int rr = min(max(c0 + 16 * tb + c16 - a.P, 0), a.L - 1);
#pragma unroll
      for (int jj = 0; jj < 2; jj++) zq[tb][jj] = ld4(zb + (size_t)rr * a.stride + 16 * jj);
    }
  }
  // the packed state at the chunk's start, once the four state workgroups of this (sequence, head) have published it
  // (a bounded number of polls of about a microsecond: they are resident or done, so the wait ends; one that runs out
  // is reported through the engine's error word)
  if (tid == 0) {
    const unsigned want = (a.sync_epoch << kDuoEpochShift) + a.wait.skew + (unsigned)(p + 1);
    const unsigned* progress = a.sync_flags + (size_t)bh * 64;
    bool late = false;
    for (int g = 0; g < kSG; g++) {
      int i = 0;
      for (; i < a.wait.polls && ld_counter(progress + 16 * g) < want; i++) __builtin_amdgcn_s_sleep(2);
      late |= i == a.wait.polls;
    }
    if (late) report_wait(a.wait, kErrSplitWait);
  }
  __syncthreads();
  h8 Sb[4][2];
  {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(src) + kOffSnap, 0, kSnap, 0x00020000);
#pragma unroll
    for (int kb = 0; kb < 4; kb++)
#pragma unroll
      for (int jj = 0; jj < 2; jj++)
        Sb[kb][jj] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rs, (((w * 4 + kb) * 2 + jj) * 64 + lane) * 16, 0, kCacheSc1));
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const unsigned char* im = sm.img;

  f4 X[4][2], O[2][4];
  const f4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int kb = 0; kb < 4; kb++) {
    h8 wa[4];
#pragma unroll
    for (int tb = 0; tb < 4; tb++) wa[tb] = lds16(im + kOffW + (tb * 4 + kb) * kBlk + lo16);
#pragma unroll
    for (int tb = 0; tb < 4; tb++)
#pragma unroll
      for (int jj = 0; jj < 2; jj++) X[tb][jj] = mfma16(wa[tb], Sb[kb][jj], kb ? X[tb][jj] : z4);
  }
#pragma unroll
  for (int kb = 0; kb < 4; kb++) {
    h8 qa[4];
#pragma unroll
    for (int tb = 0; tb < 4; tb++) qa[tb] = lds16(im + kOffQ + (tb * 4 + kb) * kBlk + lo16);
#pragma unroll
    for (int jj = 0; jj < 2; jj++)
#pragma unroll
      for (int tb = 0; tb < 4; tb++) O[jj][tb] = mfma16(Sb[kb][jj], qa[tb], kb ? O[jj][tb] : z4);
  }
  h8 Vb[2][2];
  {
    f4 Vn[4][2];
#pragma unroll
    for (int tb = 0; tb < 4; tb++)
#pragma unroll
      for (int jj = 0; jj < 2; jj++) {
        const h4 u = *reinterpret_cast<const h4*>(im + kOffU + (tb * 8 + 2 * w + jj) * 512 + 8 * lane);
        Vn[tb][jj] = f4{(float)u[0], (float)u[1], (float)u[2], (float)u[3]} - X[tb][jj];
      }
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int jj = 0; jj < 2; jj++) Vb[kb][jj] = pack_b(Vn[2 * kb][jj], Vn[2 * kb + 1][jj]);
  }
#pragma unroll
  for (int tb = 0; tb < 4; tb++) {
    const h8 a0 = lds16(im + kOffA + (tb * 2 + 0) * kBlk + lo16);
#pragma unroll
    for (int jj = 0; jj < 2; jj++) O[jj][tb] = mfma16(Vb[0][jj], a0, O[jj][tb]);
    if (tb >= 2) {
      const h8 a1 = lds16(im + kOffA + (tb * 2 + 1) * kBlk + lo16);
#pragma unroll
      for (int jj = 0; jj < 2; jj++) O[jj][tb] = mfma16(Vb[1][jj], a1, O[jj][tb]);
    }
  }
  if (a.gnorm) {
#pragma unroll
    for (int tb = 0; tb < 4; tb++) {
      float v = 0.0f;
#pragma unroll
      for (int jj = 0; jj < 2; jj++)
#pragma unroll
        for (int e = 0; e < 4; e++) v = fmaf(O[jj][tb][e], O[jj][tb][e], v);
      v = sum_col4(v);
      if (grp == tb) sm.red[(16 * tb + c16) * kCW + w] = v;
    }
    __syncthreads();
#pragma unroll
    for (int tb = 0; tb < 4; tb++) {
      const f4 r = lds4(&sm.red[(16 * tb + c16) * kCW]);
      const float iv = rsqrtf(((r[0] + r[1]) + (r[2] + r[3])) / kDV + 1e-6f);
#pragma unroll
      for (int jj = 0; jj < 2; jj++) {
        f4 g;
#pragma unroll
        for (int e = 0; e < 4; e++) g[e] = gw[jj][e] * silu(zq[tb][jj][e]);
        O[jj][tb] = O[jj][tb] * iv * g;
      }
    }
  }
  const int ostride = a.H * kDV;
  __attribute__((address_space(1))) T* ob = gpw<T>(a.out) + (size_t)b * a.L * ostride + (size_t)h * kDV + 32 * w + 4 * grp;
#pragma unroll
  for (int tb = 0; tb < 4; tb++) {
    const int t = 16 * tb + c16, r = c0 + t;
    if (t < m && r >= a.P) {
      __attribute__((address_space(1))) T* orow = ob + (size_t)(r - a.P) * ostride;
      store4(orow, O[0][tb]);
      store4(orow + 16, O[1][tb]);
    }
  }
}

// Block i < kSG * B * H: the state pass of (sequence, head) i / kSG, value columns 32 (i % kSG) ..; then one block per
// (chunk, sequence, head), chunk-major, for the outputs.
constexpr size_t kScanLds = sizeof(StateLds) > sizeof(OutLds) ? sizeof(StateLds) : sizeof(OutLds);
template <typename T>
__global__ __launch_bounds__(kCT) void gdn_scan_kernel(GdnArgs a) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds_raw[];
  const int bhn = a.B * a.H, nst = kSG * bhn, id = blockIdx.x;
  if (id < nst) {
    if (threadIdx.x >= kSVT) return;  // two waves (a barrier waits only for the waves still running)
    state_pass<T>(a, lds_raw, id % kSG, id / kSG);
  } else {
    out_pass<T>(a, lds_raw, (id - nst) / bhn, (id - nst) % bhn);
  }
}

template <typename T>
hipError_t launch(const GdnArgs& a, hipStream_t s) {
  const int nchunks = (a.L + (a.P - a.s0) + kCH - 1) / kCH;
  if (nchunks > a.img_chunks) return hipErrorInvalidValue;
  auto kp = gdn_prep_kernel<T>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kp), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)sizeof(PrepLds));
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kp, dim3(nchunks, a.B * a.H), dim3(kPT), sizeof(PrepLds), s, a);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  auto kc = gdn_scan_kernel<T>;
  e = hipFuncSetAttribute(reinterpret_cast<const void*>(kc), hipFuncAttributeMaxDynamicSharedMemorySize, (int)kScanLds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kc, dim3((kSG + nchunks) * a.B * a.H), dim3(kCT), kScanLds, s, a);
  return hipGetLastError();
}

}  // namespace

size_t gdn_split_image_bytes() { return (size_t)kChunkScratch; }

hipError_t launch_gdn_split(const GdnArgs& a, hipStream_t s) {
  if (a.DK != kDK || a.DV != kDV || a.KC != kKC || !a.img) return hipErrorInvalidValue;
  if (a.P - a.s0 >= kCH || a.P < a.s0) return hipErrorInvalidValue;  // at most one open chunk is replayed
  if (!a.sync_flags || a.sync_epoch == 0 || a.sync_epoch >= (1u << (32 - kDuoEpochShift))) return hipErrorInvalidValue;
  if ((a.L + (a.P - a.s0) + kCH - 1) / kCH + 1 >= (1 << kDuoEpochShift)) return hipErrorInvalidValue;
  return a.dtype == 0 ? launch<float>(a, s) : launch<_Float16>(a, s);
}

}  // namespace ha
