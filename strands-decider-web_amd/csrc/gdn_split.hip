// Chunked gated-delta prefill in two kernels, gfx950.
//
// Same semantics and chunk geometry as gdn_chunk.hip (the sequential rule of reference
// web/public/engine/wgsl.js:124-187 + 252-268 in the chunked WY/UT form, chunk 64, chunk boundaries at s0 + 64 k),
// split along the one dependency that is sequential: everything derived from a chunk's own rows (the q/k/v conv,
// l2 norms, gates, A = strictly_lower(beta k k^T decay) and T = (I + A)^-1) does not depend on the state, so
//   gdn_prep_kernel  runs one workgroup per (chunk, sequence, head), all chunks at once over the whole chip, and
//                    writes each chunk's "image" (q^, k^, T diag(beta), v^T in f16 and the gate vectors) to a
//                    scratch buffer, in the exact layout the recurrence keeps in LDS;
//   gdn_recur_kernel runs one workgroup per (sequence, head) through the chunks in order, holding the fp32 state in
//                    MFMA accumulators (8 waves x 16 value columns). Per chunk it DMAs the next image into LDS while
//                    it does the state work of the current one, and builds k^T and the decay-masked scores q^ k^T
//                    itself (cheap, and their images would cost more HBM traffic than they save). V_new is formed as
//                    T diag(beta) (v - diag(e^gc) k^ S), one product instead of two.
// The state-independent work is then off the per-chunk critical path, which is what bounds the fused kernel when
// there are fewer (sequence, head) pairs than CUs (B = 1: 16 of 256 CUs).
//
// Both kernels share the fused kernel's helpers and MFMA operand conventions (gdn_common.h); the per-column state
// arithmetic follows the fused kernel's except for the V_new bracket, and the gated norm's row sums are formed in
// a different order (16-column partials).
#include <stddef.h>

#include "gdn_common.h"

namespace ha {
namespace {

// One chunk's image. Member order and padding match the recurrence kernel's LDS copy byte for byte.
struct Img {
  _Float16 Qs[kCH * kQP];  // q^ / sqrt(DK), [t][i]
  _Float16 Ks[kCH * kQP];  // k^, [t][i]
  _Float16 Tb[kCH * kTP];  // T diag(beta), [t][t'] (blocks above the diagonal zero)
  _Float16 VT[kDV * kTP];  // v^ = SiLU(conv(v)) transposed, [j][t], 8-row groups swizzled by vt16
  float eg[kCH];           // e^gc
  float ed[kCH];           // e^(gc_63 - gc)
  float gc[kCH];           // cumulative log decay inside the chunk
  float rowf[kCH];         // e^(gc_t - gc_16(t/16)), in (0, 1]
  float colf[3][kCH];      // colf[i-1][t'] = e^(gc_16i - gc_t') for t' < 16 i, in (0, 1]
};
static_assert(sizeof(Img) % 16 == 0, "image is copied in 16-byte words");
constexpr int kImg = (int)((sizeof(Img) + 1023) / 1024 * 1024);  // image size: whole 1 KiB DMA instructions
// Per chunk, the image is followed by the gated norm's gate factors gnorm_w[j] * SiLU(z[t][j]) in fp32, [j][t]:
// the recurrence reads them straight into the D layout of its output rows (4 consecutive rows per load).
constexpr int kGate = (int)sizeof(float) * kDV * kCH;
constexpr int kChunkScratch = kImg + kGate;

// ------------------------------------------------------------------------------------------------------------------
// gdn_prep_kernel: 4 waves. Conv lane pt: rows 8 (pt / 32) .. + 7 of the chunk, channels 4 (pt % 32) .. + 3 of each
// of q, k and v. q^ and v^ go straight from registers to the image; k^ (the operand of A = k^ k^T) and T diag(beta)
// are built in LDS and copied out with the gate vectors. Wave 3 also forms the gates, the diagonal blocks of A and
// their forward substitution; waves 0..2 the six below-diagonal blocks of A and then one block column of T each.
constexpr int kPW = 4, kPT = 64 * kPW;
constexpr int kPRG = 8;  // rows per conv lane
constexpr int kPG = kPW - 1;

struct PrepLds {
  _Float16 Ks[kCH * kQP];
  _Float16 Tb[kCH * kTP];
  float eg[kCH], ed[kCH], gc[kCH], rowf[kCH], colf[3][kCH];  // as in Img, in the same order
  float Tm[kCH * kAP];     // A, then T (fp32)
  float cw[12][32][kKC];   // conv taps: channel 4 g + c of q (c < 4), k (4 <= c < 8), v (c >= 8) at cw[c][g]
  float bt[kCH];           // beta
  float brow[kCH];         // beta_t rowf_t
};
static_assert(offsetof(PrepLds, colf) + sizeof(float) * 3 * kCH - offsetof(PrepLds, eg) ==
                  offsetof(Img, colf) + sizeof(float) * 3 * kCH - offsetof(Img, eg),
              "gate vectors are copied as one block");

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
  char* const dst = (char*)a.img + ((size_t)bh * a.img_chunks + c) * kChunkScratch;

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
  // blocks above the diagonal of T diag(beta) are read by full 32-wide K blocks and never written otherwise:
  // row block rb (< 3) has 6 - 2 rb such 8-column groups per row, from column 16 (rb + 1)
  if (tid0 < 192) {
    const int k = tid0, rb = k < 96 ? 0 : k < 160 ? 1 : 2, k2 = k - (rb == 0 ? 0 : rb == 1 ? 96 : 160);
    const int ng = 6 - 2 * rb, t = 16 * rb + k2 / ng, g = k2 % ng + 2 * (rb + 1);
    *reinterpret_cast<h8*>(sm.Tb + t * kTP + 8 * g) = h8{};
  }
  __syncthreads();  // conv taps visible

  // conv + SiLU; q and k rows l2-normalised (q also scaled by 1/sqrt(DK); a row's 128 channels of q, of k, sit in
  // the 32 lanes of a half wave): q^ to the image, k^ to LDS; v^ columns (8 rows each) to the image's v^T
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
#pragma unroll
    for (int r = 0; r < kPRG; r++) {
      float sq = row_sum16(ssq[r]), sk = row_sum16(ssk[r]);
      sq += __shfl_xor(sq, 16);
      sk += __shfl_xor(sk, 16);
      const float rq = rsqrtf(sq + 1e-6f) * qscale, rk = rsqrtf(sk + 1e-6f);
      const int t = kPRG * rg + r;
      *(__attribute__((address_space(1))) h4*)(dst + offsetof(Img, Qs) + 2 * (size_t)(t * kQP + 4 * cl)) =
          h4{(_Float16)(u[r][0] * rq), (_Float16)(u[r][1] * rq), (_Float16)(u[r][2] * rq), (_Float16)(u[r][3] * rq)};
      *reinterpret_cast<h4*>(sm.Ks + t * kQP + 4 * cl) =
          h4{(_Float16)(u[r][4] * rk), (_Float16)(u[r][5] * rk), (_Float16)(u[r][6] * rk), (_Float16)(u[r][7] * rk)};
    }
#pragma unroll
    for (int cc = 0; cc < 4; cc++) {
      h8 vt;
#pragma unroll
      for (int r = 0; r < kPRG; r++) vt[r] = (_Float16)u[r][8 + cc];
      *(__attribute__((address_space(1))) h8*)(dst + offsetof(Img, VT) + 2 * (size_t)vt16(4 * cl + cc, rg)) = vt;
    }
  }
  // z of rows 8 rg .. + 7 (this lane's 4 channels) for the gate factors, in flight behind the work below; rows
  // outside [P, P + L) are clamped (their outputs are never stored)
  float zr[kPRG][4];
  if (a.gnorm) {
#pragma unroll
    for (int r = 0; r < kPRG; r++) {
      const int rr = min(max(cs + kPRG * rg + r - a.P, 0), a.L - 1);
      load4(gp<T>(seq_in) + (size_t)rr * a.stride + a.C + h * kDV + 4 * cl, zr[r]);
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
  __syncthreads();

  const int lane = tid0 & 63, grp = lane >> 4, c16 = lane & 15;
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
    wave_sync();
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
    const float cb = sm.bt[base + c16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      sm.Tm[(base + r) * kAP + base + c16] = pc[r];
      sm.Tb[(base + r) * kTP + base + c16] = (_Float16)(pc[r] * cb);
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
  __syncthreads();
  if (w == 0)
    t_column<0, false>(sm, grp, c16);
  else if (w == 1)
    t_column<1, false>(sm, grp, c16);
  else if (w == 2)
    t_column<2, false>(sm, grp, c16);
  __syncthreads();

  if (a.gnorm) {
    const f4 gw = ld4(gp<float>(a.gnorm) + 4 * cl);
#pragma unroll
    for (int cc = 0; cc < 4; cc++) {
      float* g = (float*)(dst + kImg) + (size_t)(4 * cl + cc) * kCH + kPRG * rg;
      f4 lo, hi;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        lo[r] = gw[cc] * silu(zr[r][cc]);
        hi[r] = gw[cc] * silu(zr[r + 4][cc]);
      }
      store4(gpw<float>(g), lo);
      store4(gpw<float>(g + 4), hi);
    }
  }
  // k^, T diag(beta) and the gate vectors out, 16 bytes per lane per step
  auto copy_out = [&](size_t img_off, const void* from, int bytes) {
    for (int i = tid0; i < bytes / 16; i += kPT)
      *(__attribute__((address_space(1))) f4*)(dst + img_off + 16 * (size_t)i) =
          *reinterpret_cast<const f4*>((const char*)from + 16 * i);
  };
  copy_out(offsetof(Img, Ks), sm.Ks, (int)sizeof(sm.Ks));
  copy_out(offsetof(Img, Tb), sm.Tb, (int)sizeof(sm.Tb));
  copy_out(offsetof(Img, eg), sm.eg, (int)(sizeof(Img) - offsetof(Img, eg)));
}

// ------------------------------------------------------------------------------------------------------------------
// gdn_recur_kernel: 8 waves; wave w owns value columns 16 w .. 16 w + 15 of the fp32 state (MFMA D layout:
// S[it][e] = S[16 it + 4 grp + e][16 w + c16]) and all of every chunk's work for them. Per period p, two segments:
//   A: chunk p's state work (k^ S, V_new, q^ S, o, the state update, the gated-norm row partials); the DMA of image
//      p+1 into the other image buffer is issued at its start
//   B: chunk p's gated norm and output store; k^T and the masked scores of chunk p+1; z of p+1
constexpr int kRW = 8, kRT = 64 * kRW;

// One halving step of a transposed 16-lane reduction over v[0 .. 2N): a lane whose selection bit is clear keeps the
// low half v[0 .. N), otherwise the high half, adds the partner's copy (DPP control CTRL) and leaves it in v[0 .. N).
template <int N, int CTRL>
__device__ __forceinline__ void halve(float* v, int hi) {
#pragma unroll
  for (int i = 0; i < N; i++) {
    const float keep = hi ? v[N + i] : v[i], send = hi ? v[i] : v[N + i];
    v[i] = keep + DPP_F(send, CTRL);
  }
}

struct RecLds {
  unsigned char img[2][kImg];  // chunk images; chunk p in img[p & 1]
  _Float16 KT[kDK * kTP];      // k^ transposed, [i][t], 8-column groups swizzled by kt16
  _Float16 Att[kCH * kTP];     // decay-masked causal q^ k^T, [t][t']
  float red[kCH * kRW];        // gated-norm partial sums, [t][wave]
  float inv[kRW][kCH];         // per wave: 1 / rms of each row
};

template <typename T>
__global__ __launch_bounds__(kRT) void gdn_recur_kernel(GdnArgs a) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds_raw[];
  RecLds& sm = *reinterpret_cast<RecLds*>(lds_raw);
  const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
  const int tid0 = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  const int end = a.P + a.L;
  const int nchunks = (a.L + (a.P - a.s0) + kCH - 1) / kCH;
  const unsigned rowb = (unsigned)a.stride * sizeof(T);
  const unsigned orowb = (unsigned)(a.H * kDV) * sizeof(T);
  const char* const seq_in = (const char*)a.in + (size_t)b * a.L * rowb;
  const char* const imgs = (const char*)a.img + (size_t)bh * a.img_chunks * kChunkScratch;
  const size_t sbase = ((size_t)b * a.H + h) * kDK * kDV;

  for (int idx = tid0; idx < kCH * kCH; idx += kRT) {
    const int t = idx >> 6, tp = idx & 63;
    if ((tp >> 4) > (t >> 4)) sm.Att[t * kTP + tp] = (_Float16)0.0f;
  }

  // this wave's share of one chunk image: 1 KiB DMA instructions w, w + 8, ...
  auto issue_img = [&](int p) {
    const char* src = imgs + (size_t)p * kChunkScratch;
    unsigned char* dst = sm.img[p & 1];
    const int ln = opaque(tid0) & 63;
    for (int i = w; i < kImg / 1024; i += kRW)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + 1024 * (size_t)i + 16 * ln),
                                       (__attribute__((address_space(3))) void*)(dst + 1024 * i), 16, 0, 0);
  };
  // gate factors of chunk q in the MFMA D layout of this lane's output: rows 16 ti + 4 grp .. +3, column 16 w + c16
  f4 zq[4];
  auto fetch_z = [&](int q) {
    const int lane = opaque(tid0) & 63, grp = lane >> 4, c16 = lane & 15;
    gptr<float> g = gp<float>(imgs + (size_t)q * kChunkScratch + kImg) + (size_t)(16 * w + c16) * kCH + 4 * grp;
#pragma unroll
    for (int ti = 0; ti < 4; ti++) zq[ti] = ld4(g + 16 * ti);
  };

  f4 S[8];
  {
    const int g0 = (tid0 & 63) >> 4, l16 = tid0 & 15;
#pragma unroll
    for (int it = 0; it < 8; it++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        S[it][e] = a.S_in ? gp<float>(a.S_in)[sbase + (size_t)(16 * it + 4 * g0 + e) * kDV + 16 * w + l16] : 0.0f;
  }
  // Drain these loads here: the compiler's wait counting merges the loop's entry state into every iteration, so a
  // state load still outstanding at the loop head would make each period's first use of S wait for the image DMA
  // issued just before it.
  __builtin_amdgcn_s_waitcnt(0);

  // chunk q's k^T and decay-masked scores (image q in LDS)
  auto prep_chunk = [&](int q) {
    const int tid = opaque(tid0), lane = tid & 63, grp = lane >> 4, c16 = lane & 15;
    const Img& nx = *reinterpret_cast<const Img*>(sm.img[q & 1]);
    // k^T from k^: items (channel i, 8-row group g8), two per lane
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int item = tid + kRT * k, i = item & 127, g8 = item >> 7;
      h8 v;
#pragma unroll
      for (int r = 0; r < 8; r++) v[r] = nx.Ks[(8 * g8 + r) * kQP + i];
      *reinterpret_cast<h8*>(sm.KT + kt16(i, g8)) = v;
    }
    // decay-masked causal scores q^ k^T: tiles w and, for waves 0 and 1, w + 8 of the 10 on or below the diagonal
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int jt = w + 8 * k;
      if (jt < 10) {
        const int ti = jt >= 6 ? 3 : jt >= 3 ? 2 : jt >= 1 ? 1 : 0, tj = jt - ti * (ti + 1) / 2;
        const _Float16* ab = nx.Qs + (16 * ti + c16) * kQP + 8 * grp;
        const _Float16* bb = nx.Ks + (16 * tj + c16) * kQP + 8 * grp;
        f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < 4; ks++)
          acc = mfma16(*reinterpret_cast<const h8*>(ab + 32 * ks), *reinterpret_cast<const h8*>(bb + 32 * ks), acc);
        const int tp = 16 * tj + c16, t0 = 16 * ti + 4 * grp;
        if (ti != tj) {
          const float cf = nx.colf[ti - 1][tp];
          const f4 rf = lds4(&nx.rowf[t0]);
#pragma unroll
          for (int e = 0; e < 4; e++) sm.Att[(t0 + e) * kTP + tp] = (_Float16)(acc[e] * rf[e] * cf);
        } else {
          const float gp_ = nx.gc[tp];
          const f4 gt = lds4(&nx.gc[t0]);
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int t = t0 + e;
            const float dec = __expf(fminf(gt[e] - gp_, 0.0f));
            sm.Att[t * kTP + tp] = (_Float16)(tp <= t ? acc[e] * dec : 0.0f);
          }
        }
      }
    }
  };

  // prologue: chunk 0's image, then its k^T and scores. The loop is entered with only z loads in flight, which
  // nothing in segment A overwrites, so no wait in A depends on the DMA issued at its start.
  issue_img(0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  prep_chunk(0);
  if (a.gnorm) fetch_z(0);
  __syncthreads();
  for (int p = 0; p < nchunks; p++) {
    const int c0 = a.s0 + kCH * p;
    f4 O[4];
    const int m = min(kCH, end - c0);
    const bool full = m == kCH;
    const int tid = opaque(tid0), lane = tid & 63, grp = lane >> 4, c16 = lane & 15;
    const int col = 16 * w + c16;

    // ---- A: chunk p ----
    {
      // The MFMA work runs in groups; the LDS operands of each group are read while the previous group's MFMAs
      // issue. An empty asm that takes a group's B operand and clobbers memory sits after the next group's reads,
      // so those reads are issued before the group's MFMAs without waiting for them, and a scheduling barrier
      // after the MFMAs keeps the reads of the group after next from being hoisted above them.
      if (p + 1 < nchunks) issue_img(p + 1);
      const Img& im = *reinterpret_cast<const Img*>(sm.img[p & 1]);
      // k^ S and q^ S, one 32-wide K block of the state per group, 8 accumulator chains
      h8 Aq[2][8];
      auto read_kq = [&](h8* A, int kb) {
#pragma unroll
        for (int ti = 0; ti < 4; ti++) {
          A[ti] = perm_a(im.Ks, kQP, 16 * ti + c16, kb, grp);
          A[4 + ti] = perm_a(im.Qs, kQP, 16 * ti + c16, kb, grp);
        }
      };
      read_kq(Aq[0], 0);
      f4 KS[4];
      h8 tb[4][2];
      h4 vlo[2], vhi[2];
      f4 eg4[4];
#pragma unroll
      for (int kb = 0; kb < 4; kb++) {
        if (kb < 3) {
          read_kq(Aq[(kb + 1) & 1], kb + 1);
        } else {
          // V_new operands: rows of T diag(beta) in the permuted K order, this column's v^ rows in the same order
          // (rows 32 k2 + 4 grp .. +3 and 32 k2 + 16 + 4 grp .. +3), e^gc of this lane's D-layout rows
#pragma unroll
          for (int ti = 0; ti < 4; ti++) {
#pragma unroll
            for (int k2 = 0; k2 <= (ti >> 1); k2++) tb[ti][k2] = perm_a(im.Tb, kTP, 16 * ti + c16, k2, grp);
            eg4[ti] = lds4(&im.eg[16 * ti + 4 * grp]);
          }
#pragma unroll
          for (int k2 = 0; k2 < 2; k2++) {
            vlo[k2] = *reinterpret_cast<const h4*>(im.VT + vt16(col, 4 * k2 + (grp >> 1)) + 4 * (grp & 1));
            vhi[k2] = *reinterpret_cast<const h4*>(im.VT + vt16(col, 4 * k2 + 2 + (grp >> 1)) + 4 * (grp & 1));
          }
        }
        h8 S16 = pack_b(S[2 * kb], S[2 * kb + 1]);
        asm volatile("" : "+v"(S16)::"memory");
#pragma unroll
        for (int ti = 0; ti < 4; ti++) {
          const f4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};
          KS[ti] = mfma16(Aq[kb & 1][ti], S16, kb ? KS[ti] : z4);
          O[ti] = mfma16(Aq[kb & 1][4 + ti], S16, kb ? O[ti] : z4);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // V_new = T diag(beta) (v - diag(e^gc) k^ S): the bracket is formed in fp32 in the D layout of k^ S and
      // rounded once to f16 as the B operand
      h8 Bv[2];
#pragma unroll
      for (int k2 = 0; k2 < 2; k2++) {
        const f4 lo = f4{(float)vlo[k2][0], (float)vlo[k2][1], (float)vlo[k2][2], (float)vlo[k2][3]} - eg4[2 * k2] * KS[2 * k2];
        const f4 hi = f4{(float)vhi[k2][0], (float)vhi[k2][1], (float)vhi[k2][2], (float)vhi[k2][3]} - eg4[2 * k2 + 1] * KS[2 * k2 + 1];
        Bv[k2] = pack_b(lo, hi);
      }
      f4 Vn[4];
#pragma unroll
      for (int ti = 0; ti < 4; ti++) {
        f4 u = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k2 = 0; k2 <= (ti >> 1); k2++) u = mfma16(tb[ti][k2], Bv[k2], u);
        Vn[ti] = u;
      }
      __builtin_amdgcn_sched_barrier(0);
      // o = e^gc (q^ S) + scores V_new
      {
        h8 att[4][2];
#pragma unroll
        for (int ti = 0; ti < 4; ti++) {
          att[ti][0] = perm_a(sm.Att, kTP, 16 * ti + c16, 0, grp);
          if (ti >= 2) att[ti][1] = perm_a(sm.Att, kTP, 16 * ti + c16, 1, grp);
        }
        const h8 Vb0 = pack_b(Vn[0], Vn[1]), Vb1 = pack_b(Vn[2], Vn[3]);
#pragma unroll
        for (int ti = 0; ti < 4; ti++) {
          O[ti] = mfma16(att[ti][0], Vb0, O[ti] * eg4[ti]);
          if (ti >= 2) O[ti] = mfma16(att[ti][1], Vb1, O[ti]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (full) {
        // rows of V_new scaled by e^(gl - gc_t), then S <- e^gl S + k^T (scaled V_new), in two halves of the rows
        // of S; the second half's k^T operands are read behind the first half's MFMAs
        h8 kt[2][4][2];
        auto read_kt = [&](h8 (*K)[2], int half) {
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int it = 4 * half + i;
            K[i][0] = perm_a_kt(sm.KT, 16 * it + c16, 0, grp);
            K[i][1] = perm_a_kt(sm.KT, 16 * it + c16, 1, grp);
          }
        };
        read_kt(kt[0], 0);
#pragma unroll
        for (int ti = 0; ti < 4; ti++) Vn[ti] *= lds4(&im.ed[16 * ti + 4 * grp]);
        h8 Vd0 = pack_b(Vn[0], Vn[1]), Vd1 = pack_b(Vn[2], Vn[3]);
        const float el = im.eg[kCH - 1];
#pragma unroll
        for (int half = 0; half < 2; half++) {
          if (half == 0) read_kt(kt[1], 1);
          asm volatile("" : "+v"(Vd0), "+v"(Vd1)::"memory");
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int it = 4 * half + i;
            S[it] = mfma16(kt[half][i][1], Vd1, mfma16(kt[half][i][0], Vd0, S[it] * el));
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if (a.gnorm) {
        // This wave's 16-column partial of the sum of squares of each of its 16 rows, reduced over the 16 lanes of
        // a DPP row by halving: at each step a lane keeps the half of its values selected by one lane bit, adds the
        // partner lane's copy of that half, and passes on the other half. The partners are the row mirror (lane
        // 15 - i), the half-row mirror (7 - i), then i ^ 2 and i ^ 1; each keeps the bits already used for selection,
        // so partners always hold the same index set. Lane c16 ends with value index c16 = 4 ti + e.
        float v[16];
#pragma unroll
        for (int ti = 0; ti < 4; ti++)
#pragma unroll
          for (int e = 0; e < 4; e++) v[4 * ti + e] = O[ti][e] * O[ti][e];
        halve<8, 0x140>(v, c16 & 8);
        halve<4, 0x141>(v, c16 & 4);
        halve<2, 0x4E>(v, c16 & 2);
        halve<1, 0xB1>(v, c16 & 1);
        sm.red[(16 * (c16 >> 2) + 4 * grp + (c16 & 3)) * kRW + w] = v[0];
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's part of the next image has landed
    __syncthreads();                // B

    // ---- B: chunk p's gated norm and store; k^T, scores and v conv of chunk p+1; z of p+1 ----
    {
      float Y[4][4];
#pragma unroll
      for (int ti = 0; ti < 4; ti++)
#pragma unroll
        for (int e = 0; e < 4; e++) Y[ti][e] = O[ti][e];
      if (a.gnorm) {
        // lane t: row t's eight wave partials -> 1 / rms, through this wave's slot to the lanes that hold row t
        const f4 r0 = lds4(&sm.red[lane * kRW]), r1 = lds4(&sm.red[lane * kRW + 4]);
        sm.inv[w][lane] = rsqrtf((((r0[0] + r0[1]) + (r0[2] + r0[3])) + ((r1[0] + r1[1]) + (r1[2] + r1[3]))) / kDV + 1e-6f);
        wave_sync();
#pragma unroll
        for (int ti = 0; ti < 4; ti++) {
          const f4 iv = lds4(&sm.inv[w][16 * ti + 4 * grp]);
#pragma unroll
          for (int e = 0; e < 4; e++) Y[ti][e] = Y[ti][e] * iv[e] * zq[ti][e];
        }
      }
      __attribute__((address_space(1))) T* ob = gpw<T>(a.out) + (size_t)b * a.L * (a.H * kDV) + (size_t)h * kDV + col;
      if (m == kCH && c0 >= a.P) {
#pragma unroll
        for (int ti = 0; ti < 4; ti++)
#pragma unroll
          for (int e = 0; e < 4; e++) ob[(size_t)(c0 - a.P + 16 * ti + 4 * grp + e) * (a.H * kDV)] = (T)Y[ti][e];
      } else {
#pragma unroll
        for (int ti = 0; ti < 4; ti++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int t = 16 * ti + 4 * grp + e, r = c0 + t;
            if (t < m && r >= a.P) ob[(size_t)(r - a.P) * (a.H * kDV)] = (T)Y[ti][e];
          }
      }
    }
    if (p + 1 < nchunks) prep_chunk(p + 1);
    // The v and z loads run every period (past the last chunk on the last chunk's rows, never used): conditional
    // loads would make the loop-carried registers a merge of old and new values, resolved with copies that wait
    // for the loads right after they are issued.
    if (a.gnorm) fetch_z(min(p + 1, nchunks - 1));
    __syncthreads();  // A
  }
  const int g0 = (tid0 & 63) >> 4, l16 = tid0 & 15;
#pragma unroll
  for (int it = 0; it < 8; it++)
#pragma unroll
    for (int e = 0; e < 4; e++)
      gpw<float>(a.S_out)[sbase + (size_t)(16 * it + 4 * g0 + e) * kDV + 16 * w + l16] = S[it][e];
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
  auto kr = gdn_recur_kernel<T>;
  e = hipFuncSetAttribute(reinterpret_cast<const void*>(kr), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)sizeof(RecLds));
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kr, dim3(a.B * a.H), dim3(kRT), sizeof(RecLds), s, a);
  return hipGetLastError();
}

}  // namespace

size_t gdn_split_image_bytes() { return (size_t)kChunkScratch; }

hipError_t launch_gdn_split(const GdnArgs& a, hipStream_t s) {
  if (a.DK != kDK || a.DV != kDV || a.KC != kKC || !a.img) return hipErrorInvalidValue;
  if (a.P - a.s0 >= kCH || a.P < a.s0) return hipErrorInvalidValue;  // at most one open chunk is replayed
  return a.dtype == 0 ? launch<float>(a, s) : launch<_Float16>(a, s);
}

}  // namespace ha
