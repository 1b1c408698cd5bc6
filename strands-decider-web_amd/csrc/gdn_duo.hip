// Chunked gated-delta prefill on two CUs per (sequence, head) (ha_recurrence HA_CHUNKED for 16 < B*H <= 128,
// HA_CHUNKED_PAIRED), gfx950.
//
// Same semantics as the sequential rule (reference web/public/engine/wgsl.js:124-187 + 252-268), evaluated in the
// chunked WY/UT form (Yang et al. 2024, "Parallelizing Linear Transformers with the Delta Rule over Sequence
// Length"; Yang, Kautz & Hatamizadeh, "Gated Delta Networks"). For a chunk of 32 rows with cumulative log-decay gc
// and the state S at its start:
//   A   = strictly_lower(beta_t (k^_t . k^_t') exp(gc_t - gc_t'))      T = (I + A)^-1
//   V_new = T diag(beta) v - T diag(beta e^gc) (k^ S)
//   o_t = exp(gc_t) q^_t S + sum_{t'<=t} (q^_t . k^_t') exp(gc_t - gc_t') V_new_t'
//   S  <- exp(gc_31) S + k^T diag(exp(gc_31 - gc)) V_new
//
// One CU's VALU and latency chains bound a one-workgroup form at a period of about 10K cycles per 32 rows, and at
// B = 8 half the CUs have no head. So each (sequence, head) gets two workgroups:
//   producer: everything that does not depend on the state, chunk by chunk: q/k conv + SiLU + l2 norm, the gates, the
//     A and score tiles, T = (I + A)^-1, T diag(beta) and T diag(beta e^gc). In one period wave 0 runs chunk q's T
//     chain, waves 1..2 its score tiles, wave 3 chunk q + 1's gates, waves 4..7 chunk q + 1's q/k conv, and waves
//     1..3 copy chunk q - 1's finished tile set (22.25 KiB: q^, k^, the three [32][32] tiles and two gate vectors,
//     no padding) into that chunk's slot in device memory.
//   consumer: waves 0..3 own 32 value columns each of the fp32 state in MFMA accumulators and do the state work of
//     chunk p (the state update reads its k^T operand from k^ itself with transposing LDS reads); meanwhile waves
//     4..7 (helpers) DMA chunk p + 1's tile set from its slot into LDS, apply the gated RMSNorm to chunk p - 1's output
//     and store it, and run chunk p + 1's v conv.
// Each role passes one workgroup barrier per period.
// The two exchange progress through counters: `produced` (tile sets in their slots) and `consumed` (sets copied into
// the consumer's LDS). Counter values carry a per-launch epoch (epoch << kDuoEpochShift | chunks), so values left by
// earlier launches never satisfy a wait and nothing is cleared between launches. Data is written with device-coherent
// (sc1) stores and waited for (vmcnt 0) before the counter store; readers load counters and data with sc1.
// Ordinary launch, no co-residency guarantee: every chunk has its own slot, so the producer never needs the consumer
// (it only holds back, for a bounded time, while it is more than kLead chunks ahead, which keeps the sets it writes
// in the caches), and it is dispatched first (see the block mapping at the kernel). A consumer that is resident
// therefore waits only for a producer that is resident or finished. Every wait is bounded.
//
// Chunk boundaries sit at s0 + 32k and the state advances over every complete chunk. The state written out is the
// one at the end of the call's last complete 64-row span (the position the engine stores it at); a resumed call
// replays the rows from there with the same chunk boundaries, so prefix + suffix is bit-identical to one forward.
//
// MFMA operand conventions are those of gdn_common.h: lane l supplies row (l & 15) of A and column (l & 15) of B;
// a D tile pair reused as a B operand is matched by A operands read in the permuted K order
// {4 grp + e} U {16 + 4 grp + e}.
#include "gdn_common.h"

namespace ha {
namespace {

constexpr int kC = 32;          // chunk rows
constexpr int kP = kC + 8;      // row pitch (halves) of [*][32] f16 tiles
constexpr int kMP = kC + 4;     // row pitch (floats) of the fp32 A / T tile
constexpr int kThreads = 512;   // 8 waves per workgroup
constexpr int kOP = kDV + 4;    // row pitch (floats) of the consumer's output rows
constexpr int kLead = 24;       // chunks the producer may run ahead of the consumer before it holds back
// Vector memory instructions a helper wave issues after its tile-set DMA in every period: the v rows (kKC + 7 loads), the
// z rows (4) and the counter (1). s_waitcnt with vmcnt = kAfterDma (expcnt and lgkmcnt not waited for) then covers
// the DMA alone.
constexpr int kAfterDma = kKC + 7 + 4 + 1;
// s_waitcnt operand that waits until at most n vector memory instructions are outstanding (expcnt, lgkmcnt: no wait)
constexpr int wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kWaitDma = wait_vm(kAfterDma);

typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i2v __attribute__((ext_vector_type(2)));

// One chunk's tiles, as the producer builds them in LDS and the consumer reads them; copied between the two as bytes.
// No padding: the row layouts are swizzled in 8-half (16-byte) units instead (qk_at, sq_at), so the whole set is data.
struct Set {
  _Float16 Qs[kC * kDK];   // q^ / sqrt(DK), [t][i], by qk_at
  _Float16 Ks[kC * kDK];   // k^, [t][i], by qk_at
  _Float16 Tb[kC * kC];    // T diag(beta), [t][t'], by sq_at (the block above the diagonal stays zero)
  _Float16 Tw[kC * kC];    // T diag(beta e^gc), by sq_at
  _Float16 Att[kC * kC];   // decay-masked causal q^ k^T, by sq_at
  float eg[kC];            // e^gc
  float ed[kC];            // e^(gc_31 - gc)
};
static_assert(sizeof(Set) <= kDuoSetBytes, "a tile set fits one ring slot");
static_assert(sizeof(Set) % 16 == 0 && sizeof(Set) / 16 > 22 * 64 && sizeof(Set) / 16 <= 23 * 64,
              "the producer's copy (7 + 8 + 8 instructions of 64 units) and the consumer's DMA (23 of 1 KiB) cover the set");
static_assert(kDuoSetBytes % 1024 == 0, "ring slots are whole 1 KiB DMA instructions");
union SetBuf {
  Set s;
  unsigned char raw[kDuoSetBytes];
};
// The gate vectors only the producer reads
struct Gates {
  float gc[kC];            // cumulative log decay inside the chunk
  float bt[kC];            // beta
  float rowf[kC];          // e^(gc_t - gc_16(t/16)), in (0, 1]
  float brow[kC];          // beta_t rowf_t
  float colf[kC];          // e^(gc_16 - gc_t') for t' < 16, in (0, 1]
};

struct ProducerLds {
  SetBuf s[3];                 // chunk q (T chain), q + 1 (written by the conv waves), q - 1 (copied out), by c % 3
  Gates g[3];                  // the same chunks' producer-side gate vectors
  float Tm[kC * kMP];          // A, then T, fp32
  float cwq[4][64][kKC];       // q/k conv taps: channel 4 g + c (g < 64: q then k) at cwq[c][g]
};
struct ConsumerLds {
  SetBuf s[2];                 // chunk p (state waves) and chunk p + 1 (DMA target)
  _Float16 VT[2][kDV * kP];    // v^ transposed, [j][t] (8-row groups swizzled by vt32), by chunk parity
  float osg[2][kC * kOP];      // output rows before the gated norm, by chunk parity
  float red[2][kC * 4];        // gated-norm partial sums, [t][state wave], by chunk parity
  float cwv[4][32][kKC];       // v conv taps: channel 4 g + c at cwv[c][g]
};

// q^ / k^ element (t, i): 8-half unit i / 8 of row t sits at unit (i / 8) ^ rot(t % 16), rot a one-bit rotation of the
// row's 4 low bits. A bijection of t % 16: the 16 rows an MFMA operand read covers at one column land on 16 different
// units. The rotation puts rows 4 g .. 4 g + 3 on units that differ in bits 1..2, so the transposing reads of the
// state update (two units of each of 4 rows per 16 lanes) touch 8 different units.
__device__ __forceinline__ int qk_at(int t, int i) {
  return t * kDK + 8 * ((i >> 3) ^ (((t << 1) | ((t >> 3) & 1)) & 15)) + (i & 7);
}
// k^T operand of the state update, read from k^ itself with ds_read_b64_tr_b16. In each 16-lane group of that
// instruction, lane m receives element (4 e + m / 4, m % 4) of the 16 x 4 matrix whose row j is the 4 halves at lane
// j's address. Lane (grp, m) supplying the address of k^[r0 + 4 grp + m / 4][i0 + 4 (m % 4)] therefore receives
// k^[r0 + 4 grp + e][i0 + m], e = 0..3: row i0 + m of k^T at the K indices 4 grp + e of the permuted order.
__device__ __forceinline__ h4 kT_piece(const _Float16* Ks, int r0, int i0, int grp, int m) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  const _Float16* p = Ks + qk_at(r0 + 4 * grp + (m >> 2), i0 + 4 * (m & 3));
  const s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)(p));
  return __builtin_bit_cast(h4, v);
}
// element (t, t') of a [32][32] f16 tile: unit t' / 8 of row t sits at unit (t' / 8) ^ ((t / 4) % 4)
__device__ __forceinline__ int sq_at(int t, int j) { return t * kC + 8 * ((j >> 3) ^ ((t >> 2) & 3)) + (j & 7); }
// perm_a (gdn_common.h) for the swizzled tiles: A row r, K block kb, lane group grp, the two 4-half pieces at
// K = 32 kb + 4 grp and 32 kb + 16 + 4 grp
template <int (*AT)(int, int)>
__device__ __forceinline__ h8 perm_a_sw(const _Float16* base, int r, int kb, int grp) {
  const h4 lo = *reinterpret_cast<const h4*>(base + AT(r, 32 * kb + 4 * grp));
  const h4 hi = *reinterpret_cast<const h4*>(base + AT(r, 32 * kb + 16 + 4 * grp));
  return h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// v^T element (j, t) lives at j * kP + 8 * ((t / 8) ^ ((j / 16) % 4)) + t % 8: the state waves read 8 rows of one
// channel (16 bytes, a B operand) and the helpers write 4 rows of channels 4 cvg + c, which without the swizzle
// would put every fourth lane on the same banks
__device__ __forceinline__ int vt32(int j, int g8) { return j * kP + 8 * (g8 ^ ((j >> 4) & 3)); }

// sum over 32 lanes (0..31 or 32..63): the 16 lanes of a DPP row, then the paired row
__device__ __forceinline__ float sum32(float v) {
  v = row_sum16(v);
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v), false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}

// Progress counters: device-coherent loads and stores (no release fence: the writer drains its data stores first)
__device__ __forceinline__ unsigned ld_counter(const unsigned* c) {
  return __hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_counter(unsigned* c, unsigned v) {
  __hip_atomic_store(c, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until the counter reaches v and returns the value read, for at most `polls` polls of about a microsecond.
// Callers keep the value and poll again only when it falls short.
__device__ __forceinline__ unsigned wait_counter(const unsigned* c, unsigned v, int polls) {
  unsigned x = 0;
  for (int i = 0; i < polls; i++) {
    x = ld_counter(c);
    if (x >= v) break;
    __builtin_amdgcn_s_sleep(2);
  }
  return x;
}

// NC consecutive channels of one row (one 8- or 16-byte load)
__device__ __forceinline__ void loadc(gptr<float> p, float (&o)[4]) { load4(p, o); }
__device__ __forceinline__ void loadc(gptr<_Float16> p, float (&o)[4]) { load4(p, o); }
__device__ __forceinline__ void loadc(gptr<float> p, float (&o)[2]) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  const f2 x = *(gptr<f2>)(p);
  o[0] = x[0]; o[1] = x[1];
}
__device__ __forceinline__ void loadc(gptr<_Float16> p, float (&o)[2]) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 x = *(gptr<h2>)(p);
  o[0] = (float)x[0]; o[1] = (float)x[1];
}

// Loads rows cs + r0 - 3 .. cs + r0 + NR - 4 (NR = the rows x holds) at element column `col`, NC channels. Uniform
// row bases and 32-bit lane offsets when no row is a replay row or past the end; per-lane row pointers otherwise.
// Rows past the end repeat the last row: they only feed conv outputs past the end, which are masked.
template <typename T, int NR, int NC>
__device__ __forceinline__ void fetch_rows(const GdnArgs& a, const RowSrc& src, int b, int cs, int r0, int col,
                                           float (&x)[NR][NC]) {
  const int end = a.P + a.L;
  const unsigned rowb = (unsigned)a.stride * sizeof(T);
  if (cs - (kKC - 1) >= a.P && cs + kC <= end) {
    const char* base = (const char*)a.in + ((size_t)b * a.L + (cs - (kKC - 1) - a.P)) * rowb;
    const unsigned off = (unsigned)r0 * rowb + (unsigned)col * (unsigned)sizeof(T);
#pragma unroll
    for (int i = 0; i < NR; i++) loadc(gp<T>(base + (size_t)i * rowb + off), x[i]);
  } else {
#pragma unroll
    for (int i = 0; i < NR; i++) {
      const int r = cs + r0 - (kKC - 1) + i, rc = min(r, end - 1);
      loadc(row_of<T>(a, src, b, rc) + col, x[i]);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Producer

// One 16x16 tile of K K^T (-> A, fp32, in Tm) or Q K^T (-> decay-masked scores, f16) of the chunk in st; block row
// ti, block column tj <= ti
__device__ __forceinline__ void tile(Set& st, const Gates& gt, float* Tm, bool isq, int ti, int tj, int grp, int c16) {
  const _Float16* ab = isq ? st.Qs : st.Ks;
  const int ra = 16 * ti + c16, rb = 16 * tj + c16;
  f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int ks = 0; ks < 4; ks++)
    acc = mfma16(*reinterpret_cast<const h8*>(ab + qk_at(ra, 8 * grp + 32 * ks)),
                 *reinterpret_cast<const h8*>(st.Ks + qk_at(rb, 8 * grp + 32 * ks)), acc);
  const int tp = 16 * tj + c16, t0 = 16 * ti + 4 * grp;
  if (ti != tj) {
    // below the diagonal blocks gc_t <= gc_16 <= gc_t', so e^(gc_t - gc_t') factors into two terms <= 1
    const float cf = gt.colf[tp];
    if (!isq) {
      const f4 bf = lds4(&gt.brow[t0]);
#pragma unroll
      for (int e = 0; e < 4; e++) Tm[(t0 + e) * kMP + tp] = acc[e] * bf[e] * cf;
    } else {
      const f4 rf = lds4(&gt.rowf[t0]);
#pragma unroll
      for (int e = 0; e < 4; e++) st.Att[sq_at(t0 + e, tp)] = (_Float16)(acc[e] * rf[e] * cf);
    }
  } else {
    const float gq = gt.gc[tp];
    const f4 gv = lds4(&gt.gc[t0]), bv = lds4(&gt.bt[t0]);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int t = t0 + e;
      const float dec = __expf(fminf(gv[e] - gq, 0.0f));
      if (!isq)
        Tm[t * kMP + tp] = tp < t ? bv[e] * acc[e] * dec : 0.0f;
      else
        st.Att[sq_at(t, tp)] = (_Float16)(tp <= t ? acc[e] * dec : 0.0f);
    }
  }
}

// The two diagonal blocks of T = (I + A)^-1 by forward substitution: lane group grp solves block grp % 2, lane c16
// owning column c16. Right-looking: once entry r of the column is final, it is eliminated from the rows below, so each
// step's updates are independent (column r of A read as broadcasts within the group). Groups 0 and 1 store their
// block: T_bb in Tm, T diag(beta) and T diag(beta e^gc) in the f16 tiles.
__device__ __forceinline__ void solve_diag(Set& st, const Gates& gt, float* Tm, int grp, int c16) {
  const int base = 16 * (grp & 1);
  float pc[16];
#pragma unroll
  for (int r = 0; r < 16; r++) pc[r] = r == c16 ? 1.0f : 0.0f;
#pragma unroll
  for (int r = 0; r < 15; r++) {
#pragma unroll
    for (int r2 = r + 1; r2 < 16; r2++) pc[r2] = fmaf(-Tm[(base + r2) * kMP + base + r], pc[r], pc[r2]);
  }
  wave_sync();  // every lane has read A's block before it is overwritten
  if (grp < 2) {
    const float cb = gt.bt[base + c16], cbw = cb * st.eg[base + c16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      Tm[(base + r) * kMP + base + c16] = pc[r];
      st.Tb[sq_at(base + r, base + c16)] = (_Float16)(pc[r] * cb);
      st.Tw[sq_at(base + r, base + c16)] = (_Float16)(pc[r] * cbw);
    }
  }
}

// The block below the diagonal: T_10 = -T_11 (A_10 T_00) on v_mfma_f32_16x16x4f32, D layout (rows 4 grp + e of the
// block, column c16) used directly as the next product's B operand, the A operand read in the same K order
__device__ __forceinline__ void solve_offdiag(Set& st, const Gates& gt, const float* Tm, int grp, int c16) {
  f4 X = {0.0f, 0.0f, 0.0f, 0.0f}, Y = X;
  const f4 av = lds4(&Tm[(16 + c16) * kMP + 4 * grp]);
  f4 t0;
#pragma unroll
  for (int e = 0; e < 4; e++) t0[e] = Tm[(4 * grp + e) * kMP + c16];
#pragma unroll
  for (int e = 0; e < 4; e++) X = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], t0[e], X, 0, 0, 0);
  const f4 tv = lds4(&Tm[(16 + c16) * kMP + 16 + 4 * grp]);
#pragma unroll
  for (int e = 0; e < 4; e++) Y = __builtin_amdgcn_mfma_f32_16x16x4f32(tv[e], X[e], Y, 0, 0, 0);
  const float fb = gt.bt[c16], fw = fb * st.eg[c16];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const int t = 16 + 4 * grp + e;
    st.Tb[sq_at(t, c16)] = (_Float16)(-Y[e] * fb);
    st.Tw[sq_at(t, c16)] = (_Float16)(-Y[e] * fw);
  }
}

template <typename T>
__device__ __forceinline__ void produce(const GdnArgs& a, int b, int h, ProducerLds& sm, char* ring, unsigned* produced,
                                        const unsigned* consumed, unsigned ep) {
  const int tid0 = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  const int end = a.P + a.L;
  const int n = (end - a.s0 + kC - 1) / kC;
  const float qscale = 0.08838834764831845f;  // 1/sqrt(128)
  const unsigned rowb = (unsigned)a.stride * sizeof(T);
  const char* const seq_in = (const char*)a.in + (size_t)b * a.L * rowb;

  for (int i = tid0; i < 2 * 128 * kKC; i += kThreads) {
    const int lc = i / kKC, j = i % kKC;
    const int ch = lc < 128 ? h * kDK + lc : a.H * kDK + h * kDK + (lc - 128);
    sm.cwq[lc & 3][lc >> 2][j] = gp<float>(a.conv_w)[(size_t)ch * kKC + j];
  }
  // the block above the diagonal of every set's f16 T and score tiles is read by full K blocks and never written
  for (int idx = tid0; idx < 3 * 16 * 16; idx += kThreads) {
    const int st = idx >> 8, t = (idx >> 4) & 15, tp = 16 + (idx & 15);
    sm.s[st].s.Tb[sq_at(t, tp)] = (_Float16)0.0f;
    sm.s[st].s.Tw[sq_at(t, tp)] = (_Float16)0.0f;
    sm.s[st].s.Att[sq_at(t, tp)] = (_Float16)0.0f;
  }
  const float na = gp<float>(a.negA)[h], db = gp<float>(a.dtb)[h];
  const int aoff = a.C + a.H * kDV + h, boff = aoff + a.H;
  const RowSrc src = row_src(a);
  const int last_cs = a.s0 + kC * (n - 1);

  // conv waves 4..7: wave cw -> rows 8 cw .. 8 cw + 7 of a chunk; lane l -> channels 4 (l % 32) .. + 3 of q (l < 32)
  // or k (l >= 32). Wave 3's lanes 0..31 hold rows 0..31's a/b inputs for the gates. Both are loaded a period ahead,
  // every period (on clamped rows past the end): conditional loads would make the loop-carried registers a merge of
  // old and new values, which the compiler resolves with copies that wait for the loads right after they are issued.
  const bool conv = w >= 4;
  const int cw = w - 4;
  float xq[kKC + 7][4], ga = 0.0f, gb = 0.0f;
  auto fetch_qk = [&](int cs) {
    const int l = opaque(tid0) & 63;
    fetch_rows<T>(a, src, b, min(cs, last_cs), 8 * cw, (l < 32 ? 0 : a.H * kDK) + h * kDK + 4 * (l & 31), xq);
  };
  auto fetch_ab = [&](int cs) {
    const int lane = opaque(tid0) & 31;
    cs = min(cs, last_cs);
    // rows past the end: their gates are never used (the gate lanes mask them)
    const gptr<T> grow = cs >= a.P && cs + kC <= end ? gp<T>(seq_in + (size_t)(cs - a.P + lane) * rowb)
                                                     : row_of<T>(a, src, b, min(cs + lane, end - 1));
    ga = (float)grow[aoff];
    gb = (float)grow[boff];
  };
  if (conv) fetch_qk(a.s0);
  if (w == 3) fetch_ab(a.s0);
  unsigned seen = 0;  // the consumer's progress as last read (copy waves)
  __syncthreads();  // conv taps and zero blocks visible

  // Chunk q - 1's set into its slot: copy wave w (1..3) takes NU 16-byte units from unit u0 on (one store instruction
  // per 64 units; the set's last instruction is partial); the period's end waits for those stores. While the consumer
  // has not yet taken chunk q - 1 - kLead, the wave holds back for up to 64 polls first (the slot is this chunk's
  // alone, so going on is always safe).
  constexpr int kSetUnits = (int)sizeof(Set) / 16;
  auto copy_out = [&](int c, int u0, auto nu) {
    constexpr int NU = decltype(nu)::value;
    if (c >= kLead && seen < ep + (unsigned)(c - kLead + 1))
      seen = wait_counter(consumed, ep + (unsigned)(c - kLead + 1), 64);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(ring + (size_t)c * kDuoSetBytes, 0, kDuoSetBytes, 0x00020000);
    const unsigned char* from = sm.s[c % 3].raw;
    const int lane = opaque(tid0) & 63;
#pragma unroll
    for (int it = 0; it < NU; it++) {
      const int u = u0 + 64 * it + lane;
      if (u < kSetUnits) {
        const f4 v = lds4(reinterpret_cast<const float*>(from + 16 * u));
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i4v, v), rs, 16 * u, 0, 16);
      }
    }
  };

  // Period q: wave 0 runs chunk q's T chain (set q % 3); waves 1..3 copy chunk q - 1's finished set (q - 1) % 3 into
  // its ring slot, waves 1 and 2 after making chunk q's score tiles, wave 3 after the gates of chunk q + 1; the conv
  // waves write chunk q + 1 into set (q + 1) % 3. One barrier per period. The copy waves wait for their stores at the
  // period's end (they were issued a good part of a period earlier), so chunk q - 1 is published after period q's
  // barrier.
  for (int q = -1; q <= n + 1; q++) {
    const int c1 = a.s0 + kC * (q + 1);  // chunk q + 1
    const int tid = opaque(tid0), lane = tid & 63, grp = lane >> 4, c16 = lane & 15;
    if (conv) {
      if (q + 1 < n) {
        const int isk = lane >> 5, l32 = lane & 31, m = min(kC, end - c1);
        float uq[8][4], ss[8];
#pragma unroll
        for (int r = 0; r < 8; r++) ss[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const f4 wc = lds4(sm.cwq[c][lane]);
#pragma unroll
          for (int r = 0; r < 8; r++) {
            float sv = wc[0] * xq[r][c];
            sv = fmaf(wc[1], xq[r + 1][c], sv);
            sv = fmaf(wc[2], xq[r + 2][c], sv);
            sv = fmaf(wc[3], xq[r + 3][c], sv);
            uq[r][c] = 8 * cw + r < m ? silu(sv) : 0.0f;
            ss[r] = fmaf(uq[r][c], uq[r][c], ss[r]);
          }
        }
        fetch_qk(c1 + kC);
        Set& st = sm.s[(q + 1) % 3].s;
#pragma unroll
        for (int r = 0; r < 8; r++) {
          const float rs = rsqrtf(sum32(ss[r]) + 1e-6f) * (isk ? 1.0f : qscale);
#pragma unroll
          for (int c = 0; c < 4; c++) uq[r][c] *= rs;
          const h4 hv = {(_Float16)uq[r][0], (_Float16)uq[r][1], (_Float16)uq[r][2], (_Float16)uq[r][3]};
          *reinterpret_cast<h4*>((isk ? st.Ks : st.Qs) + qk_at(8 * cw + r, 4 * l32)) = hv;
        }
      } else {
        fetch_qk(c1 + kC);
      }
    } else if (w == 0) {
      if (q >= 0 && q < n) {
        Set& st = sm.s[q % 3].s;
        const Gates& gt = sm.g[q % 3];
        tile(st, gt, sm.Tm, false, 0, 0, grp, c16);
        tile(st, gt, sm.Tm, false, 1, 1, grp, c16);
        tile(st, gt, sm.Tm, false, 1, 0, grp, c16);
        wave_sync();
        solve_diag(st, gt, sm.Tm, grp, c16);
        wave_sync();
        solve_offdiag(st, gt, sm.Tm, grp, c16);
      }
    } else {
      if (q >= 0 && q < n) {
        Set& st = sm.s[q % 3].s;
        const Gates& gt = sm.g[q % 3];
        if (w == 1) {
          tile(st, gt, sm.Tm, true, 0, 0, grp, c16);
          tile(st, gt, sm.Tm, true, 1, 0, grp, c16);
        } else if (w == 2) {
          tile(st, gt, sm.Tm, true, 1, 1, grp, c16);
        }
      }
      if (w == 3) {
        if (q + 1 < n) {
          // beta and the cumulative log decay of row `lane` (lanes 0..31) of chunk q + 1
          const int gl = lane & 31, m = min(kC, end - c1);
          float gcr = 0.0f, btr = 0.0f;
          if (lane < 32 && gl < m) {
            btr = __builtin_amdgcn_rcpf(1.0f + __expf(-gb));
            const float xs = ga + db;
            gcr = na * (xs > 20.0f ? xs : log1pf(__expf(xs)));
          }
#pragma unroll
          for (int d = 1; d < 32; d <<= 1) {
            const float o = __shfl_up(gcr, d);
            if (gl >= d) gcr += o;
          }
          const float glast = __shfl(gcr, 31), g16 = __shfl(gcr, 16);
          const float rf = __expf(gcr - __shfl(gcr, lane & 16));
          Set& st = sm.s[(q + 1) % 3].s;
          Gates& gt = sm.g[(q + 1) % 3];
          if (lane < 32) {
            gt.gc[lane] = gcr;
            st.eg[lane] = __expf(gcr);
            gt.bt[lane] = btr;
            st.ed[lane] = __expf(glast - gcr);
            gt.rowf[lane] = rf;
            gt.brow[lane] = btr * rf;
            gt.colf[lane] = lane < 16 ? __expf(g16 - gcr) : 0.0f;
          }
        }
        // issued before the copy's stores, so that the next period's wait for them does not wait for the stores too
        fetch_ab(c1 + kC);
      }
      if (q >= 1 && q <= n) {
        if (w == 1)
          copy_out(q - 1, 15 * 64, Width<8>{});
        else if (w == 2)
          copy_out(q - 1, 7 * 64, Width<8>{});
        else
          copy_out(q - 1, 0, Width<7>{});
      }
      __builtin_amdgcn_s_waitcnt(wait_vm(0));  // this period's set stores (and wave 3's gate loads) are complete
    }
    __syncthreads();
    if (tid0 == 64 && q >= 1) st_counter(produced, ep + (unsigned)min(q, n));  // chunks 0 .. q - 1 are in their slots
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Consumer

template <typename T, bool kDebugWaits>
__device__ __forceinline__ void consume(const GdnArgs& a, int b, int h, ConsumerLds& sm, const char* ring,
                                        const unsigned* produced, unsigned* consumed, unsigned ep) {
  const int tid0 = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  const int end = a.P + a.L;
  const int n = (end - a.s0 + kC - 1) / kC;
  const int s1 = a.s0 + 64 * ((end - a.s0) / 64);  // the stored state position
  const unsigned orowb = (unsigned)(a.H * kDV) * sizeof(T);
  // this sequence's output rows as a buffer: stores at offsets past its L rows are dropped by the hardware
  const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(
      (char*)a.out + (size_t)b * a.L * orowb, 0, (int)((unsigned)a.L * orowb), 0x00020000);
  const char* const seq_in = (const char*)a.in + (size_t)b * a.L * ((unsigned)a.stride * sizeof(T));
  const size_t sbase = ((size_t)b * a.H + h) * kDK * kDV;
  const bool state = w < 4;
  const int hw = w - 4;  // helper wave
  const int last_cs = a.s0 + kC * (n - 1);

  for (int i = tid0; i < 128 * kKC; i += kThreads) {
    const int lc = i / kKC, j = i % kKC;
    sm.cwv[lc & 3][lc >> 2][j] = gp<float>(a.conv_w)[(size_t)(2 * a.H * kDK + h * kDV + lc) * kKC + j];
  }

  // Helper lanes: v conv of rows 8 vrg .. + 7 (vrg = the helper wave), channels 2 cvg, 2 cvg + 1 (a row's 128 channels
  // are one 512-byte load across the wave, and the 11 rows a lane loads for its 8 outputs overlap the next wave's by
  // only 3); gated norm of row fr, columns fc + 32 q .. + 3
  // (q < 4), so that the 8 lanes of a row cover one contiguous 128-byte span per z load and output store.
  // They hold the raw v rows and the z rows of the chunks they work on next, loaded a period ahead (every period, on
  // clamped rows past the end, so that the registers are never a merge of old and new loads) into second buffers.
  const int ht0 = tid0 - 256;
  const RowSrc src = row_src(a);
  float xv[kKC + 7][2], xn[kKC + 7][2];
  f4 zq[4], zn[4], gw[4] = {};
  if (!state && a.gnorm)
#pragma unroll
    for (int q = 0; q < 4; q++) gw[q] = ld4(gp<float>(a.gnorm) + 4 * (ht0 & 7) + 32 * q);
  unsigned seen = 0;   // the producer's progress as last read (helper waves)
  unsigned ahead = 0;  // the read issued in the previous period, taken into `seen` at the next period's start
  auto fetch_v = [&](int cs) {
    const int ht = opaque(tid0) - 256, vrg = ht >> 6, cvg = ht & 63;
    fetch_rows<T>(a, src, b, min(cs, last_cs), 8 * vrg, 2 * a.H * kDK + h * kDV + 2 * cvg, xn);
  };
  f4 wcv[2];  // the lane's two channels' conv taps, read from LDS once the taps are staged
  auto vconv = [&](int cs) {
    const int ht = opaque(tid0) - 256, vrg = ht >> 6, cvg = ht & 63;
    const int mv = min(kC, end - cs);
    _Float16* VT = sm.VT[((cs - a.s0) / kC) & 1];
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const int j = 2 * cvg + c;
      const f4 wc = wcv[c];
      h8 vt;
#pragma unroll
      for (int r = 0; r < 8; r++) {
        float sv = wc[0] * xv[r][c];
        sv = fmaf(wc[1], xv[r + 1][c], sv);
        sv = fmaf(wc[2], xv[r + 2][c], sv);
        sv = fmaf(wc[3], xv[r + 3][c], sv);
        vt[r] = (_Float16)(8 * vrg + r < mv ? silu(sv) : 0.0f);
      }
      *reinterpret_cast<h8*>(VT + vt32(j, vrg)) = vt;
    }
  };
  auto fetch_z = [&](int c0) {
    const int ht = opaque(tid0) - 256, fr = ht >> 3, fc = 4 * (ht & 7);
    const int rr = min(max(min(c0, last_cs) + fr - a.P, 0), a.L - 1);
    const gptr<T> zr = gp<T>(seq_in) + (size_t)rr * a.stride + a.C + h * kDV + fc;
#pragma unroll
    for (int q = 0; q < 4; q++) zn[q] = ld4(zr + 32 * q);
  };
  // chunk c's tile set from its slot into LDS: whole 1 KiB DMA instructions, helper wave wq issues every fourth. The
  // producer is resident or done (it is dispatched first and waits for nothing), so the wait ends; its bound only
  // keeps the kernel finite. A wait that runs out sets `seen` to ~0u, a value no counter takes (the chunk field stays
  // below 4095): the launch's outputs are undefined from there on, later waits pass at once, and the kernel's end
  // reports it through the engine's error word (the test instantiation kDebugWaits waits with a.wait's skew and poll
  // bound instead of none and kWaitPolls).
  const unsigned epw = kDebugWaits ? ep + a.wait.skew : ep;
  auto dma_set = [&](int c, int wq) {
    const unsigned want = epw + (unsigned)(c + 1);
    if (seen < want) {
      const unsigned x = wait_counter(produced, want, kDebugWaits ? a.wait.polls : kWaitPolls);
      seen = x >= want ? max(seen, x) : ~0u;
    }
    const char* from = ring + (size_t)c * kDuoSetBytes;
    unsigned char* to = sm.s[c & 1].raw;
    const int ln = opaque(tid0) & 63;
    for (int i = wq; i < kDuoSetBytes / 1024; i += 4)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(from + 1024 * (size_t)i + 16 * ln),
                                       (__attribute__((address_space(3))) void*)(to + 1024 * i), 16, 0, 16);
  };
  f4 S[2][8];  // state waves: S[ct][it][e] = S[16 it + 4 grp + e][32 w + 16 ct + c16]
  if (state) {
    const int g0 = (tid0 & 63) >> 4, l16 = tid0 & 15;
#pragma unroll
    for (int ct = 0; ct < 2; ct++)
#pragma unroll
      for (int it = 0; it < 8; it++)
#pragma unroll
        for (int e = 0; e < 4; e++)
          S[ct][it][e] = a.S_in ? gp<float>(a.S_in)[sbase + (size_t)(16 * it + 4 * g0 + e) * kDV + 32 * w + 16 * ct + l16]
                                : 0.0f;
  } else {
    // the first chunk's v conv and the next rows' loads before the wait for the producer's first tile set, which
    // they do not need
    fetch_v(a.s0);
    __syncthreads();  // v conv taps visible (the state waves pass this barrier below)
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const int j = 2 * (ht0 & 63) + c;
      wcv[c] = lds4(sm.cwv[j & 3][j >> 2]);
    }
#pragma unroll
    for (int r = 0; r < kKC + 7; r++)
#pragma unroll
      for (int c = 0; c < 2; c++) xv[r][c] = xn[r][c];
    vconv(a.s0);
    fetch_v(a.s0 + kC);
    fetch_z(a.s0);
    dma_set(0, hw);
  }
  // Drain the prologue's loads: the compiler's wait counting merges the loop's entry state into every period, so a load
  // still outstanding at the loop head would make each period's first use of its registers wait for every global access
  // issued before it.
  __builtin_amdgcn_s_waitcnt(0);
  if (state) __syncthreads();
  __syncthreads();
  if (tid0 == 256) st_counter(consumed, ep + 1u);

  // Period p: the state waves run chunk p (its rows into osg[p % 2]); the helpers bring chunk p + 1's tile set, normalise
  // and store chunk p - 1, run chunk p + 1's v conv and load the next rows. One barrier per period.
  auto period = [&](int p) __attribute__((always_inline)) {
    const int c0 = a.s0 + kC * p;  // chunk p
    const int tid = opaque(tid0), lane = tid & 63, grp = lane >> 4, c16 = lane & 15;
    if (state) {
      if (p < n) {
        const int m = min(kC, end - c0);
        Set& st = sm.s[p & 1].s;

        const _Float16* VT = sm.VT[p & 1];
        float* osg = sm.osg[p & 1];
        // k^ S and q^ S together, K block outermost (one f16 copy of that block of S at a time)
        f4 KS[2][2], O[2][2], Vn[2][2];
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
          h8 S16[2];
#pragma unroll
          for (int ct = 0; ct < 2; ct++) S16[ct] = pack_b(S[ct][2 * kb], S[ct][2 * kb + 1]);
#pragma unroll
          for (int ti = 0; ti < 2; ti++) {
            const h8 ka = perm_a_sw<qk_at>(st.Ks, 16 * ti + c16, kb, grp);
            const h8 qa = perm_a_sw<qk_at>(st.Qs, 16 * ti + c16, kb, grp);
#pragma unroll
            for (int ct = 0; ct < 2; ct++) {
              const f4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};
              KS[ct][ti] = mfma16(ka, S16[ct], kb ? KS[ct][ti] : z4);
              O[ct][ti] = mfma16(qa, S16[ct], kb ? O[ct][ti] : z4);
            }
          }
        }
        // V_new = T diag(beta) v - T diag(beta e^gc) (k^ S)
        {
          h8 KSb[2];
#pragma unroll
          for (int ct = 0; ct < 2; ct++) KSb[ct] = pack_b(KS[ct][0], KS[ct][1]);
#pragma unroll
          for (int ti = 0; ti < 2; ti++) {
            const h8 tb = *reinterpret_cast<const h8*>(st.Tb + sq_at(16 * ti + c16, 8 * grp));
            const h8 tw = perm_a_sw<sq_at>(st.Tw, 16 * ti + c16, 0, grp);
#pragma unroll
            for (int ct = 0; ct < 2; ct++) {
              const int col = 32 * w + 16 * ct + c16;
              const f4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};
              const f4 u = mfma16(tb, *reinterpret_cast<const h8*>(VT + vt32(col, grp)), z4);
              const f4 ws = mfma16(tw, KSb[ct], z4);
              Vn[ct][ti] = u - ws;
            }
          }
        }
        // o = e^gc (q^ S) + scores V_new
        {
          h8 Vb[2];
#pragma unroll
          for (int ct = 0; ct < 2; ct++) Vb[ct] = pack_b(Vn[ct][0], Vn[ct][1]);
#pragma unroll
          for (int ti = 0; ti < 2; ti++) {
            const f4 eg = lds4(&st.eg[16 * ti + 4 * grp]);
            const h8 at = perm_a_sw<sq_at>(st.Att, 16 * ti + c16, 0, grp);
#pragma unroll
            for (int ct = 0; ct < 2; ct++) O[ct][ti] = mfma16(at, Vb[ct], O[ct][ti] * eg);
          }
        }
        if (m == kC) {
          // rows of V_new scaled by e^(gc_31 - gc_t), then S <- e^gc_31 S + k^T (scaled V_new)
          h8 Vd[2];
#pragma unroll
          for (int ti = 0; ti < 2; ti++) {
            const f4 ed = lds4(&st.ed[16 * ti + 4 * grp]);
#pragma unroll
            for (int ct = 0; ct < 2; ct++) Vn[ct][ti] *= ed;
          }
#pragma unroll
          for (int ct = 0; ct < 2; ct++) Vd[ct] = pack_b(Vn[ct][0], Vn[ct][1]);
          const float el = st.eg[kC - 1];
#pragma unroll
          for (int it = 0; it < 8; it++) {
            const h4 lo = kT_piece(st.Ks, 0, 16 * it, grp, c16), hi = kT_piece(st.Ks, 16, 16 * it, grp, c16);
            const h8 k = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
            for (int ct = 0; ct < 2; ct++) S[ct][it] = mfma16(k, Vd[ct], S[ct][it] * el);
          }
        }
        // O (D layout) -> the output rows; this wave's gated-norm partial sums over its 32 columns
#pragma unroll
        for (int ti = 0; ti < 2; ti++)
#pragma unroll
          for (int ct = 0; ct < 2; ct++)
#pragma unroll
            for (int e = 0; e < 4; e++) osg[(16 * ti + 4 * grp + e) * kOP + 32 * w + 16 * ct + c16] = O[ct][ti][e];
        if (a.gnorm) {
          wave_sync();
          const int er = lane >> 3, ec = 32 * w + 4 * (lane & 7);
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const f4 y = lds4(&osg[(8 * q + er) * kOP + ec]);
            const float sq = sum8((y[0] * y[0] + y[1] * y[1]) + (y[2] * y[2] + y[3] * y[3]));
            if ((lane & 7) == 0) sm.red[p & 1][(8 * q + er) * 4 + w] = sq;
          }
        }
      }
    } else {
      // the rows loaded during the previous period (their loads had that period and its barrier to land)
      seen = max(seen, ahead);
#pragma unroll
      for (int r = 0; r < kKC + 7; r++)
#pragma unroll
        for (int c = 0; c < 2; c++) xv[r][c] = xn[r][c];
#pragma unroll
      for (int q = 0; q < 4; q++) zq[q] = zn[q];
      // the tile set's DMA first, so that it lands behind this period's work; then exactly kAfterDma loads, none of
      // them conditional (z too: its columns exist with or without the gated norm), which the period's end does not
      // wait for
      if (p + 1 < n) dma_set(p + 1, hw);
      asm volatile("" ::: "memory");  // the loads below stay behind the DMA, in the compiler and the scheduler
      __builtin_amdgcn_sched_barrier(0);
      fetch_v(c0 + 2 * kC);
      fetch_z(c0);
      ahead = ld_counter(produced);  // for the next period's check
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      {
        // chunk p - 1's gated norm and store, and chunk p + 1's v conv, without branches so that the compiler can
        // interleave the two chains: in period 0 the norm works on unused LDS and every row is masked, past the last
        // chunk the conv writes a v^T buffer no state wave reads. Rows outside the call get a buffer offset past the
        // sequence's output rows, and the hardware drops those stores.
        const int cp = c0 - kC, mp = min(kC, end - cp), fr = ht0 >> 3, fc = 4 * (ht0 & 7);
        const float* osg = sm.osg[(p - 1) & 1];
        f4 y[4];
#pragma unroll
        for (int q = 0; q < 4; q++) y[q] = lds4(&osg[fr * kOP + fc + 32 * q]);
        if (a.gnorm) {
          const f4 r = lds4(&sm.red[(p - 1) & 1][fr * 4]);
          const float iv = rsqrtf(((r[0] + r[1]) + (r[2] + r[3])) / kDV + 1e-6f);
#pragma unroll
          for (int q = 0; q < 4; q++)
#pragma unroll
            for (int c = 0; c < 4; c++) y[q][c] = y[q][c] * iv * (gw[q][c] * silu(zq[q][c]));
        }
        const bool live = fr < mp && cp + fr >= a.P;
        const unsigned off = live ? (unsigned)(cp + fr - a.P) * orowb + (unsigned)(h * kDV + fc) * (unsigned)sizeof(T)
                                  : 0x80000000u;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          if constexpr (sizeof(T) == 4) {
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i4v, y[q]), orsrc, off + 128u * q, 0, 0);
          } else {
            const h4 hv = {(_Float16)y[q][0], (_Float16)y[q][1], (_Float16)y[q][2], (_Float16)y[q][3]};
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i2v, hv), orsrc, off + 64u * q, 0, 0);
          }
        }
        vconv(c0 + kC);
      }
      // chunk p + 1's tile set has landed in LDS: at most the kAfterDma loads issued after the DMA (and the stores
      // after them) may still be in flight (vmcnt counts in issue order)
      __builtin_amdgcn_s_waitcnt(kWaitDma);
    }
    __syncthreads();
    if (tid0 == 256 && p + 1 < n) st_counter(consumed, ep + (unsigned)(p + 2));
  };

  // the stored state is the one at s1: the periods before chunk (s1 - s0) / 32 advance it up to there, it is written
  // out, and the rest of the call continues from it (a separate loop, so the store is not inside the periods); one
  // period past the last chunk stores its output
  const int k1 = (s1 - a.s0) / kC;
  int p = 0;
  for (; p < k1; p++) period(p);
  if (state) {
    const int g0 = (tid0 & 63) >> 4, l16 = tid0 & 15;
#pragma unroll
    for (int ct = 0; ct < 2; ct++)
#pragma unroll
      for (int it = 0; it < 8; it++)
#pragma unroll
        for (int e = 0; e < 4; e++)
          gpw<float>(a.S_out)[sbase + (size_t)(16 * it + 4 * g0 + e) * kDV + 32 * w + 16 * ct + l16] = S[ct][it][e];
  }
  for (; p <= n; p++) period(p);
  if (seen == ~0u && (tid0 & 63) == 0) report_wait(a.wait, kErrDuoWait);
}

// Blocks 16 i + r (r < 8, the producer) and 16 i + 8 + r (the consumer) form pair 8 i + r. The dispatcher hands
// consecutive blocks to the XCDs in turn and each XCD takes its blocks in order, so both members of a pair share an
// XCD (and its L2), and the producer comes first. kDebugWaits: the instantiation a test of the wait-failure report
// launches (a.wait.skew != 0), whose consumer waits use a.wait's skew and poll bound.
template <typename T, bool kDebugWaits>
__global__ __launch_bounds__(kThreads) void gdn_duo_kernel(GdnArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  const int blk = blockIdx.x;
  const int pair = (blk >> 4) * 8 + (blk & 7);
  const int b = pair / a.H, h = pair % a.H;
  unsigned* const produced = a.sync_flags + (size_t)pair * 64;  // each counter on its own 128-byte line
  unsigned* const consumed = produced + 32;
  char* const ring = (char*)a.duo_ring + (size_t)pair * a.duo_slots * kDuoSetBytes;
  const unsigned ep = a.sync_epoch << kDuoEpochShift;
  if ((blk >> 3) & 1)
    consume<T, kDebugWaits>(a, b, h, *reinterpret_cast<ConsumerLds*>(lds_raw), ring, produced, consumed, ep);
  else
    produce<T>(a, b, h, *reinterpret_cast<ProducerLds*>(lds_raw), ring, produced, consumed, ep);
}

template <typename T>
hipError_t launch(const GdnArgs& a, hipStream_t s) {
  auto k = a.wait.skew ? gdn_duo_kernel<T, true> : gdn_duo_kernel<T, false>;
  const int lds = (int)(sizeof(ConsumerLds) > sizeof(ProducerLds) ? sizeof(ConsumerLds) : sizeof(ProducerLds));
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k, dim3(2 * a.B * a.H), dim3(kThreads), (unsigned)lds, s, a);
  return hipGetLastError();
}

}  // namespace

bool gdn_duo_fits(int B, int H) { return (B * H) % 8 == 0 && 2 * B * H <= 256; }

hipError_t launch_gdn_duo(const GdnArgs& a, hipStream_t s) {
  if (a.DK != kDK || a.DV != kDV || a.KC != kKC) return hipErrorInvalidValue;
  if (a.P - a.s0 >= 64 || a.P < a.s0) return hipErrorInvalidValue;  // at most one open 64-row span is replayed
  if (!gdn_duo_fits(a.B, a.H) || !a.duo_ring || !a.sync_flags) return hipErrorInvalidValue;
  const int n = (a.P + a.L - a.s0 + kC - 1) / kC;  // chunks of the call: one slot each, and the counters' chunk field
  if (n > a.duo_slots || n + 2 >= (1 << kDuoEpochShift) || a.sync_epoch >= (1u << (32 - kDuoEpochShift)))
    return hipErrorInvalidValue;
  return a.dtype == 0 ? launch<float>(a, s) : launch<_Float16>(a, s);
}

}  // namespace ha
