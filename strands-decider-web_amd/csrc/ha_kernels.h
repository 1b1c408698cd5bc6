// Kernel argument blocks and launchers shared by the engine host code and the HIP kernels (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace ha {

// Cross-workgroup waits of one launch (the paired form's tile-set wait, the split form's packed-state wait, the split
// GQA merge's wait for its pieces) are bounded: a workgroup polls at most `polls` times (about a microsecond each).
// Every waited-for value is published by a workgroup that is resident or done, so in a correct launch a wait always
// ends early. If one runs out anyway, the workgroup goes on (so the launch still ends), and stores its bit into
// `*err`, a word in host-visible memory the engine checks after its next stream synchronisation and at its next
// call, which then fail with HA_ERR_DEVICE.
// `skew` is 0 except in tests of this path: a launch given a non-zero skew waits for values no workgroup of it ever
// publishes (its waits give up after `polls` polls each, its outputs are undefined, every kernel still ends).
constexpr unsigned kErrDuoWait = 1u;    // paired form: a consumer gave up waiting for a tile set
constexpr unsigned kErrSplitWait = 2u;  // split form: an output workgroup gave up waiting for a packed state
constexpr unsigned kErrGqaMerge = 4u;   // split-key GQA: a merge workgroup gave up waiting for its pieces
constexpr int kWaitPolls = 1 << 16;
struct WaitCheck {
  unsigned* err = nullptr;  // host-visible error word (system-scope stores), or nullptr
  unsigned skew = 0;
  int polls = kWaitPolls;
};

// One gated-delta layer over absolute rows [s0, P + L) of `B` sequences.
// Rows r < P come from `tail` (raw rows kept by the previous call: [s0 - (KC-1), P)), rows >= P from `in`.
// The conv of row r reads rows r-3..r, so rows s0-3..s0-1 must be present in `tail` (zeros at the start of a
// sequence). Rows below P are replayed (state only, no output).
struct GdnArgs {
  int B, H, DK, DV, KC, stride, C;  // C = 2*H*DK + H*DV; a at C + H*DV, b at C + H*DV + H, z at C
  int P, L, s0;                     // state position, cached rows, new rows
  int tail_cap;                     // rows per sequence in `tail`
  int dtype;                        // 0 f32 rows/out, 1 f16
  const void* in;                   // [B][L][stride]
  const void* tail;                 // [B][tail_cap][stride]
  void* out;                        // [B][L][H*DV]
  const float* S_in;                // [B][H][DK][DV] state at s0, or nullptr for a zero state
  float* S_out;                     // [B][H][DK][DV] state at the returned position (may equal S_in)
  const float* conv_w;              // [C][KC]
  const float* negA;                // [H]
  const float* dtb;                 // [H]
  const float* gnorm;               // [DV], or nullptr to output the raw core output
  void* img;                        // chunk scratch of the split form: [B][H][img_chunks] images
  int img_chunks;                   // image slots per (sequence, head)
  float* seq_raw;                   // sequential form: raw outputs [B][H][kSegRows][DV] fp32 awaiting the gated norm
  unsigned* seq_cnt;                // sequential form: [B][H] arrival counters (zero between launches)
  void* duo_ring;                   // paired form: [B*H][duo_slots] tile-set slots of kDuoSetBytes, one per chunk
  int duo_slots;                    // paired form: slots per (sequence, head), at least the call's 32-row chunks
  unsigned* sync_flags;             // [B*H][64] progress counters between workgroups of one launch: paired form (produced
                                    // at 0, consumed at 32), split form (the state pass's workgroup g at 16 g)
  unsigned sync_epoch;              // this launch's counter epoch, >= 1 and increasing per flag buffer
  WaitCheck wait;                   // bounded cross-workgroup waits: poll limit, test skew, error word
};
constexpr int kSegRows = 64;        // output rows per launch of the sequential form
constexpr int kDuoSetBytes = 23 * 1024;   // bytes per tile-set slot of the paired form
constexpr int kDuoEpochShift = 12;        // progress counter value: epoch << kDuoEpochShift | chunks (< 4096)

// Full-attention prep (q/k RMSNorm, partial RoPE, K/V cache write) and attention for rows [P, P + L).
struct GqaArgs {
  int B, HQ, HK, HD, RD, stride, LT;
  int P, L;
  int dtype;                 // rows / out dtype: 0 f32, 1 f16
  const void* in;            // [B][L][stride]
  void* out;                 // [B][L][HQ*HD]
  const float* qw;           // [HD] stored (1 + w)
  const float* kw;           // [HD]
  const float* rope;         // [LT][RD] cos/sin pairs
  _Float16* K;               // [B][HK][LT][HD] cache, row-major
  _Float16* V;               // [B][HK][HD][LT] cache, transposed (positions contiguous)
  // Split key ranges: with split > 0, the keys of a query block are processed in pieces of `split` 64-key tiles
  // at absolute tile boundaries, by separate workgroups; a block with more than one piece writes per-piece partial
  // results to `part` (part_slots slots), marks the slot with `epoch`, and merge workgroups of the same launch
  // combine them. 0: one workgroup per block.
  int split;
  int part_slots;
  float* part;               // [slots][4][64][HD] unnormalised O, then [slots][4][64][2] (reference max, sum), then
                             // [slots] u32 epoch marks
  unsigned epoch;            // this launch's mark, >= 1 and different from every earlier launch's on `part`
  WaitCheck wait;            // the merge workgroups' bounded wait for their pieces
};

// Slots of partial results the split GQA path needs for any call on a context of at most max_ctx positions.
size_t gqa_part_slots(int pairs, int max_ctx, int split);
size_t gqa_part_slot_bytes();

// Copy the raw rows [dst_first, P + L) (dst_first >= s0 - (KC-1)) of every sequence from (tail, in) into
// `tail_out` ([B][tail_cap][stride]); only the conv channels [0, C) and the a/b columns are kept.
constexpr int kTailLayers = 32;  // gated-delta layers whose raw-row tails one launch updates
struct TailArgs {
  int B, stride, C, ab_off, ab_n;
  int P, L, s0, KC, tail_cap_in, tail_cap_out, dst_first, dtype;
  int n;                          // layers in this launch, 1..kTailLayers
  const void* in[kTailLayers];    // per layer: the call's input rows, [B][L][stride]
  const void* tail[kTailLayers];  // per layer: the raw-row tail the call resumed from, [B][tail_cap_in][stride]
  void* tail_out[kTailLayers];    // per layer: the working raw-row tail, [B][tail_cap_out][stride]
};

hipError_t launch_gdn_sequential(const GdnArgs& a, hipStream_t s);
hipError_t launch_gdn_chunked(const GdnArgs& a, hipStream_t s);
// paired form: a producer and a consumer workgroup per (sequence, head), 2*B*H workgroups
bool gdn_duo_fits(int B, int H);
hipError_t launch_gdn_duo(const GdnArgs& a, hipStream_t s);
hipError_t launch_gdn_split(const GdnArgs& a, hipStream_t s);  // chunk-parallel preparation, state pass, outputs
size_t gdn_split_image_bytes();                                // scratch bytes of one chunk
hipError_t launch_gqa(const GqaArgs& a, hipStream_t s);

// MatMulNBits projection: y[M][N] (f16) = a[M][K] (f16) x W^T, W in packed blocks of 32 (`bits` u32 words each) with
// one f16 scale (and, asymmetric, one f16 bias) per `group` values of a row.
struct MnbArgs {
  int M, N, K, bits, group, asym;
  const void* a;  // [M][K] f16
  void* y;        // [M][N] f16
  const void* q;  // [N][K/32][bits] u32
  const void* s;  // [N][K/group] f16
  const void* b;  // [N][K/group] f16 (asymmetric only)
  int split = 1;     // GEMM only: K ranges, each on its own workgroups, summed in order by a second kernel
  float* ws = nullptr;  // [split][M][N] fp32 partial products when split > 1
};
hipError_t mnb_check(const MnbArgs& a);
bool mnb_packed_path(int M, int N, int K);  // whether launch_mnb_gemv (packed weights) serves M rows
hipError_t launch_mnb_gemv(const MnbArgs& a, hipStream_t s);  // M <= 64 (mnb_packed_path picks up to 48)
int mnb_gemm_split(int M, int N, int K);  // K ranges the GEMM uses for this shape (1: none, no workspace)
hipError_t launch_mnb_gemm(const MnbArgs& a, hipStream_t s);  // any M: tiled GEMM, weights dequantised into LDS
// Scratch of the allocation-free GEMM entry point (mnb.hip): a file-scope device array of kMnbScratchBytes per GPU.
// mnb_scratch_setup looks its address up on `device`, which must be current, once per device; mnb_scratch returns
// that address (nullptr before the set-up).
constexpr size_t kMnbScratchBytes = size_t(40) << 20;
hipError_t mnb_scratch_setup(int device);
float* mnb_scratch(int device);
hipError_t launch_fwht(void* x, long elems, int n, hipStream_t s);
hipError_t launch_tail_update(const TailArgs& a, hipStream_t s);

// Torso ops around the mixers and projections (torso.hip).
struct EmbedArgs {
  int L, D, rows, bits, group, asym;  // rows: rows of the quantised table (ids >= rows give a NaN row)
  const unsigned* ids;                // [L] device
  const unsigned* q;                  // [rows][D/32][bits]
  const _Float16* s;                  // [rows][D/group]
  const _Float16* b;                  // asymmetric only
  float* x;                           // [L][D] f32
};
struct AddNormArgs {
  int R, D, nx;           // output rows, width, rows of x (a gather index >= nx gives a NaN output row)
  float* x;               // [nx][D] f32 residual stream (updated in place when y is given)
  const _Float16* y;      // [nx][D] f16 or NULL (no residual add)
  const float* w;         // [D] norm weight (already 1 + w where the model says so)
  void* h;                // [R][D] f16, or f32 with out_f32
  const unsigned* rows;   // [R] source rows, or NULL for the identity
  int out_f32;
  float eps;
};
hipError_t launch_embed(const EmbedArgs& a, hipStream_t s);
hipError_t launch_add_norm(const AddNormArgs& a, hipStream_t s);
hipError_t launch_silu_mul(const void* big, void* mid, int L, int I, hipStream_t s);
hipError_t launch_add_bias(void* y, const float* c, int L, int N, hipStream_t s);

constexpr int kChunk = 64;  // gated-delta chunk length; chunk boundaries sit at s0 + 64k

}  // namespace ha
