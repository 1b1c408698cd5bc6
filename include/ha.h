/*
 * ha.h: C ABI of the MI355X hybrid-attention engine (gated-delta + gated causal GQA token mixers with
 * prefix-cache snapshot/resume), the drop-in replacement for the hot path of the reference's WebGPU engine.
 *
 * Reference interface replaced (paths relative to the reference repository):
 *   Engine constructor state and buffers      web/public/engine/engine.js:89-111
 *   the linear_attention / full_attention
 *     branches of Engine.plan()               web/public/engine/engine.js:253-276
 *   Engine.forward({cache, keepCache,
 *     timestamps}) incl. resume and snapshot  web/public/engine/engine.js:313-375
 *   snapshot.release()                        web/public/engine/engine.js:361
 *   manifest config + per-layer tensors       convert/export_engine.py:46-65,83
 *
 * Conventions
 *   - Every function returns HA_OK (0) or a negative ha_status; ha_last_error() then returns a message for the
 *     calling thread. The Node binding turns a non-zero status into a thrown Error, as the reference throws.
 *   - All tensor arguments of ha_forward are DEVICE pointers (HBM). ha_device_alloc / ha_copy_* are provided for
 *     callers without their own allocator.
 *   - One engine is bound to one HIP stream; calls on one engine must not overlap (the reference is not
 *     re-entrant either and its worker serialises calls, web/public/js/worker.js:249-253).
 *   - A snapshot is only valid with the engine that made it.
 */
#ifndef HA_H
#define HA_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HA_ABI_VERSION 2

typedef struct ha_engine ha_engine;
typedef struct ha_snapshot ha_snapshot;

typedef enum ha_status {
  HA_OK = 0,
  HA_ERR_ARG = -1,      /* bad argument, shape or config */
  HA_ERR_CONTEXT = -2,  /* P + L exceeds max_ctx (engine.js:316 "context ... exceeds") */
  HA_ERR_HANDLE = -3,   /* invalid, foreign or released engine / snapshot handle */
  HA_ERR_DEVICE = -4,   /* a HIP runtime call failed, or a kernel of an earlier call reported a bounded wait
                           that ran out (engine.js:373 throws the device errors a forward collected) */
  HA_ERR_NOMEM = -5,    /* device or host allocation failed */
  HA_ERR_PARAM = -6     /* unknown tensor name or wrong element count (engine.js:177 "no tensor ...") */
} ha_status;

typedef enum ha_layer_kind {
  HA_LINEAR_ATTENTION = 0, /* manifest layer_types "linear_attention" */
  HA_FULL_ATTENTION = 1,   /* manifest layer_types "full_attention" */
  HA_ADAPTER = 2           /* manifest layer_types "adapter": a projection + bias stand-in with no token mixer
                              (engine.js:256-261); the engine keeps no state for it and ha_forward skips it, so its
                              layer_in / layer_out entries may be NULL */
} ha_layer_kind;

typedef enum ha_dtype { HA_F32 = 0, HA_F16 = 1 } ha_dtype;

typedef enum ha_recurrence {
  HA_CHUNKED = 0,        /* prefill form: chunks at absolute positions, MFMA products, the state stored at the last
                            64-row boundary (default; the engine picks one of the implementations below from its batch
                            and head count B*H: the split form up to 32, the paired form for a multiple of 8 up to 128,
                            the fused kernel beyond) */
  HA_SEQUENTIAL = 1,     /* token-by-token fp32 rule with the state in registers (decode / resume) */
  HA_CHUNKED_FUSED = 2,  /* the chunked form in one kernel per layer: one workgroup per (sequence, head), 64-row chunks */
  HA_CHUNKED_SPLIT = 3,  /* the chunked form in two launches, 64-row chunks: every chunk's state-independent part at
                            once, then the state alone through the chunks (four workgroups per (sequence, head))
                            with every chunk's outputs on the other CUs as soon as its state is known */
  HA_CHUNKED_PAIRED = 4  /* the chunked form on two workgroups per (sequence, head), 32-row chunks: one prepares the
                            chunks' tiles, the other runs the recurrence (B*H a multiple of 8, at most 128) */
} ha_recurrence;

/* Engine shape. Field names follow the manifest config keys (export_engine.py:83). */
typedef struct ha_config {
  int n_layers;
  const unsigned char* layer_kind; /* [n_layers] ha_layer_kind */
  int batch;                       /* independent sequences per forward (the reference is batch 1) */
  int max_ctx;                     /* LT, K/V cache rows per sequence (engine.js:92: 4096) */
  /* gated-delta layers: linear_num_key_heads (= value heads), linear_key_head_dim, linear_value_head_dim,
     linear_conv_kernel_dim */
  int H, DK, DV, conv_k;
  int lin_stride;   /* row stride (elements) of the fused in_proj rows qkv | z | a | b (8256 in the engine); a
                       multiple of 8, so every head's 128-channel row segment is 16-byte aligned */
  int lin_dtype;    /* ha_dtype of linear-layer input rows and outputs */
  int lin_gnorm;    /* 1: output the gated RMSNorm (GNORM, the engine's layer output); 0: the raw core output */
  /* full-attention layers: num_attention_heads, num_key_value_heads, head_dim, rotary_dim */
  int HQ, HK, HD, rot_dim;
  int full_stride;  /* row stride of the fused qkv rows [q|gate] x HQ | k x HK | v x HK (5120) */
  int full_dtype;   /* ha_dtype of full-layer input rows and outputs; the K/V cache is f16 */
  float rope_theta; /* 1e7 */
  float eps;        /* rms_norm_eps; must be 1e-6, the value the reference kernels hard-code */
} ha_config;

/* Per-call options of ha_forward (engine.js:313 options). NULL means all defaults (zeros). */
typedef struct ha_forward_opts {
  int recurrence;  /* ha_recurrence for the gated-delta layers */
  int timestamps;  /* 1: time the whole forward with HIP events; result in gpu_ms (engine.js:331-348) */
  int sync;        /* 1: wait for the stream before returning */
  float gpu_ms;    /* out: forward time when timestamps = 1 (implies a wait) */
  float* layer_ms; /* optional out [n_layers]: per-layer GPU ms (the reference's profile(), engine.js:292-307),
                      each gated-delta layer's raw-row tail copy included */
  float* mixer_ms; /* optional out [n_layers]: GPU ms of each layer's token-mixer kernels alone (without the tail
                      copy; 0 for adapter layers). No counterpart in the reference: the kernel time a roofline is
                      computed on. Implies a wait, like layer_ms */
  int debug_unpublished_waits; /* test only, 0 otherwise. No counterpart in the reference. 1: every bounded
                      cross-workgroup wait of this call (the paired form's tile-set wait, the split form's
                      packed-state wait, the split-key attention merge) waits for a value no workgroup of it
                      publishes, for a few polls each, then goes on; every kernel still ends, the outputs are
                      undefined, and the failure is reported as HA_ERR_DEVICE (exercises that path from the host) */
} ha_forward_opts;

const char* ha_last_error(void);
int ha_abi_version(void);
/* The architecture name of HIP device `device` ("gfx950"), into name[bytes]: what the reference's adapter guard
   engineProblems(adapter) inspects (engine.js:50-52); every kernel here is built for gfx950 only. HA_ERR_DEVICE when
   no HIP device is visible. */
int ha_device_arch(int device, char* name, size_t bytes);

/* Engine.create / constructor (engine.js:63-111): validates the config, allocates the working state, history
   and K/V buffers and the RoPE table on HIP device `device`, and creates the engine's stream. */
int ha_create(const ha_config* cfg, int device, ha_engine** out);
int ha_destroy(ha_engine* e);

/* Bind the engine to an existing HIP stream (hipStream_t passed as void*), e.g. a framework's current stream.
   NULL rebinds the engine's own stream. An engine that shares its call-time buffers with other engines
   (ha_share_scratch) and moves to a different stream first gets a set of its own again (waiting for the device),
   so that engines holding one set always run on one stream. */
int ha_set_stream(ha_engine* e, void* stream);
/* Let engine e use the call-time device buffers of `holder` (chunk images, the sequential form's raw outputs and
   counters, split-GQA partials, the zero history), growing them to what e's shape needs, and free e's own set once
   nothing else holds it. For the per-layer engines of one torso on one stream: their calls then run one after
   another and one set serves all of them. Both engines must already run on one stream (HA_ERR_ARG otherwise), and
   ha_set_stream keeps it so. The set lives until the last engine holding it is destroyed. No counterpart in the
   reference, whose engine holds one set of buffers for all its layers (engine.js:89-107). Waits for the device to
   finish queued work. */
int ha_share_scratch(ha_engine* e, ha_engine* holder);
/* The stream the engine's calls run on (hipStream_t as void*): for a host that queues its own work, such as the
   projection matmuls (ha_mnb_forward), in order with the token mixers. No counterpart in the reference, whose
   WebGPU queue is implicit (engine.js:236-246 records everything into one command encoder). */
int ha_get_stream(ha_engine* e, void** stream);

/* Upload one per-layer tensor under its manifest name (export_engine.py:55-58,64-65), as f32 host data:
     linear layers: "conv" [C][conv_k] with C = 2*H*DK + H*DV, "neg_exp_A" [H], "dt_bias" [H], "gnorm" [DV]
     full layers:   "q_norm" [HD], "k_norm" [HD] (stored as 1 + w, as the manifest stores them)
   count is the number of floats. Unset tensors default to zeros (conv, neg_exp_A, dt_bias) or ones (norms). */
int ha_set_param(ha_engine* e, int layer, const char* name, const float* host, size_t count);

/* One forward over L new rows per sequence (engine.js:313-375, token-mixer part).
     layer_in[i]:  [batch][L][lin_stride] (linear) or [batch][L][full_stride] (full) rows in that kind's dtype
     layer_out[i]: [batch][L][H*DV] or [batch][L][HQ*HD] in that kind's dtype
   resume: continue from this snapshot (engine.js:325-327); NULL starts from an empty context. Its GQA K/V rows are
           copied back into the engine's working caches unless the engine knows they are still there (a completed
           call resumed from it or kept it, and no later call wrote below its P or copied another snapshot in)
   keep:   if non-NULL, receives a new snapshot of the context after this call (engine.js:349-362)
   Returns HA_ERR_CONTEXT if P + L > max_ctx. Layers run in order on the engine's stream. No layer_out buffer may
   overlap any layer_in buffer of the same call: the gated-delta layers' raw rows (conv history and replay rows) are
   copied from layer_in after all layers have run.
   Device errors: the kernels' cross-workgroup waits are bounded; a wait that runs out (never in a correct launch)
   lets its kernel end and marks the engine's error word. The call that synchronises (sync, timestamps, layer_ms,
   mixer_ms), the next ha_forward, ha_synchronize and ha_copy_to_host then return HA_ERR_DEVICE once, and no
   snapshot of the failed call is kept. */
int ha_forward(ha_engine* e, int L, const void* const* layer_in, void* const* layer_out, const ha_snapshot* resume,
               ha_snapshot** keep, ha_forward_opts* opts);

/* Snapshot queries. P is the number of tokens the snapshot covers (engine.js:352 snap.P). Every snapshot entry point
   looks the handle up among the live snapshots first: a destroyed or forged handle gives HA_ERR_HANDLE. */
int ha_snapshot_tokens(const ha_snapshot* s, int* P);
/* Position of the stored recurrent state (a multiple of 64 after chunked forwards, P after sequential ones) and
   the number of raw rows kept for replay and conv history, [state_pos - (conv_k-1), P). */
int ha_snapshot_layout(const ha_snapshot* s, int* state_pos, int* tail_rows);
/* Copy one part of a snapshot to host memory (linear layers: "state", "state_stored", "tail"; full layers: "K",
   "V"):
     "state"        f32 [batch][H][DK][DV]: the recurrent state after all P tokens, as the reference's snapshot holds
                    it (engine.js:352-356). When the stored state sits at an earlier chunk boundary (state_pos < P),
                    it is advanced over the replay rows [state_pos, P) with the sequential fp32 rule for this read
                    (a resume replays those rows in the chunked form instead, so that prefix + suffix stays
                    bit-identical to one forward; the two agree within the recurrence tolerance)
     "state_stored" f32 [batch][H][DK][DV]: the stored state at state_pos (what a resume starts from)
     "tail"         [batch][tail_rows][lin_stride] in lin_dtype: the raw rows [state_pos - (conv_k-1), P)
     "K" / "V"      f16 [batch][HK][P][HD]. */
int ha_snapshot_read(const ha_snapshot* s, int layer, const char* what, void* host, size_t bytes);
/* Free the snapshot's device memory (snapshot.release(), engine.js:361). Idempotent. */
int ha_snapshot_release(ha_snapshot* s);
/* Release (if needed) and free the handle itself. */
int ha_snapshot_destroy(ha_snapshot* s);

/* Device memory helpers for callers without their own HIP allocator (the Node binding). */
int ha_device_alloc(ha_engine* e, size_t bytes, void** dptr);
int ha_device_free(ha_engine* e, void* dptr);
int ha_copy_to_device(ha_engine* e, void* dst, const void* host, size_t bytes);
int ha_copy_to_host(ha_engine* e, void* host, const void* src, size_t bytes);
/* Wait for the engine's stream; HA_ERR_DEVICE if a kernel of an earlier call reported a wait that ran out. */
int ha_synchronize(ha_engine* e);

/* ---- MatMulNBits projections: the matmuls either side of the path ----
   Weight formats of web/public/gemmbench/kernels.js:1-14: blocks of 32 consecutive k of one output row n, `bits`
   u32 words each ([N][K/32][bits]); 4 bits = MatMulNBits (element 2i in the low nibble of byte i, zero point 8),
   2 bits = element e at bits 2(e%16) of word e/16, 3 bits = 2-bit low words plus a word of high bits. One f16 scale
   per `group` (32 or 64) values of a row ([N][K/group]); symmetric w = (q - 2^(bits-1)) * scale, asymmetric
   w = q * scale + bias with an f16 bias of the same shape. convert/export_engine.py:17-26 writes int4, group 32,
   symmetric. */
typedef struct ha_mnb ha_mnb;
typedef struct ha_mnb_format {
  int bits;  /* 2, 3 or 4 */
  int group; /* 32 or 64 */
  int asym;  /* 0 symmetric, 1 per-group bias */
} ha_mnb_format;

/* A quantised weight matrix on HIP device `device`: q, s and (asymmetric) b are device pointers the caller keeps
   alive (the reference's weight storage buffers, engine.js:236-246). K must be a multiple of 32 and of the group;
   a matmul (ha_mnb_forward) also needs N % 16 == 0 (the export pads N to 64), an embedding table (ha_embed) does
   not. */
int ha_mnb_create(int N, int K, const ha_mnb_format* fmt, const void* q, const void* s, const void* b, int device,
                  ha_mnb** out);
/* y[M][N] = a[M][K] x W^T (f16 in and out, fp32 accumulation) on `stream` (hipStream_t as void*, NULL: the null
   stream): the matmul dispatch of engine.js:236-246, kernel chosen by M as engine.js:17-33 does. a and y are device
   pointers (16-byte aligned). Up to 64 rows a GEMV kernel reads the packed weights; above that a tiled MFMA GEMM
   dequantises weight tiles into LDS. With few output tiles it splits K over workgroups, using a workspace the
   handle owns (grown on demand, at most 64 MiB), so calls on one handle must be ordered. */
int ha_mnb_forward(ha_mnb* w, int M, const void* a, void* y, void* stream);
/* No counterpart in the reference. ha_mnb_forward for callers that cannot allocate device memory (code under HIP
   graph capture, serving loops or harnesses that forbid hipMalloc): the same kernels, K split and results, but a
   split product's fp32 partials go to a fixed scratch array inside the library (HA_MNB_SCRATCH_BYTES per GPU, held
   until the process ends) instead of the handle's on-demand workspace. It allocates nothing. The partials take
   split x M x N x 4 bytes; K is split only when there are fewer than 256 output tiles of 128 x 128, which keeps
   split x M x N below 638 x 128 x 128, so the scratch fits every shape (the 2B torso's projections need at most
   33 MiB); a shape that did not fit would return HA_ERR_ARG. Every partial is written before it is read, so
   nothing needs clearing. All calls
   on one GPU share its scratch array and it keeps the last call's contents: calls that overlap on one GPU (other
   streams, other threads) race, so order them on one stream. */
#define HA_MNB_SCRATCH_BYTES (40u << 20)
int ha_mnb_forward_noalloc(ha_mnb* w, int M, const void* a, void* y, void* stream);
int ha_mnb_destroy(ha_mnb* w);
/* In-place orthonormal Walsh-Hadamard transform of every contiguous n-block of the f16 array x (elems values, a
   multiple of n; n a power of two up to 8192): the online input rotation of a tensor exported with `had: n`
   (FWHT, web/public/engine/wgsl.js:94-110; applied before the matmul at engine.js:240). */
int ha_fwht(void* x, long elems, int n, int device, void* stream);

/* ---- The rest of the torso forward (web/public/engine/engine.js:247-284): all device pointers, all on `stream`
   (hipStream_t as void*, NULL: the null stream), on HIP device `device`. */

/* x[t][0..K) = f32 row ids[t] of the quantised embedding table held by `table` (a MatMulNBits handle with N = table
   rows, K = hidden size; EMBED, web/public/engine/wgsl.js:33-52): (q - 2^(bits-1)) * scale, or q * scale + bias, in
   f32. ids: L u32 on the device; an id >= N gives a row of NaN. */
int ha_embed(const ha_mnb* table, int L, const void* ids, void* x, void* stream);

/* Residual add + RMSNorm (ADD_NORM, wgsl.js:55-78): for output row r with source row s = rows[r] (rows NULL: s = r),
   if y != NULL first x[s] += y[s] (f32 += f16, written back), then
   h[r] = x[s] * (mean(x[s]^2) + eps)^-1/2 * w   (w: D f32, already 1 + w where the model says so),
   h f16, or f32 when out_f32 (the final norm, engine.js:283-284, 342). x has nx rows of D (D % 8 == 0, D <= 8192);
   a source row >= nx gives a NaN output row. */
int ha_add_norm(int R, int D, int nx, void* x, const void* y, const float* w, void* h, int out_f32,
                const void* rows, float eps, int device, void* stream);

/* mid[t][j] = silu(big[t][j]) * big[t][I + j] for t < L, j < I (SILU_MUL, wgsl.js:81-90); f16, I % 8 == 0. */
int ha_silu_mul(int L, int I, const void* big, void* mid, int device, void* stream);

/* y[t][j] += c[j] for t < L, j < N (ADD_BIAS, wgsl.js:113-121): y f16, c f32 on the device, N % 8 == 0. */
int ha_add_bias(int L, int N, void* y, const float* c, int device, void* stream);

/* ---- GPU timestamps for diagnostics: the counterpart of the reference's WebGPU timestamp query sets, written at
   compute-pass boundaries and resolved after the submit (engine.js:292-307 profile(), 331-348 timestamps). */
typedef struct ha_timer ha_timer;
/* n timestamps on HIP device `device` (createQuerySet({type: "timestamp", count: n})). */
int ha_timer_create(int device, int n, ha_timer** t);
/* Record timestamp i on `stream` (hipStream_t as void*, NULL: the null stream) after the work queued so far. */
int ha_timer_mark(ha_timer* t, int i, void* stream);
/* Wait for timestamps i and j (both recorded) and give the GPU time from i to j in milliseconds. */
int ha_timer_elapsed(ha_timer* t, int i, int j, float* ms);
int ha_timer_destroy(ha_timer* t);

#ifdef __cplusplus
}
#endif

#endif /* HA_H */
