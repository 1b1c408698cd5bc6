// Host side of the MI355X hybrid-attention engine: the C ABI declared in include/ha.h.
//
// Mirrors the reference engine's host logic for the token mixers (web/public/engine/engine.js):
//   constructor buffers (engine.js:89-107)        -> ha_create: per-layer state, raw-row tail, K/V cache, RoPE table
//   plan() linear / full branches (253-276)       -> ha_forward: layer-kind dispatch, one stream, layers in order
//   forward() resume (325-328)                    -> the snapshot's state / tail feed the kernels; K/V rows copied
//   forward() snapshot (349-362)                  -> ha_forward(keep): new device buffers sized to the context
//   context guard (316), missing tensor (177)     -> HA_ERR_CONTEXT, HA_ERR_PARAM
//
// Gated-delta layers keep, instead of the reference's 3-row conv history, the raw rows from 3 before the stored
// state position up to P. The stored state sits at the last chunk boundary (chunked forwards) so that a resumed
// call replays the rows of the open chunk with exactly the arithmetic a single full forward would use; this makes
// prefix + suffix bit-identical to one forward for any split.
#include <algorithm>
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_set>
#include <vector>

#include "ha.h"
#include "ha_kernels.h"

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

#define HA_HIP(expr)                                                                          \
  do {                                                                                        \
    hipError_t e_ = (expr);                                                                   \
    if (e_ != hipSuccess) return fail(HA_ERR_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)

constexpr uint32_t kEngineMagic = 0x4841454eu, kSnapMagic = 0x48415350u, kDeadMagic = 0xdeadbeefu;
constexpr int kKC = 4;                          // conv kernel the kernels are built for
constexpr int kTailCap = ha::kChunk - 1 + kKC;  // at most 63 open rows + 3 history rows (+1 spare)
std::atomic<uint64_t> g_engine_ids{1};
std::atomic<uint64_t> g_snap_uid{0};  // snapshot uids: 1, 2, ...
// Engines that exist right now. Handle checks look a pointer up here before reading through it, so a snapshot
// outliving its engine (any order of release is allowed, e.g. under a garbage collector) never touches freed memory.
std::mutex g_live_mu;
std::unordered_set<const ha_engine*> g_live;
// Snapshot handles that exist (created and not yet destroyed): every snapshot entry point looks a handle up here
// before reading through it, so a destroyed handle is refused instead of read after it was freed.
std::unordered_set<const ha_snapshot*> g_live_snaps;
std::unordered_set<const void*> g_live_mnbs;  // MatMulNBits handles, likewise
std::unordered_set<const void*> g_live_timers;  // timestamp sets, likewise
constexpr uint32_t kTimerMagic = 0x48415449u;

struct Layer {
  int kind = 0;
  float* conv = nullptr;
  float* negA = nullptr;
  float* dtb = nullptr;
  float* gnorm = nullptr;
  float* qn = nullptr;
  float* kn = nullptr;
  float* S = nullptr;     // [B][H][DK][DV] working state
  void* tail = nullptr;   // [B][kTailCap][lin_stride] working raw-row tail
  _Float16* K = nullptr;  // [B][HK][LT][HD]
  _Float16* V = nullptr;  // [B][HK][HD][LT] (transposed: positions contiguous)
};

size_t dtype_size(int dt) { return dt == HA_F16 ? 2 : 4; }

// Device memory an engine's kernels use only inside a call: the split form's chunk images, the sequential
// form's raw outputs and per-head arrival counters (zero between calls), split-GQA partial results, and the zero
// history of an empty context. Engines whose calls never overlap may hold one set between them (ha_share_scratch);
// it is freed with the last engine holding it. Every buffer only has to be large enough for each holder's shape.
struct Scratch {
  struct Buf {
    void* p = nullptr;
    size_t bytes = 0;
  };
  int device = 0;
  Buf img, seq_raw, seq_cnt, gqa_part, zeros, duo_ring, sync_flags;
  unsigned sync_epoch = 0;  // the progress counters' epoch of the last launch that used them (they start at zero)
  unsigned gqa_epoch = 0;   // the split-GQA slot marks' epoch of the last launch (the marks start at zero)
  // the engines holding this set (guarded by g_live_mu); all of them run on one stream, so their calls never overlap
  std::vector<const ha_engine*> holders;
  ~Scratch() {
    (void)hipSetDevice(device);
    for (Buf* b : {&img, &seq_raw, &seq_cnt, &gqa_part, &zeros, &duo_ring, &sync_flags})
      if (b->p) (void)hipFree(b->p);
  }
};

// Makes b hold at least `bytes`, zero-filled when a larger buffer replaces it. A buffer is only replaced after the
// device has finished every queued call, since a call of any engine holding the set may still read the old one.
int grow(Scratch::Buf& b, size_t bytes) {
  if (bytes <= b.bytes) return HA_OK;
  void* p = nullptr;
  hipError_t he = hipMalloc(&p, bytes);
  if (he != hipSuccess) return fail(HA_ERR_NOMEM, std::string("hipMalloc: ") + hipGetErrorString(he));
  if ((he = hipMemset(p, 0, bytes)) != hipSuccess || (he = hipDeviceSynchronize()) != hipSuccess) {
    (void)hipFree(p);
    return fail(HA_ERR_DEVICE, std::string("scratch set-up: ") + hipGetErrorString(he));
  }
  if (b.p) (void)hipFree(b.p);
  b.p = p;
  b.bytes = bytes;
  return HA_OK;
}

}  // namespace

struct ha_engine {
  uint32_t magic = kEngineMagic;
  uint64_t id = 0;
  // snapshots (by uid) whose K/V rows [0, rows) the working caches are known to hold (uid 0: empty entry). A call
  // from position P writes only rows from P on, so it keeps the entries with rows <= P and adds the snapshot it
  // resumed from (P rows) and the one it kept (P + L rows); the list is cleared while a call runs
  static constexpr int kKvHeld = 8;
  struct KvHeld { uint64_t uid; int rows; };
  KvHeld kv_held[kKvHeld] = {};
  // one released snapshot's device block, kept for the next snapshot that fits in it (guarded by g_live_mu)
  void* spare = nullptr;
  size_t spare_bytes = 0;
  ha_config cfg{};
  std::vector<unsigned char> kinds;
  int device = 0;
  hipStream_t own = nullptr, stream = nullptr;
  std::vector<Layer> layers;
  float* rope = nullptr;
  // call-time buffers, possibly held with other engines: zeros [B][3][lin_stride] (the history of an empty context),
  // images [B][H][img_chunks] of the split form (allocated when a call can use that form), the sequential
  // form's raw outputs [B][H][kSegRows][DV] and counters [B][H], split-GQA partials [gqa_part_slots]
  std::shared_ptr<Scratch> scratch;
  size_t need_zeros = 0, need_img = 0, need_seq_raw = 0, need_seq_cnt = 0, need_gqa = 0, need_duo_ring = 0,
         need_sync_flags = 0;
  int img_chunks = 0, duo_slots = 0;
  int gqa_split = 0, gqa_part_slots = 0;
  hipEvent_t ev[2] = {nullptr, nullptr};
  std::vector<hipEvent_t> lev, mev;  // per-layer events: layer starts (and the end), ends of each layer's mixer kernels
  // error word of this engine's launches (ha::WaitCheck): pinned, host-coherent memory that a kernel whose bounded
  // wait ran out writes its bit into; read on the host without a copy, at the next call and after synchronisation
  volatile unsigned* err_host = nullptr;
  unsigned* err_dev = nullptr;
  int C = 0;
  bool any_linear = false, any_full = false;
};

struct ha_snapshot {
  uint32_t magic = kSnapMagic;
  const ha_engine* owner = nullptr;
  uint64_t owner_id = 0;
  uint64_t uid = 0;  // unique over the process, never reused
  void* block = nullptr;  // one device allocation holding every part below
  size_t block_bytes = 0;
  int P = 0, s0 = 0, tail_rows = 0;
  bool released = false;
  struct Part {
    float* S = nullptr;
    void* tail = nullptr;
    _Float16* K = nullptr;
    _Float16* V = nullptr;
  };
  std::vector<Part> layers;
};

namespace {

bool engine_ok(const ha_engine* e) {
  std::lock_guard<std::mutex> lock(g_live_mu);
  return e && g_live.count(e) && e->magic == kEngineMagic;
}

bool snap_ok(const ha_snapshot* s) {
  std::lock_guard<std::mutex> lock(g_live_mu);
  return s && g_live_snaps.count(s) && s->magic == kSnapMagic;
}

// The live engine that made a snapshot, or nullptr once that engine is gone.
const ha_engine* snapshot_owner(const ha_snapshot* s) {
  std::lock_guard<std::mutex> lock(g_live_mu);
  const ha_engine* e = s->owner;
  return (e && g_live.count(e) && e->id == s->owner_id) ? e : nullptr;
}

// HA_CHUNKED's choice of gated-delta prefill, from the engine's shape alone so that every call rounds alike: the
// split form (every chunk's preparation spread over the chip, then the state pass with the outputs beside it) up to
// 32 sequence-heads, the paired form above that while its two workgroups per recurrence fit the 256 CUs in one round
// (B*H a multiple of 8, at most 128), the fused kernel beyond. Measured per layer at T = 2048, 18 forwards back to
// back (split / paired / fused, us): B=1 68 / 175 / -, B=2 114 / 176 / -, B=3 189 / 183 / -, B=4 252 / 196 / -,
// B=8 - / 271 / 303, B=16 - / - / 350.
bool split_by_shape(const ha_config& c) { return c.batch * c.H <= 32; }
bool paired_by_shape(const ha_config& c) { return !split_by_shape(c) && ha::gdn_duo_fits(c.batch, c.H); }

int check_config(const ha_config* c) {
  if (!c) return fail(HA_ERR_ARG, "config is NULL");
  if (c->n_layers <= 0 || !c->layer_kind) return fail(HA_ERR_ARG, "n_layers must be > 0 with a layer_kind array");
  if (c->batch <= 0 || c->max_ctx <= 0) return fail(HA_ERR_ARG, "batch and max_ctx must be > 0");
  if (std::fabs(c->eps - 1e-6f) > 1e-12f) return fail(HA_ERR_ARG, "eps must be 1e-6 (the value the kernels use)");
  bool lin = false, full = false;
  for (int i = 0; i < c->n_layers; i++) {
    if (c->layer_kind[i] == HA_LINEAR_ATTENTION) lin = true;
    else if (c->layer_kind[i] == HA_FULL_ATTENTION) full = true;
    else if (c->layer_kind[i] == HA_ADAPTER) continue;
    else return fail(HA_ERR_ARG, "layer " + std::to_string(i) + ": unknown layer kind " + std::to_string(c->layer_kind[i]));
  }
  if (lin) {
    if (c->H <= 0 || c->DK != 128 || c->DV != 128 || c->conv_k != kKC)
      return fail(HA_ERR_ARG, "linear_attention layers need d_k = d_v = 128, conv kernel 4 and H > 0");
    const int C = 2 * c->H * c->DK + c->H * c->DV;
    if (c->lin_stride < C + c->H * c->DV + 2 * c->H)
      return fail(HA_ERR_ARG, "lin_stride smaller than the fused row qkv | z | a | b");
    if (c->lin_stride % 8) return fail(HA_ERR_ARG, "lin_stride must be a multiple of 8 (16-byte row segments)");
    if (c->lin_dtype != HA_F32 && c->lin_dtype != HA_F16) return fail(HA_ERR_ARG, "lin_dtype must be HA_F32 or HA_F16");
  }
  if (full) {
    if (c->HD != 256 || c->HK <= 0 || c->HQ <= 0 || c->HQ % c->HK || c->HQ / c->HK != 4)
      return fail(HA_ERR_ARG, "full_attention layers need head_dim 256 and 4 query heads per KV head");
    if (c->rot_dim != 64) return fail(HA_ERR_ARG, "rotary_dim must be 64 (partial RoPE on 64 of 256 dims)");
    if (c->max_ctx % 64) return fail(HA_ERR_ARG, "max_ctx must be a multiple of 64 for full_attention layers");
    if (c->full_stride < c->HQ * 2 * c->HD + 2 * c->HK * c->HD)
      return fail(HA_ERR_ARG, "full_stride smaller than the fused row [q|gate] x HQ | k | v");
    if (c->full_dtype != HA_F32 && c->full_dtype != HA_F16) return fail(HA_ERR_ARG, "full_dtype must be HA_F32 or HA_F16");
    if (!(c->rope_theta > 0.0f)) return fail(HA_ERR_ARG, "rope_theta must be > 0");
  }
  return HA_OK;
}

template <typename T>
int dalloc(T** p, size_t bytes) {
  hipError_t e = hipMalloc(reinterpret_cast<void**>(p), bytes ? bytes : 16);
  if (e != hipSuccess) { *p = nullptr; return fail(HA_ERR_NOMEM, std::string("hipMalloc: ") + hipGetErrorString(e)); }
  return HA_OK;
}

int fill_f32(float* d, size_t n, float v) {
  std::vector<float> h(n, v);
  HA_HIP(hipMemcpy(d, h.data(), n * sizeof(float), hipMemcpyHostToDevice));
  return HA_OK;
}

void free_engine(ha_engine* e) {
  if (!e) return;
  (void)hipSetDevice(e->device);
  if (e->stream) (void)hipStreamSynchronize(e->stream);
  for (auto& l : e->layers) {
    for (void* p : {(void*)l.conv, (void*)l.negA, (void*)l.dtb, (void*)l.gnorm, (void*)l.qn, (void*)l.kn, (void*)l.S,
                    l.tail, (void*)l.K, (void*)l.V})
      if (p) (void)hipFree(p);
  }
  if (e->rope) (void)hipFree(e->rope);
  if (e->scratch) {
    std::lock_guard<std::mutex> lock(g_live_mu);
    auto& hs = e->scratch->holders;
    hs.erase(std::remove(hs.begin(), hs.end(), e), hs.end());
  }
  e->scratch.reset();
  for (auto ev : e->ev) if (ev) (void)hipEventDestroy(ev);
  for (auto ev : e->lev) if (ev) (void)hipEventDestroy(ev);
  for (auto ev : e->mev) if (ev) (void)hipEventDestroy(ev);
  if (e->own) (void)hipStreamDestroy(e->own);
  if (e->err_host) (void)hipHostFree(const_cast<unsigned*>(e->err_host));
  void* spare = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_live_mu);
    g_live.erase(e);
    spare = e->spare;
    e->spare = nullptr;
  }
  if (spare) (void)hipFree(spare);
  e->magic = kDeadMagic;
  delete e;
}

// The snapshot's block goes back to its engine as the spare when that engine is alive and holds none (the caller has
// synchronised the engine's stream), else to hipFree.
void free_snapshot_buffers(ha_snapshot* s) {
  for (auto& p : s->layers) p = ha_snapshot::Part{};
  if (!s->block) return;
  bool parked = false;
  {
    std::lock_guard<std::mutex> lock(g_live_mu);
    ha_engine* e = const_cast<ha_engine*>(s->owner);
    if (e && g_live.count(e) && e->id == s->owner_id && !e->spare) {
      e->spare = s->block;
      e->spare_bytes = s->block_bytes;
      parked = true;
    }
  }
  if (!parked) (void)hipFree(s->block);
  s->block = nullptr;
  s->block_bytes = 0;
}

// A bounded cross-workgroup wait of one of e's launches ran out (see ha::WaitCheck): report it once, as
// HA_ERR_DEVICE, and clear the word. The engine.js counterpart throws the device errors a forward collected
// (engine.js:373).
int take_device_error(ha_engine* e) {
  const unsigned v = *e->err_host;
  if (!v) return HA_OK;
  *e->err_host = 0u;
  std::string what;
  if (v & ha::kErrDuoWait) what += " a paired-form consumer gave up waiting for a tile set;";
  if (v & ha::kErrSplitWait) what += " a split-form output workgroup gave up waiting for a packed state;";
  if (v & ha::kErrGqaMerge) what += " a split-key attention merge gave up waiting for its pieces;";
  if (what.empty()) what = " unknown code " + std::to_string(v) + ";";
  return fail(HA_ERR_DEVICE, "device error in an earlier kernel of this engine (its outputs are undefined):" +
                                 what.substr(0, what.size() - 1));
}

}  // namespace

static_assert(ha::kMnbScratchBytes == HA_MNB_SCRATCH_BYTES, "ha.h states the no-allocation scratch size");
constexpr uint32_t kMnbMagic = 0x48414d4eu;
struct ha_mnb {
  uint32_t magic = kMnbMagic;
  ha::MnbArgs args{};
  int device = 0;
  float* ws = nullptr;  // fp32 partial products of a split GEMM, grown on demand
  size_t ws_bytes = 0;
};

namespace {
bool mnb_ok(const ha_mnb* w) {
  std::lock_guard<std::mutex> lock(g_live_mu);
  return w && g_live_mnbs.count(w) && w->magic == kMnbMagic;
}
}  // namespace

extern "C" {

const char* ha_last_error(void) { return g_err.c_str(); }
int ha_abi_version(void) { return HA_ABI_VERSION; }

int ha_device_arch(int device, char* name, size_t bytes) {
  if (!name || bytes == 0) return fail(HA_ERR_ARG, "name must be non-NULL with bytes > 0");
  name[0] = 0;
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return fail(HA_ERR_DEVICE, "no HIP device is visible");
  if (device < 0 || device >= ndev) return fail(HA_ERR_ARG, "no HIP device " + std::to_string(device));
  hipDeviceProp_t p;
  HA_HIP(hipGetDeviceProperties(&p, device));
  std::string a(p.gcnArchName);
  a = a.substr(0, a.find(':'));  // "gfx950:sramecc+:xnack-" -> "gfx950"
  std::snprintf(name, bytes, "%s", a.c_str());
  return HA_OK;
}

int ha_create(const ha_config* cfg, int device, ha_engine** out) {
  if (!out) return fail(HA_ERR_ARG, "out is NULL");
  *out = nullptr;
  int rc = check_config(cfg);
  if (rc) return rc;
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return fail(HA_ERR_DEVICE, "no HIP device is visible");
  if (device < 0 || device >= ndev) return fail(HA_ERR_ARG, "device index out of range");
  HA_HIP(hipSetDevice(device));

  ha_engine* e = new ha_engine();
  e->id = g_engine_ids.fetch_add(1);
  {
    std::lock_guard<std::mutex> lock(g_live_mu);
    g_live.insert(e);
  }
  e->cfg = *cfg;
  e->kinds.assign(cfg->layer_kind, cfg->layer_kind + cfg->n_layers);
  e->cfg.layer_kind = e->kinds.data();
  e->device = device;
  const ha_config& c = e->cfg;
  const size_t B = c.batch;
  auto bail = [&](int code) { free_engine(e); return code; };

  if (hipStreamCreateWithFlags(&e->own, hipStreamNonBlocking) != hipSuccess) return bail(fail(HA_ERR_DEVICE, "hipStreamCreate failed"));
  e->stream = e->own;
  if (hipEventCreate(&e->ev[0]) != hipSuccess || hipEventCreate(&e->ev[1]) != hipSuccess)
    return bail(fail(HA_ERR_DEVICE, "hipEventCreate failed"));
  e->lev.assign(c.n_layers + 1, nullptr);
  e->mev.assign(c.n_layers, nullptr);
  for (auto* evs : {&e->lev, &e->mev})
    for (auto& ev : *evs)
      if (hipEventCreate(&ev) != hipSuccess) return bail(fail(HA_ERR_DEVICE, "hipEventCreate failed"));
  {
    void* w = nullptr;
    if (hipHostMalloc(&w, 64, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess)
      return bail(fail(HA_ERR_NOMEM, "hipHostMalloc of the error word failed"));
    e->err_host = static_cast<volatile unsigned*>(w);
    *e->err_host = 0u;
    void* d = nullptr;
    if (hipHostGetDevicePointer(&d, w, 0) != hipSuccess) return bail(fail(HA_ERR_DEVICE, "hipHostGetDevicePointer failed"));
    e->err_dev = static_cast<unsigned*>(d);
  }

  e->layers.resize(c.n_layers);
  for (int i = 0; i < c.n_layers; i++) {
    Layer& l = e->layers[i];
    l.kind = c.layer_kind[i];
    if (l.kind == HA_LINEAR_ATTENTION) {
      e->any_linear = true;
      e->C = 2 * c.H * c.DK + c.H * c.DV;
      const size_t esz = dtype_size(c.lin_dtype);
      if ((rc = dalloc(&l.conv, sizeof(float) * e->C * kKC)) || (rc = dalloc(&l.negA, sizeof(float) * c.H)) ||
          (rc = dalloc(&l.dtb, sizeof(float) * c.H)) || (rc = dalloc(&l.gnorm, sizeof(float) * c.DV)) ||
          (rc = dalloc(&l.S, sizeof(float) * B * c.H * c.DK * c.DV)) ||
          (rc = dalloc(&l.tail, esz * B * kTailCap * c.lin_stride)))
        return bail(rc);
      if (hipMemset(l.conv, 0, sizeof(float) * e->C * kKC) != hipSuccess || hipMemset(l.negA, 0, sizeof(float) * c.H) != hipSuccess ||
          hipMemset(l.dtb, 0, sizeof(float) * c.H) != hipSuccess || hipMemset(l.tail, 0, esz * B * kTailCap * c.lin_stride) != hipSuccess)
        return bail(fail(HA_ERR_DEVICE, "hipMemset failed"));
      if ((rc = fill_f32(l.gnorm, c.DV, 1.0f))) return bail(rc);
    } else if (l.kind == HA_FULL_ATTENTION) {
      e->any_full = true;
      const size_t kv = B * c.HK * (size_t)c.max_ctx * c.HD;
      if ((rc = dalloc(&l.qn, sizeof(float) * c.HD)) || (rc = dalloc(&l.kn, sizeof(float) * c.HD)) ||
          (rc = dalloc(&l.K, sizeof(_Float16) * kv)) || (rc = dalloc(&l.V, sizeof(_Float16) * kv)))
        return bail(rc);
      if ((rc = fill_f32(l.qn, c.HD, 1.0f)) || (rc = fill_f32(l.kn, c.HD, 1.0f))) return bail(rc);
      if (hipMemset(l.K, 0, sizeof(_Float16) * kv) != hipSuccess || hipMemset(l.V, 0, sizeof(_Float16) * kv) != hipSuccess)
        return bail(fail(HA_ERR_DEVICE, "hipMemset failed"));
    }
  }
  e->scratch = std::make_shared<Scratch>();
  e->scratch->device = device;
  {
    std::lock_guard<std::mutex> lock(g_live_mu);
    e->scratch->holders.push_back(e);
  }
  if (e->any_linear) {
    e->need_zeros = dtype_size(c.lin_dtype) * B * (kKC - 1) * c.lin_stride;
    // chunk images: every chunk a call can touch (max_ctx / 64, plus the replayed open chunk); allocated here only
    // when HA_CHUNKED picks the split form for this shape, else by the first call that forces that form
    e->img_chunks = (c.max_ctx + ha::kChunk - 1) / ha::kChunk + 1;
    e->need_img = ha::gdn_split_image_bytes() * B * c.H * e->img_chunks;
    e->need_seq_raw = sizeof(float) * B * c.H * ha::kSegRows * c.DV;
    e->need_seq_cnt = sizeof(unsigned) * B * c.H;
    // the paired form's tile sets (a slot for every 32-row chunk a call can have) and progress counters, likewise
    // only where HA_CHUNKED picks that form
    e->duo_slots = (c.max_ctx + 31) / 32;
    e->need_duo_ring = (size_t)e->duo_slots * ha::kDuoSetBytes * B * c.H;
    e->need_sync_flags = sizeof(unsigned) * 64 * B * c.H;
    if ((rc = grow(e->scratch->zeros, e->need_zeros)) || (rc = grow(e->scratch->seq_raw, e->need_seq_raw)) ||
        (rc = grow(e->scratch->seq_cnt, e->need_seq_cnt)) || (rc = grow(e->scratch->sync_flags, e->need_sync_flags)) ||
        (split_by_shape(c) && (rc = grow(e->scratch->img, e->need_img))) ||
        (paired_by_shape(c) && (rc = grow(e->scratch->duo_ring, e->need_duo_ring))))
      return bail(rc);
  }
  if (e->any_full) {
    // RoPE table as engine.js:105-106 builds it: angle t / theta^(2i/RD) in f64, stored as f32 (cos, sin)
    const int RD = c.rot_dim;
    std::vector<float> rope((size_t)c.max_ctx * RD);
    for (int t = 0; t < c.max_ctx; t++)
      for (int i = 0; i < RD / 2; i++) {
        const double a = (double)t / std::pow((double)c.rope_theta, (2.0 * i) / RD);
        rope[(size_t)t * RD + 2 * i] = (float)std::cos(a);
        rope[(size_t)t * RD + 2 * i + 1] = (float)std::sin(a);
      }
    if ((rc = dalloc(&e->rope, rope.size() * sizeof(float)))) return bail(rc);
    // Few (sequence, KV head) pairs leave most CUs idle behind the longest query blocks: split every block's key
    // range into pieces of gqa_split tiles (at most 8 pieces per block) on separate workgroups. Decided from the
    // engine's shape alone, so every call rounds a given row the same way. Measured at T = 2048: 0.135 -> 0.089 ms
    // for one sequence (2 pairs); at 4 pairs the partial results cost more than the idle CUs.
    if (B * c.HK <= 2) {
      const int N = (c.max_ctx + 63) / 64;
      e->gqa_split = std::max(8, (N + 7) / 8);
      const size_t slots = ha::gqa_part_slots((int)B * c.HK, c.max_ctx, e->gqa_split);
      e->gqa_part_slots = (int)slots;
      e->need_gqa = slots * ha::gqa_part_slot_bytes();
      if ((rc = grow(e->scratch->gqa_part, e->need_gqa))) return bail(rc);
    }
    if (hipMemcpy(e->rope, rope.data(), rope.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
      return bail(fail(HA_ERR_DEVICE, "hipMemcpy rope failed"));
  }
  *out = e;
  return HA_OK;
}

int ha_destroy(ha_engine* e) {
  if (!engine_ok(e)) return fail(HA_ERR_HANDLE, "invalid engine handle");
  free_engine(e);
  return HA_OK;
}

int ha_set_stream(ha_engine* e, void* stream) {
  if (!engine_ok(e)) return fail(HA_ERR_HANDLE, "invalid engine handle");
  hipStream_t to = stream ? static_cast<hipStream_t>(stream) : e->own;
  if (to == e->stream) return HA_OK;
  // Engines holding one set of call-time buffers must stay on one stream (their launches use the same progress
  // counters and tile-set slots, and a newer epoch's counters would satisfy an older launch's waits at once). An
  // engine that moves to another stream while the set is held by others gets a set of its own first.
  bool shared = false;
  {
    std::lock_guard<std::mutex> lock(g_live_mu);
    for (const ha_engine* h : e->scratch->holders) shared |= h != e;
  }
  if (shared) {
    HA_HIP(hipSetDevice(e->device));
    HA_HIP(hipDeviceSynchronize());  // no queued call may still use the set being left
    auto s = std::make_shared<Scratch>();
    s->device = e->device;
    const ha_config& c = e->cfg;
    int rc;
    if ((rc = grow(s->zeros, e->need_zeros)) || (rc = grow(s->seq_raw, e->need_seq_raw)) ||
        (rc = grow(s->seq_cnt, e->need_seq_cnt)) || (rc = grow(s->sync_flags, e->need_sync_flags)) ||
        (rc = grow(s->gqa_part, e->need_gqa)) || (rc = grow(s->img, split_by_shape(c) ? e->need_img : 0)) ||
        (rc = grow(s->duo_ring, paired_by_shape(c) ? e->need_duo_ring : 0)))
      return rc;
    std::lock_guard<std::mutex> lock(g_live_mu);
    auto& hs = e->scratch->holders;
    hs.erase(std::remove(hs.begin(), hs.end(), e), hs.end());
    s->holders.push_back(e);
    e->scratch = s;
  }
  e->stream = to;
  return HA_OK;
}

int ha_share_scratch(ha_engine* e, ha_engine* holder) {
  if (!engine_ok(e) || !engine_ok(holder)) return fail(HA_ERR_HANDLE, "invalid engine handle");
  if (e->device != holder->device) return fail(HA_ERR_ARG, "engines are on different devices");
  if (e->stream != holder->stream)
    return fail(HA_ERR_ARG, "engines sharing call-time buffers must run on one stream (ha_set_stream first)");
  if (e->scratch == holder->scratch) return HA_OK;
  HA_HIP(hipSetDevice(e->device));
  HA_HIP(hipDeviceSynchronize());  // no queued call of either engine may still use a buffer that is replaced
  Scratch& to = *holder->scratch;
  const Scratch& from = *e->scratch;
  int rc;
  // images only where e had them (its shape picks the split form, or a call forced it)
  if ((rc = grow(to.zeros, e->need_zeros)) || (rc = grow(to.img, from.img.bytes ? e->need_img : 0)) ||
      (rc = grow(to.seq_raw, e->need_seq_raw)) ||
      (rc = grow(to.seq_cnt, e->need_seq_cnt)) || (rc = grow(to.gqa_part, e->need_gqa)) ||
      (rc = grow(to.duo_ring, from.duo_ring.bytes ? e->need_duo_ring : 0)) ||
      (rc = grow(to.sync_flags, e->need_sync_flags)))
    return rc;
  std::lock_guard<std::mutex> lock(g_live_mu);
  auto& hs = e->scratch->holders;
  hs.erase(std::remove(hs.begin(), hs.end(), e), hs.end());
  holder->scratch->holders.push_back(e);
  e->scratch = holder->scratch;
  return HA_OK;
}

int ha_get_stream(ha_engine* e, void** stream) {
  if (!engine_ok(e)) return fail(HA_ERR_HANDLE, "invalid engine handle");
  if (!stream) return fail(HA_ERR_ARG, "stream must be non-NULL");
  *stream = e->stream;
  return HA_OK;
}

int ha_set_param(ha_engine* e, int layer, const char* name, const float* host, size_t count) {
  if (!engine_ok(e)) return fail(HA_ERR_HANDLE, "invalid engine handle");
  if (!name || !host) return fail(HA_ERR_ARG, "name and data must be non-NULL");
  if (layer < 0 || layer >= e->cfg.n_layers) return fail(HA_ERR_ARG, "layer index out of range");
  const ha_config& c = e->cfg;
  Layer& l = e->layers[layer];
  float* dst = nullptr;
  size_t want = 0;
  const std::string n(name);
  if (l.kind == HA_LINEAR_ATTENTION) {
    if (n == "conv") { dst = l.conv; want = (size_t)e->C * kKC; }
    else if (n == "neg_exp_A") { dst = l.negA; want = c.H; }
    else if (n == "dt_bias") { dst = l.dtb; want = c.H; }
    else if (n == "gnorm") { dst = l.gnorm; want = c.DV; }
  } else if (l.kind == HA_FULL_ATTENTION) {
    if (n == "q_norm") { dst = l.qn; want = c.HD; }
    else if (n == "k_norm") { dst = l.kn; want = c.HD; }
  }
  if (!dst) return fail(HA_ERR_PARAM, "no tensor layers." + std::to_string(layer) + "." + n + " for this layer kind");
  if (count != want)
    return fail(HA_ERR_PARAM, "layers." + std::to_string(layer) + "." + n + ": expected " + std::to_string(want) +
                                  " floats, got " + std::to_string(count));
  HA_HIP(hipSetDevice(e->device));
  HA_HIP(hipMemcpy(dst, host, want * sizeof(float), hipMemcpyHostToDevice));
  return HA_OK;
}

int ha_forward(ha_engine* e, int L, const void* const* layer_in, void* const* layer_out, const ha_snapshot* resume,
               ha_snapshot** keep, ha_forward_opts* opts) {
  if (!engine_ok(e)) return fail(HA_ERR_HANDLE, "invalid engine handle");
  if (keep) *keep = nullptr;
  const ha_config& c = e->cfg;
  if (L <= 0) return fail(HA_ERR_ARG, "L must be > 0");
  if (!layer_in || !layer_out) return fail(HA_ERR_ARG, "layer_in and layer_out must be non-NULL");
  for (int i = 0; i < c.n_layers; i++)
    if (e->layers[i].kind != HA_ADAPTER && (!layer_in[i] || !layer_out[i]))
      return fail(HA_ERR_ARG, "layer " + std::to_string(i) + ": NULL input or output");
  if (resume) {
    if (!snap_ok(resume)) return fail(HA_ERR_HANDLE, "invalid snapshot handle");
    if (resume->owner != e || resume->owner_id != e->id) return fail(HA_ERR_HANDLE, "snapshot belongs to another engine");
    if (resume->released) return fail(HA_ERR_HANDLE, "snapshot was released");
    if ((int)resume->layers.size() != c.n_layers) return fail(HA_ERR_HANDLE, "snapshot layer count mismatch");
  }
  const int P = resume ? resume->P : 0;
  const int s0 = resume ? resume->s0 : 0;
  if ((long)P + L > c.max_ctx)
    return fail(HA_ERR_CONTEXT, "context " + std::to_string((long)P + L) + " exceeds " + std::to_string(c.max_ctx));
  const int mode = opts ? opts->recurrence : HA_CHUNKED;
  if (mode < HA_CHUNKED || mode > HA_CHUNKED_PAIRED) return fail(HA_ERR_ARG, "unknown recurrence mode");
  if (mode == HA_CHUNKED_PAIRED && !ha::gdn_duo_fits(c.batch, c.H))
    return fail(HA_ERR_ARG, "the paired form needs batch * H a multiple of 8 and at most 128");
  const bool chunked = mode != HA_SEQUENTIAL;
  const bool per_layer = opts && (opts->layer_ms || opts->mixer_ms);
  const bool timing = opts && (opts->timestamps || per_layer);
  // a bounded wait of an earlier call that ran out (its outputs are undefined) fails this call before it runs
  if (int rc = take_device_error(e)) return rc;
  ha::WaitCheck wait;
  wait.err = e->err_dev;
  const bool unpublished = opts && opts->debug_unpublished_waits;
  if (unpublished) wait.polls = 4;
  HA_HIP(hipSetDevice(e->device));
  hipStream_t st = e->stream;
  const size_t B = c.batch;

  // resume: K/V rows [0, P) back into the working caches (engine.js:327), unless they already hold them (the last
  // completed call resumed from or kept this snapshot, and calls write only rows from their P on); state and tail
  // are read in place
  bool kv_held = false;
  ha_engine::KvHeld held[ha_engine::kKvHeld];
  int nheld = 0;
  for (const auto& h : e->kv_held) {
    if (!h.uid) continue;
    if (resume && h.uid == resume->uid && h.rows >= P) kv_held = true;
    if (h.rows <= P) held[nheld++] = h;  // still in place after this call
  }
  // a restore copy rewrites rows [0, P): then no earlier entry holds any more (only the resumed snapshot does)
  if (resume && P > 0 && !kv_held) nheld = 0;
  for (auto& h : e->kv_held) h = {0, 0};  // unknown until this call completes
  if (resume && P > 0 && !kv_held)
    for (int i = 0; i < c.n_layers; i++)
      if (e->layers[i].kind == HA_FULL_ATTENTION) {
        const size_t w = (size_t)P * c.HD * sizeof(_Float16), dp = (size_t)c.max_ctx * c.HD * sizeof(_Float16);
        HA_HIP(hipMemcpy2DAsync(e->layers[i].K, dp, resume->layers[i].K, w, w, B * c.HK, hipMemcpyDeviceToDevice, st));
        // V^T: P positions of every (sequence, KV head, dim) row
        const size_t vw = (size_t)P * sizeof(_Float16), vp = (size_t)c.max_ctx * sizeof(_Float16);
        HA_HIP(hipMemcpy2DAsync(e->layers[i].V, vp, resume->layers[i].V, vw, vw, B * c.HK * c.HD, hipMemcpyDeviceToDevice, st));
      }

  const int end = P + L;
  const int s1 = chunked ? s0 + ha::kChunk * ((end - s0) / ha::kChunk) : end;  // new state position
  // HA_CHUNKED picks the implementation from the engine's shape alone (split_by_shape, paired_by_shape). The forms
  // round differently, so the choice must not depend on the call: a resumed suffix must match the same rows of one
  // longer forward bit for bit.
  const bool split = mode == HA_CHUNKED_SPLIT || (mode == HA_CHUNKED && split_by_shape(c));
  const bool paired = mode == HA_CHUNKED_PAIRED || (mode == HA_CHUNKED && paired_by_shape(c));
  Scratch& sc = *e->scratch;
  if (e->any_linear && chunked && split && sc.img.bytes < e->need_img) {
    int rc = grow(sc.img, e->need_img);  // first call that forces the split form on a larger shape
    if (rc) return rc;
  }
  if (e->any_linear && chunked && paired && sc.duo_ring.bytes < e->need_duo_ring) {
    int rc;  // first call that forces the paired form on another shape
    if ((rc = grow(sc.duo_ring, e->need_duo_ring))) return rc;
  }
  // raw-row tails: the copy reads only the call's input rows and the resumed tail, so the layers' copies are
  // gathered into one launch after the mixers (per layer when per-layer times are asked for, so that each layer's
  // time includes its own copy)
  ha::TailArgs t{};
  t.B = c.batch; t.stride = c.lin_stride; t.C = e->C; t.ab_off = e->C + c.H * c.DV; t.ab_n = 2 * c.H;
  t.P = P; t.L = L; t.s0 = s0; t.KC = kKC; t.tail_cap_in = resume ? resume->tail_rows : kKC - 1;
  t.tail_cap_out = kTailCap; t.dst_first = s1 - (kKC - 1); t.dtype = c.lin_dtype == HA_F16 ? 1 : 0;
  auto flush_tails = [&]() {
    const hipError_t he = ha::launch_tail_update(t, st);
    t.n = 0;
    return he;
  };
  if (timing) HA_HIP(hipEventRecord(e->ev[0], st));
  for (int i = 0; i < c.n_layers; i++) {
    Layer& l = e->layers[i];
    if (per_layer) HA_HIP(hipEventRecord(e->lev[i], st));
    if (l.kind == HA_LINEAR_ATTENTION) {
      ha::GdnArgs a{};
      a.B = c.batch; a.H = c.H; a.DK = c.DK; a.DV = c.DV; a.KC = kKC; a.stride = c.lin_stride; a.C = e->C;
      a.P = P; a.L = L; a.s0 = s0;
      a.tail = resume ? resume->layers[i].tail : sc.zeros.p;
      a.tail_cap = resume ? resume->tail_rows : kKC - 1;
      a.dtype = c.lin_dtype == HA_F16 ? 1 : 0;
      a.in = layer_in[i]; a.out = layer_out[i];
      a.S_in = resume ? resume->layers[i].S : nullptr; a.S_out = l.S;
      a.conv_w = l.conv; a.negA = l.negA; a.dtb = l.dtb; a.gnorm = c.lin_gnorm ? l.gnorm : nullptr;
      a.img = sc.img.p; a.img_chunks = e->img_chunks;
      a.seq_raw = static_cast<float*>(sc.seq_raw.p); a.seq_cnt = static_cast<unsigned*>(sc.seq_cnt.p);
      // progress counter values are epoch << kDuoEpochShift | chunks: a skew of one epoch is never published
      a.wait = wait;
      if (unpublished) a.wait.skew = 1u << ha::kDuoEpochShift;
      hipError_t he;
      if (!chunked) {
        he = ha::launch_gdn_sequential(a, st);
      } else if (split || paired) {
        // a fresh progress-counter epoch per launch; before the epoch field runs out, the counters are cleared
        if (sc.sync_epoch + 1 >= (1u << (32 - ha::kDuoEpochShift))) {
          HA_HIP(hipStreamSynchronize(st));
          HA_HIP(hipMemset(sc.sync_flags.p, 0, sc.sync_flags.bytes));
          sc.sync_epoch = 0;
        }
        a.sync_flags = static_cast<unsigned*>(sc.sync_flags.p); a.sync_epoch = ++sc.sync_epoch;
        a.duo_ring = sc.duo_ring.p; a.duo_slots = e->duo_slots;
        he = split ? ha::launch_gdn_split(a, st) : ha::launch_gdn_duo(a, st);
      } else {
        he = ha::launch_gdn_chunked(a, st);
      }
      if (he != hipSuccess) return fail(HA_ERR_DEVICE, "layer " + std::to_string(i) + " gated-delta launch: " + hipGetErrorString(he));
      if (per_layer) HA_HIP(hipEventRecord(e->mev[i], st));
      t.in[t.n] = a.in; t.tail[t.n] = a.tail; t.tail_out[t.n] = l.tail; t.n++;
      if (per_layer || t.n == ha::kTailLayers) {
        he = flush_tails();
        if (he != hipSuccess) return fail(HA_ERR_DEVICE, "layer " + std::to_string(i) + " tail update: " + hipGetErrorString(he));
      }
    } else if (l.kind == HA_FULL_ATTENTION) {
      ha::GqaArgs a{};
      a.B = c.batch; a.HQ = c.HQ; a.HK = c.HK; a.HD = c.HD; a.RD = c.rot_dim; a.stride = c.full_stride; a.LT = c.max_ctx;
      a.P = P; a.L = L; a.dtype = c.full_dtype == HA_F16 ? 1 : 0;
      a.in = layer_in[i]; a.out = layer_out[i]; a.qw = l.qn; a.kw = l.kn; a.rope = e->rope;
      a.K = l.K; a.V = l.V;
      a.split = e->gqa_split; a.part_slots = e->gqa_part_slots; a.part = static_cast<float*>(sc.gqa_part.p);
      if (a.split > 0) {
        // a fresh mark per launch; if the counter wraps, the marks (and partials) are cleared first
        if (++sc.gqa_epoch == 0) {
          HA_HIP(hipStreamSynchronize(st));
          HA_HIP(hipMemset(sc.gqa_part.p, 0, sc.gqa_part.bytes));
          sc.gqa_epoch = 1;
        }
        a.epoch = sc.gqa_epoch;
      }
      // the merge waits for marks equal to this launch's epoch: epoch + 1 is never written by it
      a.wait = wait;
      if (unpublished) a.wait.skew = 1u;
      hipError_t he = ha::launch_gqa(a, st);
      if (he != hipSuccess) return fail(HA_ERR_DEVICE, "layer " + std::to_string(i) + " attention launch: " + hipGetErrorString(he));
      if (per_layer) HA_HIP(hipEventRecord(e->mev[i], st));
    } else if (per_layer) {  // HA_ADAPTER: no token mixer, nothing to run
      HA_HIP(hipEventRecord(e->mev[i], st));
    }
  }
  if (t.n > 0) {
    const hipError_t he = flush_tails();
    if (he != hipSuccess) return fail(HA_ERR_DEVICE, std::string("tail update: ") + hipGetErrorString(he));
  }
  if (per_layer) HA_HIP(hipEventRecord(e->lev[c.n_layers], st));
  if (timing) HA_HIP(hipEventRecord(e->ev[1], st));

  if (keep) {
    ha_snapshot* s = new ha_snapshot();
    s->owner = e; s->owner_id = e->id; s->uid = ++g_snap_uid; s->P = end; s->s0 = e->any_linear ? s1 : end;
    s->tail_rows = s->P - (s->s0 - (kKC - 1));
    s->layers.resize(c.n_layers);
    auto bail = [&](int code) { (void)hipStreamSynchronize(st); free_snapshot_buffers(s); s->magic = kDeadMagic; delete s; return code; };
    // every part in one device block (256-byte aligned offsets), the engine's spare block when it is large enough;
    // a new block is rounded up to 2 MiB so that the next snapshots of a growing context fit in it when it returns
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    size_t total = 0;
    for (int i = 0; i < c.n_layers; i++) {
      const Layer& l = e->layers[i];
      if (l.kind == HA_LINEAR_ATTENTION)
        total += al(sizeof(float) * B * c.H * c.DK * c.DV) + al(dtype_size(c.lin_dtype) * c.lin_stride * B * s->tail_rows);
      else if (l.kind == HA_FULL_ATTENTION)
        total += 2 * al((size_t)end * c.HD * sizeof(_Float16) * B * c.HK);
    }
    {
      std::lock_guard<std::mutex> lock(g_live_mu);
      if (e->spare && e->spare_bytes >= total) {
        s->block = e->spare; s->block_bytes = e->spare_bytes;
        e->spare = nullptr; e->spare_bytes = 0;
      }
    }
    if (!s->block) {
      const size_t bytes = (total + ((size_t)2 << 20) - 1) & ~(((size_t)2 << 20) - 1);
      int rc = dalloc(reinterpret_cast<char**>(&s->block), bytes);
      if (rc) return bail(rc);
      s->block_bytes = bytes;
    }
    size_t off = 0;
    auto take = [&](size_t b) { void* q = static_cast<char*>(s->block) + off; off += al(b); return q; };
    for (int i = 0; i < c.n_layers; i++) {
      Layer& l = e->layers[i];
      ha_snapshot::Part& p = s->layers[i];
      if (l.kind == HA_LINEAR_ATTENTION) {
        const size_t sb = sizeof(float) * B * c.H * c.DK * c.DV, esz = dtype_size(c.lin_dtype);
        const size_t rowb = esz * c.lin_stride;
        p.S = static_cast<float*>(take(sb));
        p.tail = take(rowb * B * s->tail_rows);
        if (hipMemcpyAsync(p.S, l.S, sb, hipMemcpyDeviceToDevice, st) != hipSuccess ||
            hipMemcpy2DAsync(p.tail, rowb * s->tail_rows, l.tail, rowb * kTailCap, rowb * s->tail_rows, B,
                             hipMemcpyDeviceToDevice, st) != hipSuccess)
          return bail(fail(HA_ERR_DEVICE, "snapshot copy failed"));
      } else if (l.kind == HA_FULL_ATTENTION) {
        const size_t w = (size_t)end * c.HD * sizeof(_Float16), sp = (size_t)c.max_ctx * c.HD * sizeof(_Float16);
        const size_t vw = (size_t)end * sizeof(_Float16), vp = (size_t)c.max_ctx * sizeof(_Float16);
        p.K = static_cast<_Float16*>(take(w * B * c.HK));
        p.V = static_cast<_Float16*>(take(w * B * c.HK));
        if (hipMemcpy2DAsync(p.K, w, l.K, sp, w, B * c.HK, hipMemcpyDeviceToDevice, st) != hipSuccess ||
            hipMemcpy2DAsync(p.V, vw, l.V, vp, vw, B * c.HK * c.HD, hipMemcpyDeviceToDevice, st) != hipSuccess)
          return bail(fail(HA_ERR_DEVICE, "snapshot copy failed"));
      }
    }
    {
      std::lock_guard<std::mutex> lock(g_live_mu);
      g_live_snaps.insert(s);
    }
    *keep = s;
  }
  if (timing || (opts && opts->sync)) {
    HA_HIP(hipStreamSynchronize(st));
    if (int rc = take_device_error(e)) {
      // this call's outputs are undefined: no snapshot of them is handed out
      if (keep && *keep) {
        (void)ha_snapshot_destroy(*keep);
        *keep = nullptr;
      }
      return rc;
    }
    if (opts && opts->timestamps) HA_HIP(hipEventElapsedTime(&opts->gpu_ms, e->ev[0], e->ev[1]));
    if (opts && opts->layer_ms)
      for (int i = 0; i < c.n_layers; i++) HA_HIP(hipEventElapsedTime(&opts->layer_ms[i], e->lev[i], e->lev[i + 1]));
    if (opts && opts->mixer_ms)
      for (int i = 0; i < c.n_layers; i++) HA_HIP(hipEventElapsedTime(&opts->mixer_ms[i], e->lev[i], e->mev[i]));
  }
  hipError_t le = hipGetLastError();
  if (le != hipSuccess) return fail(HA_ERR_DEVICE, std::string("device error: ") + hipGetErrorString(le));
  // the working caches now hold the kept snapshot's rows, the resumed one's rows [0, P), and those of the earlier
  // entries that ended at or before P (newest first; the oldest drop out when the list is full)
  {
    int n = 0;
    auto add = [&](uint64_t uid, int rows) {
      for (int i = 0; i < n; i++)
        if (e->kv_held[i].uid == uid) return;
      if (n < ha_engine::kKvHeld) e->kv_held[n++] = {uid, rows};
    };
    if (keep) add((*keep)->uid, end);
    if (resume) add(resume->uid, P);
    for (int i = 0; i < nheld; i++) add(held[i].uid, held[i].rows);
  }
  return HA_OK;
}

int ha_snapshot_tokens(const ha_snapshot* s, int* P) {
  if (!snap_ok(s)) return fail(HA_ERR_HANDLE, "invalid snapshot handle");
  if (!P) return fail(HA_ERR_ARG, "P is NULL");
  *P = s->P;
  return HA_OK;
}

int ha_snapshot_layout(const ha_snapshot* s, int* state_pos, int* tail_rows) {
  if (!snap_ok(s)) return fail(HA_ERR_HANDLE, "invalid snapshot handle");
  if (state_pos) *state_pos = s->s0;
  if (tail_rows) *tail_rows = s->tail_rows;
  return HA_OK;
}

int ha_snapshot_read(const ha_snapshot* s, int layer, const char* what, void* host, size_t bytes) {
  if (!snap_ok(s)) return fail(HA_ERR_HANDLE, "invalid snapshot handle");
  if (s->released) return fail(HA_ERR_HANDLE, "snapshot was released");
  if (!what || !host) return fail(HA_ERR_ARG, "what and host must be non-NULL");
  const ha_engine* e = snapshot_owner(s);
  if (!e) return fail(HA_ERR_HANDLE, "the snapshot's engine was destroyed");
  if (layer < 0 || layer >= (int)s->layers.size()) return fail(HA_ERR_ARG, "layer index out of range");
  const ha_config& c = e->cfg;
  const size_t B = c.batch;
  const std::string w(what);
  const void* src = nullptr;
  size_t want = 0;
  const bool lin = e->layers[layer].kind == HA_LINEAR_ATTENTION, full = e->layers[layer].kind == HA_FULL_ATTENTION;
  if (lin && w == "state" && s->s0 < s->P) {
    // the state at P, as the reference's snapshot holds it (engine.js:352-356): the stored state advanced over the
    // snapshot's replay rows [state_pos, P) by the sequential fp32 rule, into a temporary buffer
    want = sizeof(float) * B * c.H * c.DK * c.DV;
    if (bytes != want) return fail(HA_ERR_ARG, "expected " + std::to_string(want) + " bytes, got " + std::to_string(bytes));
    HA_HIP(hipSetDevice(e->device));
    float* tmp = nullptr;
    int rc = dalloc(&tmp, want);
    if (rc) return rc;
    const Layer& l = e->layers[layer];
    ha::GdnArgs a{};
    a.B = c.batch; a.H = c.H; a.DK = c.DK; a.DV = c.DV; a.KC = kKC; a.stride = c.lin_stride; a.C = e->C;
    a.P = s->P; a.L = 0; a.s0 = s->s0;
    a.tail = s->layers[layer].tail; a.tail_cap = s->tail_rows;
    a.dtype = c.lin_dtype == HA_F16 ? 1 : 0;
    a.S_in = s->layers[layer].S; a.S_out = tmp;
    a.conv_w = l.conv; a.negA = l.negA; a.dtb = l.dtb; a.gnorm = nullptr;  // no output rows: replay only
    hipError_t he = ha::launch_gdn_sequential(a, e->stream);
    if (he == hipSuccess) he = hipMemcpyAsync(host, tmp, want, hipMemcpyDeviceToHost, e->stream);
    const hipError_t se = hipStreamSynchronize(e->stream);  // also before the free when a step above failed
    if (he == hipSuccess) he = se;
    (void)hipFree(tmp);
    if (he != hipSuccess) return fail(HA_ERR_DEVICE, std::string("snapshot state at P: ") + hipGetErrorString(he));
    return HA_OK;
  }
  if (lin && (w == "state" || w == "state_stored")) { src = s->layers[layer].S; want = sizeof(float) * B * c.H * c.DK * c.DV; }
  else if (lin && w == "tail") { src = s->layers[layer].tail; want = dtype_size(c.lin_dtype) * B * s->tail_rows * c.lin_stride; }
  else if (full && (w == "K" || w == "V")) {
    src = w == "K" ? (const void*)s->layers[layer].K : (const void*)s->layers[layer].V;
    want = sizeof(_Float16) * B * c.HK * (size_t)s->P * c.HD;
  } else return fail(HA_ERR_PARAM, "no part '" + w + "' for this layer kind");
  if (bytes != want) return fail(HA_ERR_ARG, "expected " + std::to_string(want) + " bytes, got " + std::to_string(bytes));
  HA_HIP(hipSetDevice(e->device));
  if (w == "V") {  // stored [B][HK][HD][P]; returned as [B][HK][P][HD]
    std::vector<uint16_t> tmp(want / 2);
    HA_HIP(hipMemcpyAsync(tmp.data(), src, want, hipMemcpyDeviceToHost, e->stream));
    HA_HIP(hipStreamSynchronize(e->stream));
    uint16_t* dst = static_cast<uint16_t*>(host);
    const size_t P = s->P, HD = c.HD;
    for (size_t bh = 0; bh < B * c.HK; bh++)
      for (size_t d = 0; d < HD; d++)
        for (size_t t = 0; t < P; t++) dst[(bh * P + t) * HD + d] = tmp[(bh * HD + d) * P + t];
    return HA_OK;
  }
  HA_HIP(hipMemcpyAsync(host, src, want, hipMemcpyDeviceToHost, e->stream));
  HA_HIP(hipStreamSynchronize(e->stream));
  return HA_OK;
}

int ha_snapshot_release(ha_snapshot* s) {
  if (!snap_ok(s)) return fail(HA_ERR_HANDLE, "invalid snapshot handle");
  if (s->released) return HA_OK;
  if (const ha_engine* e = snapshot_owner(s)) {
    (void)hipSetDevice(e->device);
    (void)hipStreamSynchronize(e->stream);  // the snapshot's copies may still be in flight
  }
  free_snapshot_buffers(s);
  s->released = true;
  return HA_OK;
}

int ha_snapshot_destroy(ha_snapshot* s) {
  int rc = ha_snapshot_release(s);
  if (rc) return rc;
  {
    std::lock_guard<std::mutex> lock(g_live_mu);
    g_live_snaps.erase(s);
  }
  s->magic = kDeadMagic;
  delete s;
  return HA_OK;
}

int ha_device_alloc(ha_engine* e, size_t bytes, void** dptr) {
  if (!engine_ok(e)) return fail(HA_ERR_HANDLE, "invalid engine handle");
  if (!dptr) return fail(HA_ERR_ARG, "dptr is NULL");
  HA_HIP(hipSetDevice(e->device));
  return dalloc(dptr, bytes);
}

int ha_device_free(ha_engine* e, void* dptr) {
  if (!engine_ok(e)) return fail(HA_ERR_HANDLE, "invalid engine handle");
  HA_HIP(hipSetDevice(e->device));
  HA_HIP(hipStreamSynchronize(e->stream));
  if (dptr) HA_HIP(hipFree(dptr));
  return HA_OK;
}

int ha_copy_to_device(ha_engine* e, void* dst, const void* host, size_t bytes) {
  if (!engine_ok(e)) return fail(HA_ERR_HANDLE, "invalid engine handle");
  if (!dst || !host) return fail(HA_ERR_ARG, "NULL pointer");
  HA_HIP(hipSetDevice(e->device));
  HA_HIP(hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, e->stream));
  HA_HIP(hipStreamSynchronize(e->stream));
  return HA_OK;
}

int ha_copy_to_host(ha_engine* e, void* host, const void* src, size_t bytes) {
  if (!engine_ok(e)) return fail(HA_ERR_HANDLE, "invalid engine handle");
  if (!src || !host) return fail(HA_ERR_ARG, "NULL pointer");
  HA_HIP(hipSetDevice(e->device));
  HA_HIP(hipMemcpyAsync(host, src, bytes, hipMemcpyDeviceToHost, e->stream));
  HA_HIP(hipStreamSynchronize(e->stream));
  return take_device_error(e);  // the copied outputs of a call whose wait ran out are undefined
}

int ha_synchronize(ha_engine* e) {
  if (!engine_ok(e)) return fail(HA_ERR_HANDLE, "invalid engine handle");
  HA_HIP(hipSetDevice(e->device));
  HA_HIP(hipStreamSynchronize(e->stream));
  return take_device_error(e);
}

// ---- MatMulNBits projections ----

int ha_mnb_create(int N, int K, const ha_mnb_format* fmt, const void* q, const void* s, const void* b, int device,
                  ha_mnb** out) {
  if (!fmt || !out) return fail(HA_ERR_ARG, "fmt and out must be non-NULL");
  *out = nullptr;
  ha::MnbArgs a{};
  a.N = N; a.K = K; a.bits = fmt->bits; a.group = fmt->group; a.asym = fmt->asym ? 1 : 0;
  a.q = q; a.s = s; a.b = b;
  if (ha::mnb_check(a) != hipSuccess)
    return fail(HA_ERR_ARG, "unsupported MatMulNBits shape or format (K % 32, K % group, bits 2/3/4, group "
                            "32/64, q/s (and b when asymmetric) non-NULL)");
  int ndev = 0;
  HA_HIP(hipGetDeviceCount(&ndev));
  if (device < 0 || device >= ndev) return fail(HA_ERR_ARG, "no HIP device " + std::to_string(device));
  HA_HIP(hipSetDevice(device));
  // the allocation-free entry point's scratch address on this device, looked up once per device
  HA_HIP(ha::mnb_scratch_setup(device));
  ha_mnb* w = new ha_mnb();
  w->args = a;
  w->device = device;
  {
    std::lock_guard<std::mutex> lock(g_live_mu);
    g_live_mnbs.insert(w);
  }
  *out = w;
  return HA_OK;
}

}  // extern "C"

namespace {

// ha_mnb_forward and ha_mnb_forward_noalloc: the same kernels and K split; they differ only in where a split
// product's fp32 partials go (the handle's workspace, grown on demand, or the library's fixed per-device scratch).
int mnb_forward(ha_mnb* w, int M, const void* a, void* y, void* stream, bool noalloc) {
  if (!mnb_ok(w)) return fail(HA_ERR_HANDLE, "invalid MatMulNBits handle");
  if (M < 1 || !a || !y) return fail(HA_ERR_ARG, "M must be >= 1 and a, y non-NULL");
  if (w->args.N % 16) return fail(HA_ERR_ARG, "a matmul needs N % 16 == 0 (the exporter pads N to 64)");
  HA_HIP(hipSetDevice(w->device));
  hipStream_t st = (hipStream_t)stream;
  ha::MnbArgs g = w->args;
  g.M = M; g.a = a; g.y = y;
  if (ha::mnb_packed_path(M, g.N, g.K)) {
    HA_HIP(ha::launch_mnb_gemv(g, st));
    return HA_OK;
  }
  g.split = ha::mnb_gemm_split(M, g.N, g.K);
  if (g.split > 1 && noalloc) {
    const size_t need = sizeof(float) * (size_t)g.split * M * g.N;
    if (need > ha::kMnbScratchBytes)
      return fail(HA_ERR_ARG, "M = " + std::to_string(M) + " on this shape needs " + std::to_string(need) +
                                  " bytes of split-K scratch, more than the " + std::to_string(ha::kMnbScratchBytes) +
                                  " the allocation-free entry point has; use ha_mnb_forward");
    g.ws = ha::mnb_scratch(w->device);
    if (!g.ws) return fail(HA_ERR_DEVICE, "split-K scratch of this device was not set up");
  } else if (g.split > 1) {
    const size_t need = sizeof(float) * (size_t)g.split * M * g.N;
    if (need > w->ws_bytes) {
      if (w->ws) {
        HA_HIP(hipDeviceSynchronize());  // earlier calls on this handle may still read the old area
        (void)hipFree(w->ws);
        w->ws = nullptr;
        w->ws_bytes = 0;
      }
      int rc = dalloc(&w->ws, need);
      if (rc) return rc;
      w->ws_bytes = need;
    }
    g.ws = w->ws;
  }
  HA_HIP(ha::launch_mnb_gemm(g, st));
  return HA_OK;
}

}  // namespace

extern "C" {

int ha_mnb_forward(ha_mnb* w, int M, const void* a, void* y, void* stream) {
  return mnb_forward(w, M, a, y, stream, false);
}

int ha_mnb_forward_noalloc(ha_mnb* w, int M, const void* a, void* y, void* stream) {
  return mnb_forward(w, M, a, y, stream, true);
}

int ha_mnb_destroy(ha_mnb* w) {
  if (!w) return HA_OK;
  if (!mnb_ok(w)) return fail(HA_ERR_HANDLE, "invalid MatMulNBits handle");
  if (w->ws) {
    HA_HIP(hipSetDevice(w->device));
    HA_HIP(hipDeviceSynchronize());  // a split product in flight may still use the workspace
    (void)hipFree(w->ws);
    w->ws = nullptr;
  }
  {
    std::lock_guard<std::mutex> lock(g_live_mu);
    g_live_mnbs.erase(w);
  }
  w->magic = kDeadMagic;
  delete w;
  return HA_OK;
}

int ha_fwht(void* x, long elems, int n, int device, void* stream) {
  if (!x || elems <= 0) return fail(HA_ERR_ARG, "x must be non-NULL and elems > 0");
  HA_HIP(hipSetDevice(device));
  hipError_t he = ha::launch_fwht(x, elems, n, (hipStream_t)stream);
  if (he == hipErrorInvalidValue) return fail(HA_ERR_ARG, "n must be a power of two in [2, 8192] dividing elems");
  HA_HIP(he);
  return HA_OK;
}

int ha_embed(const ha_mnb* table, int L, const void* ids, void* x, void* stream) {
  if (!mnb_ok(table)) return fail(HA_ERR_HANDLE, "invalid MatMulNBits handle");
  if (L < 1 || !ids || !x) return fail(HA_ERR_ARG, "L must be >= 1 and ids, x non-NULL");
  HA_HIP(hipSetDevice(table->device));
  const ha::MnbArgs& t = table->args;
  ha::EmbedArgs a{};
  a.L = L; a.D = t.K; a.rows = t.N; a.bits = t.bits; a.group = t.group; a.asym = t.asym;
  a.ids = (const unsigned*)ids; a.q = (const unsigned*)t.q; a.s = (const _Float16*)t.s; a.b = (const _Float16*)t.b;
  a.x = (float*)x;
  hipError_t he = ha::launch_embed(a, (hipStream_t)stream);
  if (he == hipErrorInvalidValue) return fail(HA_ERR_ARG, "unsupported embedding table shape or format");
  HA_HIP(he);
  return HA_OK;
}

int ha_add_norm(int R, int D, int nx, void* x, const void* y, const float* w, void* h, int out_f32,
                const void* rows, float eps, int device, void* stream) {
  if (!x || !w || !h) return fail(HA_ERR_ARG, "x, w and h must be non-NULL");
  if (R < 1 || nx < 1 || D < 8 || D % 8 || D > 8192) return fail(HA_ERR_ARG, "need R, nx >= 1, D % 8 == 0, D <= 8192");
  if (!rows && R > nx) return fail(HA_ERR_ARG, "R > nx without a row list");
  HA_HIP(hipSetDevice(device));
  ha::AddNormArgs a{};
  a.R = R; a.D = D; a.nx = nx; a.x = (float*)x; a.y = (const _Float16*)y; a.w = w; a.h = h; a.out_f32 = out_f32 ? 1 : 0;
  a.rows = (const unsigned*)rows; a.eps = eps;
  HA_HIP(ha::launch_add_norm(a, (hipStream_t)stream));
  return HA_OK;
}

int ha_silu_mul(int L, int I, const void* big, void* mid, int device, void* stream) {
  if (!big || !mid || L < 1 || I < 8 || I % 8) return fail(HA_ERR_ARG, "need big, mid non-NULL, L >= 1, I % 8 == 0");
  HA_HIP(hipSetDevice(device));
  HA_HIP(ha::launch_silu_mul(big, mid, L, I, (hipStream_t)stream));
  return HA_OK;
}

int ha_add_bias(int L, int N, void* y, const float* c, int device, void* stream) {
  if (!y || !c || L < 1 || N < 8 || N % 8) return fail(HA_ERR_ARG, "need y, c non-NULL, L >= 1, N % 8 == 0");
  HA_HIP(hipSetDevice(device));
  HA_HIP(ha::launch_add_bias(y, c, L, N, (hipStream_t)stream));
  return HA_OK;
}

}  // extern "C"

struct ha_timer {
  uint32_t magic = kTimerMagic;
  int device = 0;
  std::vector<hipEvent_t> ev;
  std::vector<char> marked;
};

namespace {

bool timer_ok(const ha_timer* t) {
  std::lock_guard<std::mutex> lock(g_live_mu);
  return t && g_live_timers.count(t) && t->magic == kTimerMagic;
}

void free_timer(ha_timer* t) {
  (void)hipSetDevice(t->device);
  for (hipEvent_t ev : t->ev)
    if (ev) (void)hipEventDestroy(ev);
  {
    std::lock_guard<std::mutex> lock(g_live_mu);
    g_live_timers.erase(t);
  }
  t->magic = kDeadMagic;
  delete t;
}

}  // namespace

extern "C" {

int ha_timer_create(int device, int n, ha_timer** out) {
  if (!out) return fail(HA_ERR_ARG, "timer output pointer is NULL");
  *out = nullptr;
  if (n <= 0 || n > (1 << 20)) return fail(HA_ERR_ARG, "timestamp count must be in [1, 2^20]");
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev) return fail(HA_ERR_ARG, "device index out of range");
  HA_HIP(hipSetDevice(device));
  ha_timer* t = new ha_timer();
  t->device = device;
  t->ev.assign(n, nullptr);
  t->marked.assign(n, 0);
  {
    std::lock_guard<std::mutex> lock(g_live_mu);
    g_live_timers.insert(t);
  }
  for (auto& ev : t->ev)
    if (hipEventCreate(&ev) != hipSuccess) {
      free_timer(t);
      return fail(HA_ERR_DEVICE, "hipEventCreate failed");
    }
  *out = t;
  return HA_OK;
}

int ha_timer_mark(ha_timer* t, int i, void* stream) {
  if (!timer_ok(t)) return fail(HA_ERR_HANDLE, "invalid timer handle");
  if (i < 0 || i >= (int)t->ev.size()) return fail(HA_ERR_ARG, "timestamp index out of range");
  HA_HIP(hipSetDevice(t->device));
  HA_HIP(hipEventRecord(t->ev[i], (hipStream_t)stream));
  t->marked[i] = 1;
  return HA_OK;
}

int ha_timer_elapsed(ha_timer* t, int i, int j, float* ms) {
  if (!timer_ok(t)) return fail(HA_ERR_HANDLE, "invalid timer handle");
  if (!ms) return fail(HA_ERR_ARG, "ms must be non-NULL");
  const int n = (int)t->ev.size();
  if (i < 0 || i >= n || j < 0 || j >= n) return fail(HA_ERR_ARG, "timestamp index out of range");
  if (!t->marked[i] || !t->marked[j]) return fail(HA_ERR_ARG, "timestamp was not recorded");
  HA_HIP(hipSetDevice(t->device));
  HA_HIP(hipEventSynchronize(t->ev[i]));
  HA_HIP(hipEventSynchronize(t->ev[j]));
  HA_HIP(hipEventElapsedTime(ms, t->ev[i], t->ev[j]));
  return HA_OK;
}

int ha_timer_destroy(ha_timer* t) {
  if (!t) return HA_OK;
  if (!timer_ok(t)) return fail(HA_ERR_HANDLE, "invalid timer handle");
  free_timer(t);
  return HA_OK;
}

}  // extern "C"
