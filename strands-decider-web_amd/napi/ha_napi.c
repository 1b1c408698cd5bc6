/*
 * ha_napi.c: Node N-API binding of the hybrid-attention C ABI (include/ha.h). Thin by design: every export maps to
 * one ha_* call, a non-zero status becomes a thrown Error carrying ha_last_error() (the reference engine throws
 * Errors from Engine.forward, web/public/engine/engine.js:316,373), and handles are JS externals whose finalizers
 * free what the script leaked (a snapshot not release()d, an engine not destroy()ed).
 *
 * Device pointers cross into JS as BigInt (N-API 6+, Node >= 10.20). Host data crosses as TypedArrays.
 */
#define NAPI_VERSION 6
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ha.h"

/* Every external holds one of these boxes; `kind` tells them apart, so a handle of the wrong kind is a TypeError. */
enum { BOX_ENGINE = 0x45, BOX_SNAPSHOT = 0x53, BOX_MNB = 0x4d, BOX_TIMER = 0x54 };

typedef struct engine_box {
  int kind;
  ha_engine* e;
  /* shareStream: the engine whose stream this one runs on, held by a strong reference so that it cannot be
     collected (and its stream destroyed) while this engine lives; and the engines that run on this one's stream.
     Links are dropped from both ends: at environment teardown Node finalizes in no set order, so an owner finalized
     before its borrowers first moves each of them back to its own stream and clears their link to it. */
  napi_ref stream_owner;
  struct engine_box* owner_box;
  struct engine_box** borrower;
  int borrowers, borrower_cap;
} engine_box;

typedef struct {
  int kind;
  ha_snapshot* s;
} snap_box;

typedef struct {
  int kind;
  ha_mnb* w;
} mnb_box;

typedef struct {
  int kind;
  ha_timer* t;
} timer_box;

static napi_value throw_status(napi_env env, int rc) {
  char code[16];
  snprintf(code, sizeof(code), "HA_%d", -rc);
  const char* msg = ha_last_error();
  napi_throw_error(env, code, (msg && *msg) ? msg : "hybrid-attention call failed");
  return NULL;
}

#define CHECK_NAPI(call)                                                    \
  do {                                                                      \
    if ((call) != napi_ok) {                                                \
      const napi_extended_error_info* info = NULL;                          \
      napi_get_last_error_info(env, &info);                                 \
      bool pending = false;                                                 \
      napi_is_exception_pending(env, &pending);                             \
      if (!pending)                                                         \
        napi_throw_error(env, NULL, info && info->error_message ? info->error_message : "N-API call failed"); \
      return NULL;                                                          \
    }                                                                       \
  } while (0)

#define CHECK_HA(call)                   \
  do {                                   \
    int rc_ = (call);                    \
    if (rc_ != HA_OK) return throw_status(env, rc_); \
  } while (0)

static napi_value type_error(napi_env env, const char* msg) {
  napi_throw_type_error(env, NULL, msg);
  return NULL;
}

/* ---- argument helpers ---- */

static int get_args(napi_env env, napi_callback_info info, size_t want, napi_value* argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, NULL, NULL) != napi_ok) return 0;
  for (size_t i = argc; i < want; i++) napi_get_undefined(env, &argv[i]);
  return 1;
}

static int is_nullish(napi_env env, napi_value v) {
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok) return 1;
  return t == napi_undefined || t == napi_null;
}

static int get_int(napi_env env, napi_value obj, const char* key, int def, int* out) {
  napi_value v;
  bool has = false;
  if (napi_has_named_property(env, obj, key, &has) != napi_ok) return 0;
  if (!has) { *out = def; return 1; }
  if (napi_get_named_property(env, obj, key, &v) != napi_ok) return 0;
  if (is_nullish(env, v)) { *out = def; return 1; }
  int32_t x;
  if (napi_get_value_int32(env, v, &x) != napi_ok) return 0;
  *out = x;
  return 1;
}

static int get_float(napi_env env, napi_value obj, const char* key, float def, float* out) {
  napi_value v;
  bool has = false;
  if (napi_has_named_property(env, obj, key, &has) != napi_ok) return 0;
  if (!has) { *out = def; return 1; }
  if (napi_get_named_property(env, obj, key, &v) != napi_ok) return 0;
  if (is_nullish(env, v)) { *out = def; return 1; }
  double x;
  if (napi_get_value_double(env, v, &x) != napi_ok) return 0;
  *out = (float)x;
  return 1;
}

static int get_ptr(napi_env env, napi_value v, void** out) {
  uint64_t x;
  bool lossless = false;
  if (napi_get_value_bigint_uint64(env, v, &x, &lossless) != napi_ok || !lossless) return 0;
  *out = (void*)(uintptr_t)x;
  return 1;
}

static void* get_box(napi_env env, napi_value v, int kind) {
  napi_valuetype t;
  void* p = NULL;
  if (napi_typeof(env, v, &t) != napi_ok || t != napi_external) return NULL;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p || *(const int*)p != kind) return NULL;
  return p;
}

static engine_box* get_engine(napi_env env, napi_value v) { return (engine_box*)get_box(env, v, BOX_ENGINE); }
static snap_box* get_snap(napi_env env, napi_value v) { return (snap_box*)get_box(env, v, BOX_SNAPSHOT); }
static mnb_box* get_mnb(napi_env env, napi_value v) { return (mnb_box*)get_box(env, v, BOX_MNB); }
static timer_box* get_timer(napi_env env, napi_value v) { return (timer_box*)get_box(env, v, BOX_TIMER); }

/* host bytes of a TypedArray / ArrayBuffer view */
static int get_bytes(napi_env env, napi_value v, void** data, size_t* bytes) {
  bool is_ta = false;
  if (napi_is_typedarray(env, v, &is_ta) != napi_ok || !is_ta) return 0;
  napi_typedarray_type type;
  size_t len, off;
  napi_value ab;
  void* d;
  if (napi_get_typedarray_info(env, v, &type, &len, &d, &ab, &off) != napi_ok) return 0;
  size_t esz = 1;
  switch (type) {
    case napi_int16_array: case napi_uint16_array: esz = 2; break;
    case napi_int32_array: case napi_uint32_array: case napi_float32_array: esz = 4; break;
    case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: esz = 8; break;
    default: esz = 1;
  }
  *data = d;
  *bytes = len * esz;
  return 1;
}

/* ---- finalizers ---- */

/* drop an engine's link to the engine whose stream it borrowed (the owner is alive while the link exists) */
static void unshare_stream(napi_env env, engine_box* b) {
  engine_box* o = b->owner_box;
  if (o) {
    for (int i = 0; i < o->borrowers; i++)
      if (o->borrower[i] == b) {
        o->borrower[i] = o->borrower[--o->borrowers];
        break;
      }
  }
  if (b->stream_owner) napi_delete_reference(env, b->stream_owner);
  b->stream_owner = NULL;
  b->owner_box = NULL;
}

static int add_borrower(engine_box* o, engine_box* b) {
  if (o->borrowers == o->borrower_cap) {
    const int cap = o->borrower_cap ? 2 * o->borrower_cap : 4;
    engine_box** p = (engine_box**)realloc(o->borrower, (size_t)cap * sizeof(engine_box*));
    if (!p) return 0;
    o->borrower = p;
    o->borrower_cap = cap;
  }
  o->borrower[o->borrowers++] = b;
  return 1;
}

static void engine_finalize(napi_env env, void* data, void* hint) {
  (void)hint;
  engine_box* b = (engine_box*)data;
  /* engines still running on this one's stream (only at environment teardown, where finalizers run in no set
     order; destroy() refuses otherwise): back to their own streams before that stream goes away */
  for (int i = 0; i < b->borrowers; i++) {
    engine_box* x = b->borrower[i];
    if (x->e) ha_set_stream(x->e, NULL);
    if (x->stream_owner) napi_delete_reference(env, x->stream_owner);
    x->stream_owner = NULL;
    x->owner_box = NULL;
  }
  b->borrowers = 0;
  unshare_stream(env, b);
  if (b->e) ha_destroy(b->e);
  free(b->borrower);
  free(b);
}

static void snap_finalize(napi_env env, void* data, void* hint) {
  (void)env; (void)hint;
  snap_box* b = (snap_box*)data;
  if (b->s) ha_snapshot_destroy(b->s);
  free(b);
}

static void mnb_finalize(napi_env env, void* data, void* hint) {
  (void)env; (void)hint;
  mnb_box* b = (mnb_box*)data;
  if (b->w) ha_mnb_destroy(b->w);
  free(b);
}

static void timer_finalize(napi_env env, void* data, void* hint) {
  (void)env; (void)hint;
  timer_box* b = (timer_box*)data;
  if (b->t) ha_timer_destroy(b->t);
  free(b);
}

/* ---- exports ---- */

static napi_value js_abi_version(napi_env env, napi_callback_info info) {
  (void)info;
  napi_value r;
  CHECK_NAPI(napi_create_int32(env, ha_abi_version(), &r));
  return r;
}

static napi_value js_last_error(napi_env env, napi_callback_info info) {
  (void)info;
  napi_value r;
  CHECK_NAPI(napi_create_string_utf8(env, ha_last_error(), NAPI_AUTO_LENGTH, &r));
  return r;
}

/* create(cfg, device) -> engine. cfg uses the C field names; layerKinds is an array of 0 (linear_attention) /
   1 (full_attention). */
static napi_value js_create(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return type_error(env, "create(cfg, device)");
  napi_value cfgv = argv[0];
  napi_value kinds;
  bool is_arr = false;
  CHECK_NAPI(napi_get_named_property(env, cfgv, "layerKinds", &kinds));
  CHECK_NAPI(napi_is_array(env, kinds, &is_arr));
  if (!is_arr) return type_error(env, "cfg.layerKinds must be an array of 0/1");
  uint32_t n = 0;
  CHECK_NAPI(napi_get_array_length(env, kinds, &n));
  unsigned char* lk = (unsigned char*)malloc(n ? n : 1);
  if (!lk) return type_error(env, "out of host memory");
  for (uint32_t i = 0; i < n; i++) {
    napi_value v;
    int32_t k;
    if (napi_get_element(env, kinds, i, &v) != napi_ok || napi_get_value_int32(env, v, &k) != napi_ok) {
      free(lk);
      return type_error(env, "cfg.layerKinds must hold integers");
    }
    lk[i] = (unsigned char)k;
  }
  ha_config c;
  memset(&c, 0, sizeof(c));
  c.n_layers = (int)n;
  c.layer_kind = lk;
  int ok = get_int(env, cfgv, "batch", 1, &c.batch) && get_int(env, cfgv, "maxCtx", 4096, &c.max_ctx) &&
           get_int(env, cfgv, "H", 16, &c.H) && get_int(env, cfgv, "DK", 128, &c.DK) &&
           get_int(env, cfgv, "DV", 128, &c.DV) && get_int(env, cfgv, "convK", 4, &c.conv_k) &&
           get_int(env, cfgv, "linStride", 8256, &c.lin_stride) && get_int(env, cfgv, "linDtype", HA_F32, &c.lin_dtype) &&
           get_int(env, cfgv, "linGnorm", 1, &c.lin_gnorm) && get_int(env, cfgv, "HQ", 8, &c.HQ) &&
           get_int(env, cfgv, "HK", 2, &c.HK) && get_int(env, cfgv, "HD", 256, &c.HD) &&
           get_int(env, cfgv, "rotDim", 64, &c.rot_dim) && get_int(env, cfgv, "fullStride", 5120, &c.full_stride) &&
           get_int(env, cfgv, "fullDtype", HA_F16, &c.full_dtype) &&
           get_float(env, cfgv, "ropeTheta", 1e7f, &c.rope_theta) && get_float(env, cfgv, "eps", 1e-6f, &c.eps);
  if (!ok) {
    free(lk);
    return type_error(env, "invalid engine config field");
  }
  int32_t device = 0;
  if (!is_nullish(env, argv[1]) && napi_get_value_int32(env, argv[1], &device) != napi_ok) {
    free(lk);
    return type_error(env, "device must be an integer");
  }
  ha_engine* e = NULL;
  int rc = ha_create(&c, device, &e);
  free(lk);
  if (rc) return throw_status(env, rc);
  engine_box* b = (engine_box*)malloc(sizeof(engine_box));
  if (!b) {
    ha_destroy(e);
    return type_error(env, "out of host memory");
  }
  b->kind = BOX_ENGINE;
  b->e = e;
  b->stream_owner = NULL;
  b->owner_box = NULL;
  b->borrower = NULL;
  b->borrowers = 0;
  b->borrower_cap = 0;
  napi_value r;
  if (napi_create_external(env, b, engine_finalize, NULL, &r) != napi_ok) {
    ha_destroy(e);
    free(b);
    napi_throw_error(env, NULL, "napi_create_external failed");
    return NULL;
  }
  return r;
}

static napi_value js_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  engine_box* b = get_engine(env, argv[0]);
  if (!b) return type_error(env, "not an engine handle");
  if (b->e && b->borrowers > 0) {
    char msg[96];
    snprintf(msg, sizeof(msg), "%d engine(s) run on this engine's stream (shareStream); destroy them first",
             b->borrowers);
    napi_throw_error(env, "HA_STREAM_SHARED", msg);
    return NULL;
  }
  if (b->e) {
    ha_engine* e = b->e;
    b->e = NULL;
    unshare_stream(env, b);
    CHECK_HA(ha_destroy(e));
  }
  return NULL;
}

#define ENGINE_ARG(v)                                                  \
  engine_box* eb_ = get_engine(env, (v));                              \
  if (!eb_) return type_error(env, "not an engine handle");            \
  if (!eb_->e) return type_error(env, "engine was destroyed");         \
  ha_engine* e = eb_->e

/* setParam(engine, layer, name, Float32Array) */
static napi_value js_set_param(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  if (!get_args(env, info, 4, argv)) return NULL;
  ENGINE_ARG(argv[0]);
  int32_t layer;
  char name[64];
  size_t nlen = 0;
  if (napi_get_value_int32(env, argv[1], &layer) != napi_ok) return type_error(env, "layer must be an integer");
  if (napi_get_value_string_utf8(env, argv[2], name, sizeof(name), &nlen) != napi_ok)
    return type_error(env, "name must be a string");
  napi_typedarray_type type;
  size_t len, off;
  napi_value ab;
  void* d;
  bool is_ta = false;
  if (napi_is_typedarray(env, argv[3], &is_ta) != napi_ok || !is_ta ||
      napi_get_typedarray_info(env, argv[3], &type, &len, &d, &ab, &off) != napi_ok || type != napi_float32_array)
    return type_error(env, "data must be a Float32Array");
  CHECK_HA(ha_set_param(e, layer, name, (const float*)d, len));
  return NULL;
}

/* forward(engine, L, inputs: BigInt[], outputs: BigInt[], resume: snapshot|null, keep: bool,
           opts: {recurrence, timestamps, layerMs, sync}) -> {snapshot, gpuMs, layerMs} */
static napi_value js_forward(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  if (!get_args(env, info, 7, argv)) return NULL;
  ENGINE_ARG(argv[0]);
  int32_t L;
  if (napi_get_value_int32(env, argv[1], &L) != napi_ok) return type_error(env, "L must be an integer");
  uint32_t ni = 0, no = 0;
  bool arr = false;
  CHECK_NAPI(napi_is_array(env, argv[2], &arr));
  if (!arr) return type_error(env, "inputs must be an array of device pointers");
  CHECK_NAPI(napi_is_array(env, argv[3], &arr));
  if (!arr) return type_error(env, "outputs must be an array of device pointers");
  CHECK_NAPI(napi_get_array_length(env, argv[2], &ni));
  CHECK_NAPI(napi_get_array_length(env, argv[3], &no));
  if (ni != no) return type_error(env, "inputs and outputs must have one entry per layer");
  void** ins = (void**)calloc(ni ? ni : 1, sizeof(void*));
  void** outs = (void**)calloc(no ? no : 1, sizeof(void*));
  float* lms = NULL;
  if (!ins || !outs) {
    free(ins); free(outs);
    return type_error(env, "out of host memory");
  }
  for (uint32_t i = 0; i < ni; i++) {
    napi_value v, w;
    if (napi_get_element(env, argv[2], i, &v) != napi_ok || !get_ptr(env, v, &ins[i]) ||
        napi_get_element(env, argv[3], i, &w) != napi_ok || !get_ptr(env, w, &outs[i])) {
      free(ins); free(outs);
      return type_error(env, "device pointers must be BigInt");
    }
  }
  const ha_snapshot* resume = NULL;
  if (!is_nullish(env, argv[4])) {
    snap_box* sb = get_snap(env, argv[4]);
    if (!sb || !sb->s) { free(ins); free(outs); return type_error(env, "resume must be a snapshot handle"); }
    resume = sb->s;
  }
  bool keep = false;
  if (!is_nullish(env, argv[5])) napi_get_value_bool(env, argv[5], &keep);
  ha_forward_opts o;
  memset(&o, 0, sizeof(o));
  int want_lms = 0;
  if (!is_nullish(env, argv[6])) {
    if (!get_int(env, argv[6], "recurrence", HA_CHUNKED, &o.recurrence) ||
        !get_int(env, argv[6], "timestamps", 0, &o.timestamps) || !get_int(env, argv[6], "sync", 0, &o.sync) ||
        !get_int(env, argv[6], "layerMs", 0, &want_lms)) {
      free(ins); free(outs);
      return type_error(env, "invalid forward options");
    }
  }
  if (want_lms) {
    lms = (float*)calloc(ni ? ni : 1, sizeof(float));
    o.layer_ms = lms;
  }
  ha_snapshot* snap = NULL;
  int rc = ha_forward(e, L, (const void* const*)ins, (void* const*)outs, resume, keep ? &snap : NULL, &o);
  free(ins);
  free(outs);
  if (rc) {
    free(lms);
    return throw_status(env, rc);
  }
  napi_value res, v;
  CHECK_NAPI(napi_create_object(env, &res));
  if (snap) {
    snap_box* sb = (snap_box*)malloc(sizeof(snap_box));
    if (!sb) {
      ha_snapshot_destroy(snap);
      free(lms);
      return type_error(env, "out of host memory");
    }
    sb->kind = BOX_SNAPSHOT;
    sb->s = snap;
    if (napi_create_external(env, sb, snap_finalize, NULL, &v) != napi_ok) {
      ha_snapshot_destroy(snap);
      free(sb);
      free(lms);
      napi_throw_error(env, NULL, "napi_create_external failed");
      return NULL;
    }
  } else {
    napi_get_null(env, &v);
  }
  CHECK_NAPI(napi_set_named_property(env, res, "snapshot", v));
  if (o.timestamps) {
    CHECK_NAPI(napi_create_double(env, o.gpu_ms, &v));
    CHECK_NAPI(napi_set_named_property(env, res, "gpuMs", v));
  }
  if (lms) {
    napi_value arrv;
    CHECK_NAPI(napi_create_array_with_length(env, ni, &arrv));
    for (uint32_t i = 0; i < ni; i++) {
      napi_value x;
      napi_create_double(env, lms[i], &x);
      napi_set_element(env, arrv, i, x);
    }
    free(lms);
    CHECK_NAPI(napi_set_named_property(env, res, "layerMs", arrv));
  }
  return res;
}

#define SNAP_ARG(v)                                                      \
  snap_box* sb_ = get_snap(env, (v));                                    \
  if (!sb_ || !sb_->s) return type_error(env, "not a snapshot handle");  \
  ha_snapshot* s = sb_->s

static napi_value js_snapshot_tokens(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  SNAP_ARG(argv[0]);
  int P = 0;
  CHECK_HA(ha_snapshot_tokens(s, &P));
  napi_value r;
  CHECK_NAPI(napi_create_int32(env, P, &r));
  return r;
}

static napi_value js_snapshot_layout(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  SNAP_ARG(argv[0]);
  int sp = 0, tr = 0;
  CHECK_HA(ha_snapshot_layout(s, &sp, &tr));
  napi_value r, a, b;
  CHECK_NAPI(napi_create_object(env, &r));
  CHECK_NAPI(napi_create_int32(env, sp, &a));
  CHECK_NAPI(napi_create_int32(env, tr, &b));
  CHECK_NAPI(napi_set_named_property(env, r, "statePos", a));
  CHECK_NAPI(napi_set_named_property(env, r, "tailRows", b));
  return r;
}

/* snapshotRead(snap, layer, what, TypedArray) */
static napi_value js_snapshot_read(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  if (!get_args(env, info, 4, argv)) return NULL;
  SNAP_ARG(argv[0]);
  int32_t layer;
  char what[16];
  size_t wl = 0;
  void* d;
  size_t bytes;
  if (napi_get_value_int32(env, argv[1], &layer) != napi_ok) return type_error(env, "layer must be an integer");
  if (napi_get_value_string_utf8(env, argv[2], what, sizeof(what), &wl) != napi_ok)
    return type_error(env, "what must be a string");
  if (!get_bytes(env, argv[3], &d, &bytes)) return type_error(env, "destination must be a TypedArray");
  CHECK_HA(ha_snapshot_read(s, layer, what, d, bytes));
  return NULL;
}

static napi_value js_snapshot_release(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  SNAP_ARG(argv[0]);
  CHECK_HA(ha_snapshot_release(s));
  return NULL;
}

static napi_value js_device_alloc(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  ENGINE_ARG(argv[0]);
  double bytes;
  if (napi_get_value_double(env, argv[1], &bytes) != napi_ok || bytes < 0) return type_error(env, "bytes must be >= 0");
  void* p = NULL;
  CHECK_HA(ha_device_alloc(e, (size_t)bytes, &p));
  napi_value r;
  CHECK_NAPI(napi_create_bigint_uint64(env, (uint64_t)(uintptr_t)p, &r));
  return r;
}

static napi_value js_device_free(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  ENGINE_ARG(argv[0]);
  void* p;
  if (!get_ptr(env, argv[1], &p)) return type_error(env, "pointer must be a BigInt");
  CHECK_HA(ha_device_free(e, p));
  return NULL;
}

/* copyToDevice(engine, dptr, TypedArray) */
static napi_value js_copy_to_device(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return NULL;
  ENGINE_ARG(argv[0]);
  void* p;
  void* d;
  size_t bytes;
  if (!get_ptr(env, argv[1], &p)) return type_error(env, "pointer must be a BigInt");
  if (!get_bytes(env, argv[2], &d, &bytes)) return type_error(env, "source must be a TypedArray");
  CHECK_HA(ha_copy_to_device(e, p, d, bytes));
  return NULL;
}

/* copyToHost(engine, TypedArray, dptr) */
static napi_value js_copy_to_host(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return NULL;
  ENGINE_ARG(argv[0]);
  void* p;
  void* d;
  size_t bytes;
  if (!get_bytes(env, argv[1], &d, &bytes)) return type_error(env, "destination must be a TypedArray");
  if (!get_ptr(env, argv[2], &p)) return type_error(env, "pointer must be a BigInt");
  CHECK_HA(ha_copy_to_host(e, d, p, bytes));
  return NULL;
}

static napi_value js_synchronize(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  ENGINE_ARG(argv[0]);
  CHECK_HA(ha_synchronize(e));
  return NULL;
}

/* The stream of an optional engine argument (null / undefined: the null stream). Returns 0 on a bad argument. */
static int stream_of(napi_env env, napi_value v, void** stream) {
  *stream = NULL;
  if (is_nullish(env, v)) return 1;
  engine_box* eb = get_engine(env, v);
  if (!eb || !eb->e) return 0;
  return ha_get_stream(eb->e, stream) == HA_OK;
}

/* mnbCreate(N, K, {bits, group, asym}, q: BigInt, s: BigInt, b: BigInt|null, device) -> handle */
static napi_value js_mnb_create(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  if (!get_args(env, info, 7, argv)) return NULL;
  int32_t N, K, device = 0;
  if (napi_get_value_int32(env, argv[0], &N) != napi_ok || napi_get_value_int32(env, argv[1], &K) != napi_ok)
    return type_error(env, "N and K must be integers");
  ha_mnb_format f;
  if (is_nullish(env, argv[2])) return type_error(env, "format must be an object {bits, group, asym}");
  if (!get_int(env, argv[2], "bits", 4, &f.bits) || !get_int(env, argv[2], "group", 32, &f.group) ||
      !get_int(env, argv[2], "asym", 0, &f.asym))
    return type_error(env, "invalid format field");
  void *q, *sc, *bi = NULL;
  if (!get_ptr(env, argv[3], &q) || !get_ptr(env, argv[4], &sc)) return type_error(env, "q and s must be BigInt");
  if (!is_nullish(env, argv[5]) && !get_ptr(env, argv[5], &bi)) return type_error(env, "b must be a BigInt or null");
  if (!is_nullish(env, argv[6]) && napi_get_value_int32(env, argv[6], &device) != napi_ok)
    return type_error(env, "device must be an integer");
  ha_mnb* w = NULL;
  CHECK_HA(ha_mnb_create(N, K, &f, q, sc, bi, device, &w));
  mnb_box* b = (mnb_box*)malloc(sizeof(mnb_box));
  if (!b) {
    ha_mnb_destroy(w);
    return type_error(env, "out of host memory");
  }
  b->kind = BOX_MNB;
  b->w = w;
  napi_value r;
  if (napi_create_external(env, b, mnb_finalize, NULL, &r) != napi_ok) {
    ha_mnb_destroy(w);
    free(b);
    napi_throw_error(env, NULL, "napi_create_external failed");
    return NULL;
  }
  return r;
}

/* mnbForward(handle, M, a: BigInt, y: BigInt, engine|null): on the engine's stream when one is given */
static napi_value js_mnb_forward(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (!get_args(env, info, 5, argv)) return NULL;
  mnb_box* mb = get_mnb(env, argv[0]);
  if (!mb) return type_error(env, "not a MatMulNBits handle");
  if (!mb->w) return type_error(env, "MatMulNBits handle was destroyed");
  int32_t M;
  void *a, *y, *st;
  if (napi_get_value_int32(env, argv[1], &M) != napi_ok) return type_error(env, "M must be an integer");
  if (!get_ptr(env, argv[2], &a) || !get_ptr(env, argv[3], &y)) return type_error(env, "a and y must be BigInt");
  if (!stream_of(env, argv[4], &st)) return type_error(env, "the last argument must be an engine handle or null");
  CHECK_HA(ha_mnb_forward(mb->w, M, a, y, st));
  return NULL;
}

static napi_value js_mnb_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  mnb_box* mb = get_mnb(env, argv[0]);
  if (!mb) return type_error(env, "not a MatMulNBits handle");
  if (mb->w) {
    ha_mnb* w = mb->w;
    mb->w = NULL;
    CHECK_HA(ha_mnb_destroy(w));
  }
  return NULL;
}

/* timerCreate(device, n): n GPU timestamps (a WebGPU timestamp query set's counterpart) */
static napi_value js_timer_create(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  int32_t device, n;
  if (napi_get_value_int32(env, argv[0], &device) != napi_ok || napi_get_value_int32(env, argv[1], &n) != napi_ok)
    return type_error(env, "device and n must be integers");
  ha_timer* t = NULL;
  CHECK_HA(ha_timer_create(device, n, &t));
  timer_box* b = (timer_box*)malloc(sizeof(timer_box));
  if (!b) {
    ha_timer_destroy(t);
    return type_error(env, "out of host memory");
  }
  b->kind = BOX_TIMER;
  b->t = t;
  napi_value r;
  if (napi_create_external(env, b, timer_finalize, NULL, &r) != napi_ok) {
    ha_timer_destroy(t);
    free(b);
    napi_throw_error(env, NULL, "napi_create_external failed");
    return NULL;
  }
  return r;
}

/* timerMark(timer, i, engine|null): timestamp i after the work queued so far on the engine's stream */
static napi_value js_timer_mark(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return NULL;
  timer_box* tb = get_timer(env, argv[0]);
  if (!tb || !tb->t) return type_error(env, "not a live timer handle");
  int32_t i;
  void* st;
  if (napi_get_value_int32(env, argv[1], &i) != napi_ok) return type_error(env, "i must be an integer");
  if (!stream_of(env, argv[2], &st)) return type_error(env, "the last argument must be an engine handle or null");
  CHECK_HA(ha_timer_mark(tb->t, i, st));
  return NULL;
}

/* timerElapsed(timer, i, j) -> milliseconds from timestamp i to j (waits for both) */
static napi_value js_timer_elapsed(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return NULL;
  timer_box* tb = get_timer(env, argv[0]);
  if (!tb || !tb->t) return type_error(env, "not a live timer handle");
  int32_t i, j;
  if (napi_get_value_int32(env, argv[1], &i) != napi_ok || napi_get_value_int32(env, argv[2], &j) != napi_ok)
    return type_error(env, "i and j must be integers");
  float ms = 0.0f;
  CHECK_HA(ha_timer_elapsed(tb->t, i, j, &ms));
  napi_value r;
  CHECK_NAPI(napi_create_double(env, (double)ms, &r));
  return r;
}

static napi_value js_timer_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  timer_box* tb = get_timer(env, argv[0]);
  if (!tb) return type_error(env, "not a timer handle");
  if (tb->t) {
    ha_timer* t = tb->t;
    tb->t = NULL;
    CHECK_HA(ha_timer_destroy(t));
  }
  return NULL;
}

/* fwht(x: BigInt, elems, n, device, engine|null) */
static napi_value js_fwht(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (!get_args(env, info, 5, argv)) return NULL;
  void *x, *st;
  double elems;
  int32_t n, device = 0;
  if (!get_ptr(env, argv[0], &x)) return type_error(env, "x must be a BigInt");
  if (napi_get_value_double(env, argv[1], &elems) != napi_ok || elems < 0) return type_error(env, "elems must be >= 0");
  if (napi_get_value_int32(env, argv[2], &n) != napi_ok) return type_error(env, "n must be an integer");
  if (!is_nullish(env, argv[3]) && napi_get_value_int32(env, argv[3], &device) != napi_ok)
    return type_error(env, "device must be an integer");
  if (!stream_of(env, argv[4], &st)) return type_error(env, "the last argument must be an engine handle or null");
  CHECK_HA(ha_fwht(x, (long)elems, n, device, st));
  return NULL;
}

/* shareStream(engine, other): run `engine`'s calls on `other`'s stream, so that work on several engines stays in
   one order (ha_get_stream + ha_set_stream); their calls then never overlap, so `engine` also uses `other`'s
   call-time device buffers (ha_share_scratch) */
static napi_value js_share_stream(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  engine_box* a = get_engine(env, argv[0]);
  engine_box* b = get_engine(env, argv[1]);
  if (!a || !a->e || !b || !b->e) return type_error(env, "both arguments must be live engine handles");
  if (a == b) return type_error(env, "an engine cannot borrow its own stream");
  if (b->owner_box == a) return type_error(env, "the other engine runs on this engine's stream");
  void *st = NULL, *was = NULL;
  CHECK_HA(ha_get_stream(b->e, &st));
  CHECK_HA(ha_get_stream(a->e, &was));
  napi_ref ref;
  CHECK_NAPI(napi_create_reference(env, argv[1], 1, &ref));
  /* the stream first: engines holding one set of call-time buffers must already share a stream */
  int rc = ha_set_stream(a->e, st);
  if (!rc && (rc = ha_share_scratch(a->e, b->e)) != 0) (void)ha_set_stream(a->e, was);
  if (rc) {
    napi_delete_reference(env, ref);
    return throw_status(env, rc);
  }
  unshare_stream(env, a);
  if (!add_borrower(b, a)) {
    napi_delete_reference(env, ref);
    return type_error(env, "out of host memory");
  }
  a->stream_owner = ref;
  a->owner_box = b;
  return NULL;
}

/* embed(table, L, ids: BigInt, x: BigInt, engine|null) */
static napi_value js_embed(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (!get_args(env, info, 5, argv)) return NULL;
  mnb_box* mb = get_mnb(env, argv[0]);
  if (!mb || !mb->w) return type_error(env, "not a MatMulNBits handle");
  int32_t L;
  void *ids, *x, *st;
  if (napi_get_value_int32(env, argv[1], &L) != napi_ok) return type_error(env, "L must be an integer");
  if (!get_ptr(env, argv[2], &ids) || !get_ptr(env, argv[3], &x)) return type_error(env, "ids and x must be BigInt");
  if (!stream_of(env, argv[4], &st)) return type_error(env, "the last argument must be an engine handle or null");
  CHECK_HA(ha_embed(mb->w, L, ids, x, st));
  return NULL;
}

/* addNorm(R, D, nx, x, y|null, w, h, outF32, rows|null, eps, device, engine|null) */
static napi_value js_add_norm(napi_env env, napi_callback_info info) {
  napi_value argv[12];
  if (!get_args(env, info, 12, argv)) return NULL;
  int32_t R, D, nx, of, dev;
  double eps;
  void *x, *y = NULL, *w, *h, *rows = NULL, *st;
  if (napi_get_value_int32(env, argv[0], &R) != napi_ok || napi_get_value_int32(env, argv[1], &D) != napi_ok ||
      napi_get_value_int32(env, argv[2], &nx) != napi_ok || napi_get_value_int32(env, argv[7], &of) != napi_ok ||
      napi_get_value_double(env, argv[9], &eps) != napi_ok || napi_get_value_int32(env, argv[10], &dev) != napi_ok)
    return type_error(env, "R, D, nx, outF32, eps and device must be numbers");
  if (!get_ptr(env, argv[3], &x) || !get_ptr(env, argv[5], &w) || !get_ptr(env, argv[6], &h))
    return type_error(env, "x, w and h must be BigInt");
  if (!is_nullish(env, argv[4]) && !get_ptr(env, argv[4], &y)) return type_error(env, "y must be a BigInt or null");
  if (!is_nullish(env, argv[8]) && !get_ptr(env, argv[8], &rows)) return type_error(env, "rows must be a BigInt or null");
  if (!stream_of(env, argv[11], &st)) return type_error(env, "the last argument must be an engine handle or null");
  CHECK_HA(ha_add_norm(R, D, nx, x, y, (const float*)w, h, of, rows, (float)eps, dev, st));
  return NULL;
}

/* siluMul(L, I, big, mid, device, engine|null) and addBias(L, N, y, c, device, engine|null) */
static napi_value js_silu_mul(napi_env env, napi_callback_info info) {
  napi_value argv[6];
  if (!get_args(env, info, 6, argv)) return NULL;
  int32_t L, I, dev;
  void *big, *mid, *st;
  if (napi_get_value_int32(env, argv[0], &L) != napi_ok || napi_get_value_int32(env, argv[1], &I) != napi_ok ||
      napi_get_value_int32(env, argv[4], &dev) != napi_ok)
    return type_error(env, "L, I and device must be integers");
  if (!get_ptr(env, argv[2], &big) || !get_ptr(env, argv[3], &mid)) return type_error(env, "big and mid must be BigInt");
  if (!stream_of(env, argv[5], &st)) return type_error(env, "the last argument must be an engine handle or null");
  CHECK_HA(ha_silu_mul(L, I, big, mid, dev, st));
  return NULL;
}

static napi_value js_add_bias(napi_env env, napi_callback_info info) {
  napi_value argv[6];
  if (!get_args(env, info, 6, argv)) return NULL;
  int32_t L, N, dev;
  void *y, *c, *st;
  if (napi_get_value_int32(env, argv[0], &L) != napi_ok || napi_get_value_int32(env, argv[1], &N) != napi_ok ||
      napi_get_value_int32(env, argv[4], &dev) != napi_ok)
    return type_error(env, "L, N and device must be integers");
  if (!get_ptr(env, argv[2], &y) || !get_ptr(env, argv[3], &c)) return type_error(env, "y and c must be BigInt");
  if (!stream_of(env, argv[5], &st)) return type_error(env, "the last argument must be an engine handle or null");
  CHECK_HA(ha_add_bias(L, N, y, (const float*)c, dev, st));
  return NULL;
}

/* deviceArch(device) -> "gfx950" (the name ha_device_arch reports) */
static napi_value js_device_arch(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  int32_t dev;
  if (napi_get_value_int32(env, argv[0], &dev) != napi_ok) return type_error(env, "device must be an integer");
  char name[64];
  CHECK_HA(ha_device_arch(dev, name, sizeof(name)));
  napi_value r;
  CHECK_NAPI(napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &r));
  return r;
}

static napi_value init(napi_env env, napi_value exports) {
  const struct {
    const char* name;
    napi_callback fn;
  } fns[] = {
      {"abiVersion", js_abi_version},       {"lastError", js_last_error},
      {"deviceArch", js_device_arch},
      {"create", js_create},                {"destroy", js_destroy},
      {"setParam", js_set_param},           {"forward", js_forward},
      {"snapshotTokens", js_snapshot_tokens}, {"snapshotLayout", js_snapshot_layout},
      {"snapshotRead", js_snapshot_read},   {"snapshotRelease", js_snapshot_release},
      {"deviceAlloc", js_device_alloc},     {"deviceFree", js_device_free},
      {"copyToDevice", js_copy_to_device},  {"copyToHost", js_copy_to_host},
      {"synchronize", js_synchronize},
      {"mnbCreate", js_mnb_create},         {"mnbForward", js_mnb_forward},
      {"mnbDestroy", js_mnb_destroy},       {"fwht", js_fwht},
      {"embed", js_embed},                  {"addNorm", js_add_norm},
      {"siluMul", js_silu_mul},             {"addBias", js_add_bias},
      {"shareStream", js_share_stream},
      {"timerCreate", js_timer_create},     {"timerMark", js_timer_mark},
      {"timerElapsed", js_timer_elapsed},   {"timerDestroy", js_timer_destroy},
  };
  for (size_t i = 0; i < sizeof(fns) / sizeof(fns[0]); i++) {
    napi_value f;
    if (napi_create_function(env, fns[i].name, NAPI_AUTO_LENGTH, fns[i].fn, NULL, &f) != napi_ok ||
        napi_set_named_property(env, exports, fns[i].name, f) != napi_ok)
      return NULL;
  }
  return exports;
}

#ifndef NODE_GYP_MODULE_NAME
#define NODE_GYP_MODULE_NAME ha_napi
#endif
NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
