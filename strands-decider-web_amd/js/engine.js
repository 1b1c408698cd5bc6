'use strict';
/*
 * engine.js: the Node host side of the MI355X hybrid-attention path, shaped like the reference engine's API
 * (web/public/engine/engine.js): Engine.create(...) (engine.js:63), engine.forward(..., {cache, keepCache,
 * timestamps}) returning {cache, gpu_ms, layers} (engine.js:313-375), and snapshots with P and release()
 * (engine.js:349-362). It drives the HIP kernels through the N-API addon ha_napi.node over the C ABI in
 * include/ha.h; there is no fallback: if the addon or the library cannot load, require() throws.
 *
 * What is passed per layer is the token-mixer input that the reference's projections produce on the GPU: rows of
 * the fused in_proj output (linear layers, [batch][L][linStride]) or of the fused qkv projection (full layers,
 * [batch][L][fullStride]) in device memory, and an output buffer ([batch][L][H*DV] or [batch][L][HQ*HD]).
 * DeviceBuffer wraps device memory for callers without a HIP allocator of their own.
 *
 * Written for Node >= 12 (no optional chaining, no nullish coalescing).
 */
const path = require('path');

const native = require(path.join(__dirname, 'ha_napi.node'));

const F32 = 0;
const F16 = 1;
const CHUNKED = 0;  // the engine picks CHUNKED_SPLIT, CHUNKED_PAIRED or CHUNKED_FUSED from the batch shape
const SEQUENTIAL = 1;
const CHUNKED_FUSED = 2;
const CHUNKED_SPLIT = 3;
const CHUNKED_PAIRED = 4;
// adapter: a projection stand-in with no token mixer (engine.js:256-261); its forward buffers may be null
const LAYER_KIND = { linear_attention: 0, full_attention: 1, adapter: 2 };

function pick(obj, key, def) {
  return obj !== undefined && obj !== null && obj[key] !== undefined && obj[key] !== null ? obj[key] : def;
}

function dtypeCode(d, def) {
  if (d === undefined || d === null) return def;
  if (d === F32 || d === 'f32' || d === 'float32') return F32;
  if (d === F16 || d === 'f16' || d === 'float16') return F16;
  throw new TypeError('unsupported dtype ' + d);
}

/*
 * Engine config from the manifest's config object (convert/export_engine.py:83 writes the Hugging Face config keys:
 * layer_types, linear_num_key_heads, linear_key_head_dim, linear_value_head_dim, linear_conv_kernel_dim,
 * num_attention_heads, num_key_value_heads, head_dim, partial_rotary_factor, rope_theta, rms_norm_eps) plus
 * runtime options {batch, maxCtx, linDtype, fullDtype, linGnorm}.
 */
function configFromManifest(manifest, opts) {
  const m = manifest || {};
  const o = opts || {};
  const types = pick(m, 'layer_types', null);
  if (!Array.isArray(types)) throw new TypeError('manifest config needs layer_types');
  const layerKinds = types.map(function (t) {
    if (!(t in LAYER_KIND)) throw new TypeError('unsupported layer type ' + t + ' (this engine runs the token mixers)');
    return LAYER_KIND[t];
  });
  const H = pick(m, 'linear_num_key_heads', 16);
  const DK = pick(m, 'linear_key_head_dim', 128);
  const DV = pick(m, 'linear_value_head_dim', 128);
  const HQ = pick(m, 'num_attention_heads', 8);
  const HK = pick(m, 'num_key_value_heads', 2);
  const HD = pick(m, 'head_dim', 256);
  const rp = pick(m, 'rope_parameters', null);
  const prf = pick(rp, 'partial_rotary_factor', pick(m, 'partial_rotary_factor', 0.25));
  return {
    layerKinds: layerKinds,
    batch: pick(o, 'batch', 1),
    maxCtx: pick(o, 'maxCtx', 4096),
    H: H, DK: DK, DV: DV,
    convK: pick(m, 'linear_conv_kernel_dim', 4),
    // fused in_proj row: q | k | v | z | a | b (export_engine.py:52), padded to a multiple of 64 columns
    linStride: pick(o, 'linStride', Math.ceil((2 * H * DK + 2 * H * DV + 2 * H) / 64) * 64),
    linDtype: dtypeCode(pick(o, 'linDtype', null), F32),
    linGnorm: pick(o, 'linGnorm', true) ? 1 : 0,
    HQ: HQ, HK: HK, HD: HD,
    rotDim: Math.round(HD * prf),
    fullStride: pick(o, 'fullStride', 2 * HQ * HD + 2 * HK * HD),
    fullDtype: dtypeCode(pick(o, 'fullDtype', null), F16),
    ropeTheta: pick(rp, 'rope_theta', pick(m, 'rope_theta', 1e7)),
    eps: pick(m, 'rms_norm_eps', 1e-6),
  };
}

class DeviceBuffer {
  constructor(engine, bytes) {
    this._engine = engine;
    this.bytes = bytes;
    this.ptr = native.deviceAlloc(engine._h, bytes);
    this._borrows = 0;  // MatMulNBits handles reading this buffer (the C handle keeps only its address)
  }
  upload(typedArray) {
    if (typedArray.byteLength > this.bytes) throw new RangeError('upload larger than the buffer');
    native.copyToDevice(this._engine._h, this.ptr, typedArray);
    return this;
  }
  uploadAt(offset, typedArray) {
    if (offset < 0 || offset + typedArray.byteLength > this.bytes) throw new RangeError('upload outside the buffer');
    native.copyToDevice(this._engine._h, this.ptr + BigInt(offset), typedArray);
    return this;
  }
  download(typedArray) {
    if (typedArray.byteLength > this.bytes) throw new RangeError('download larger than the buffer');
    native.copyToHost(this._engine._h, typedArray, this.ptr);
    return typedArray;
  }
  // Frees the device memory. Refused while a MatMulNBits handle borrows the buffer: the handle would go on reading
  // memory already returned to the allocator.
  free() {
    if (this._borrows > 0) {
      const e = new Error('device buffer is borrowed by ' + this._borrows + ' MatMulNBits handle(s); destroy them first');
      e.code = 'HA_BORROWED';
      throw e;
    }
    if (this.ptr !== null) {
      native.deviceFree(this._engine._h, this.ptr);
      this.ptr = null;
    }
  }
}

// A byte offset into a DeviceBuffer: a tensor that lives inside a larger buffer (a range of a loaded shard). A
// MatMulNBits handle built on views borrows the underlying buffer.
class DeviceView {
  constructor(buf, offset) {
    if (!(buf instanceof DeviceBuffer)) throw new TypeError('a DeviceView needs a DeviceBuffer');
    if (offset < 0 || offset > buf.bytes) throw new RangeError('view offset outside the buffer');
    this.buf = buf;
    this.offset = offset;
  }
}

class Snapshot {
  constructor(handle) {
    this._h = handle;
    this.P = native.snapshotTokens(handle);
  }
  layout() {
    return native.snapshotLayout(this._h);
  }
  // what: 'state' | 'tail' (linear layers), 'K' | 'V' (full layers); into a TypedArray of the right size
  read(layer, what, typedArray) {
    native.snapshotRead(this._h, layer, what, typedArray);
    return typedArray;
  }
  // frees the snapshot's device memory; idempotent, like the reference's release() (engine.js:361)
  release() {
    native.snapshotRelease(this._h);
  }
}

function ptrOf(x) {
  if (x === null || x === undefined) return BigInt(0);  // only an adapter layer may pass none
  if (typeof x === 'bigint') return x;
  if (x instanceof DeviceBuffer) {
    if (x.ptr === null) throw new Error('device buffer was freed');
    return x.ptr;
  }
  if (x instanceof DeviceView) return ptrOf(x.buf) + BigInt(x.offset);
  throw new TypeError('layer buffers must be DeviceBuffer or BigInt device pointers');
}

/*
 * Why HIP device `device` (default 0) cannot run the engine: an empty array if it can. The counterpart of the
 * reference's adapter guard engineProblems(adapter) (engine.js:50-52, which asks for shader-f16): every kernel here
 * is built for gfx950 only. The reference's subgroups32(adapter) chooses between two WGSL variants of one kernel; a
 * gfx950 wavefront is 64 wide and there is one implementation, so it has no counterpart.
 */
function engineProblems(device) {
  const d = device === undefined || device === null ? 0 : device;
  let arch;
  try {
    arch = native.deviceArch(d);
  } catch (e) {
    return [e.message];
  }
  return arch === 'gfx950' ? [] : ['HIP device ' + d + ' is ' + arch + '; the kernels are built for gfx950 only'];
}

/*
 * The projection kernel a forward over L rows runs: the name Torso.forward returns as `kernel`, like the reference's
 * plan.kernel (its matmul kernel key chosen by L, engine.js:17-33,285,367). ha_mnb_forward reads the packed weights
 * with a GEMV kernel up to 64 rows and runs the tiled MFMA GEMM beyond (include/ha.h).
 */
function projectionKernel(L) {
  return L <= 64 ? 'mnb_gemv' : 'mnb_gemm';
}

class Engine {
  // The reference's Engine.create is async (engine.js:63); so is this one. opts: {device}
  static create(config, opts) {
    return new Promise(function (resolve) {
      resolve(new Engine(config, opts));
    });
  }
  static createSync(config, opts) {
    return new Engine(config, opts);
  }
  constructor(config, opts) {
    this.config = Array.isArray(config.layerKinds) ? config : configFromManifest(config, opts);
    this.device = pick(opts, 'device', 0);
    this._h = native.create(this.config, this.device);
  }
  // per-layer tensor under its manifest name (conv, neg_exp_A, dt_bias, gnorm, q_norm, k_norm), Float32Array
  setParam(layer, name, data) {
    native.setParam(this._h, layer, name, data);
  }
  alloc(bytes) {
    return new DeviceBuffer(this, bytes);
  }
  /*
   * One forward over L new rows of every sequence (engine.js:313). inputs / outputs: one device buffer per layer.
   * options: {cache: Snapshot to resume from, keepCache: return a snapshot of the context after this call,
   *           timestamps: report gpu_ms, layerMs: per-layer GPU ms,
   *           recurrence: CHUNKED | SEQUENTIAL | CHUNKED_FUSED | CHUNKED_SPLIT | CHUNKED_PAIRED}
   * Throws (as the reference does at engine.js:316) when the cached plus new rows exceed maxCtx.
   */
  forward(L, inputs, outputs, options) {
    const o = options || {};
    const cache = pick(o, 'cache', null);
    const r = native.forward(this._h, L, inputs.map(ptrOf), outputs.map(ptrOf), cache ? cache._h : null,
      !!pick(o, 'keepCache', false), {
        recurrence: pick(o, 'recurrence', CHUNKED),
        timestamps: pick(o, 'timestamps', false) ? 1 : 0,
        layerMs: pick(o, 'layerMs', false) ? 1 : 0,
        sync: 0,
      });
    const out = { cache: r.snapshot ? new Snapshot(r.snapshot) : null };
    if (r.gpuMs !== undefined) out.gpu_ms = r.gpuMs;
    if (r.layerMs !== undefined) out.layers = r.layerMs;
    return out;
  }
  synchronize() {
    native.synchronize(this._h);
  }
  destroy() {
    if (this._h) {
      native.destroy(this._h);
      this._h = null;
    }
  }
}

/*
 * A quantised projection weight (MatMulNBits, the formats of web/public/gemmbench/kernels.js:1-14) and its matmul,
 * y[M][N] = a[M][K] x W^T in f16 (the matmul dispatch of engine.js:236-246). q (packed blocks [N][K/32][bits] u32),
 * s (f16 scales [N][K/group]) and b (f16 biases, asymmetric formats only) are device memory the handle borrows: given
 * as DeviceBuffers, the handle holds them and their free() is refused until destroy(); given as BigInt addresses,
 * keeping them alive is the caller's duty. format {bits: 2|3|4, group: 32|64, asym: bool} defaults to the exporter's
 * int4 / 32 / symmetric. The matmuls run on the engine's stream, in order with its token mixers.
 */
class MatMulNBits {
  constructor(engine, N, K, q, s, b, format) {
    const f = format || {};
    this.engine = engine;
    this.N = N;
    this.K = K;
    this._h = native.mnbCreate(N, K, { bits: pick(f, 'bits', 4), group: pick(f, 'group', 32), asym: pick(f, 'asym', false) ? 1 : 0 },
      ptrOf(q), ptrOf(s), b === undefined || b === null ? null : ptrOf(b), engine ? engine.device : pick(f, 'device', 0));
    this._borrowed = [q, s, b].map((x) => (x instanceof DeviceView ? x.buf : x)).filter((x) => x instanceof DeviceBuffer);
    this._borrowed.forEach((x) => { x._borrows++; });
  }
  forward(M, a, y) {
    native.mnbForward(this._h, M, ptrOf(a), ptrOf(y), this.engine ? this.engine._h : null);
  }
  destroy() {
    if (this._h) {
      native.mnbDestroy(this._h);
      this._h = null;
      this._borrowed.forEach((x) => { x._borrows--; });
      this._borrowed = [];
    }
  }
}

// In-place orthonormal Walsh-Hadamard transform of every n-block of an f16 device buffer of `elems` values: the
// input rotation of a weight exported with `had: n` (web/public/engine/wgsl.js:94-110), on the engine's stream.
function fwht(engine, x, elems, n) {
  native.fwht(ptrOf(x), elems, n, engine ? engine.device : 0, engine ? engine._h : null);
}

// In-place orthonormal Walsh-Hadamard transform of each n-block of a host Float32Array row range (the CPU unrotate
// of a rotated torso's output, engine.js:365-366).
function fwhtHost(a, off, n) {
  for (let h = 1; h < n; h *= 2) {
    for (let i = 0; i < n; i += 2 * h) {
      for (let j = i; j < i + h; j++) {
        const x = a[off + j], y = a[off + j + h];
        a[off + j] = x + y;
        a[off + j + h] = x - y;
      }
    }
  }
  const s = 1 / Math.sqrt(n);
  for (let j = 0; j < n; j++) a[off + j] *= s;
}

/*
 * The whole torso forward of the reference engine (web/public/engine/engine.js:247-285, 313-376), batch 1, on this GPU:
 * EMBED; per layer the input norm (with the residual add from layer 1 on), the in_proj / qkv projection, the token
 * mixer, out_proj / o_proj, the post norm, gate_up, SILU_MUL and down (an adapter layer: proj + bias); then the final
 * norm of the requested rows, f32, and the CPU unrotate of a rotated torso. Every step runs on one stream.
 *
 * Tensors by manifest name (convert/export_engine.py): setWeight(name, {q, s, b, N, K, bits, group, asym, had}) for
 * the quantised ones ("embed", "layers.<i>.in_proj" | "qkv" | "out_proj" | "o_proj" | "gate_up" | "down" | "proj");
 * setParam(name, Float32Array) for "final_norm", "layers.<i>.in_norm" | "post_norm" | "bias" (uploaded here) and the
 * token mixers' "conv" | "neg_exp_A" | "dt_bias" | "gnorm" | "q_norm" | "k_norm" (forwarded to the layer's mixer).
 * A quantised tensor's device buffers are the caller's and must stay alive.
 */
class Torso {
  constructor(manifest, opts) {
    const o = opts || {};
    this.manifest = manifest;
    this.D = pick(manifest, 'hidden_size', 2048);
    this.I = pick(manifest, 'intermediate_size', 6144);
    this.device = pick(o, 'device', 0);
    this.types = manifest.layer_types.slice();
    this.unrotate = pick(o, 'unrotate', pick(manifest, 'unrotate', null));
    this.mixers = this.types.map((t) => {
      if (t === 'adapter') return null;
      return new Engine(configFromManifest(Object.assign({}, manifest, { layer_types: [t] }),
        { batch: 1, maxCtx: pick(o, 'maxCtx', 4096), linDtype: F16, fullDtype: F16 }), { device: this.device });
    });
    this.lead = this.mixers.find((m) => m !== null) || new Engine(configFromManifest({ layer_types: ['adapter'] },
      { batch: 1 }), { device: this.device });
    this.mixers.forEach((m) => { if (m && m !== this.lead) native.shareStream(m._h, this.lead._h); });
    this.weights = {};
    this.vectors = {};
    this.embedRows = null;  // optional ids -> rows of the embedding table (a lazily filled table, loader.js)
  }
  setWeight(name, w) {
    const h = new MatMulNBits(this.lead, w.N, w.K, w.q, w.s, pick(w, 'b', null),
      { bits: pick(w, 'bits', 4), group: pick(w, 'group', 32), asym: pick(w, 'asym', false) });
    if (this.weights[name]) this.weights[name].h.destroy();
    this.weights[name] = { h: h, N: w.N, K: w.K, had: pick(w, 'had', 0) };
  }
  // Destroys the weight handles, so that the caller may free the device buffers they borrow (before destroy(), which
  // destroys the engine those buffers were allocated on).
  dropWeights() {
    Object.keys(this.weights).forEach((k) => this.weights[k].h.destroy());
    this.weights = {};
  }
  setParam(name, data) {
    const m = /^layers\.(\d+)\.(conv|neg_exp_A|dt_bias|gnorm|q_norm|k_norm)$/.exec(name);
    if (m) {
      const e = this.mixers[+m[1]];
      if (!e) throw new Error('layer ' + m[1] + ' has no token mixer');
      e.setParam(0, m[2], data);
      return;
    }
    if (this.vectors[name]) this.vectors[name].free();
    this.vectors[name] = this.lead.alloc(data.byteLength).upload(data);
  }
  _w(name) {
    const w = this.weights[name];
    if (!w) throw new Error('no tensor ' + name);
    return w;
  }
  _v(name) {
    const v = this.vectors[name];
    if (!v) throw new Error('no tensor ' + name);
    return v;
  }
  // One step of the forward: with a profile running, timestamps on the shared stream before and after it.
  _step(label, fn) {
    const pr = this._prof;
    if (!pr) return fn();
    if (2 * pr.labels.length + 2 > pr.cap) throw new Error('profile: more steps than timestamps');
    native.timerMark(pr.timer, 2 * pr.labels.length, this.lead._h);
    const r = fn();
    native.timerMark(pr.timer, 2 * pr.labels.length + 1, this.lead._h);
    pr.labels.push(label);
    return r;
  }
  _matmul(L, a, name, y, label) {
    const w = this._w(name);
    if (w.had) {  // a is not read again
      this._step(label + '/had', () => native.fwht(a.ptr, L * w.K, w.had, this.device, this.lead._h));
    }
    this._step(label, () => w.h.forward(L, a, y));
    return w.N;
  }
  _norm(R, nx, x, y, wname, h, outF32, rows) {
    native.addNorm(R, this.D, nx, x.ptr, y ? y.ptr : null, this._v(wname).ptr, h.ptr, outF32 ? 1 : 0,
      rows ? rows.ptr : null, pick(this.manifest, 'rms_norm_eps', 1e-6), this.device, this.lead._h);
  }
  /*
   * ids: token rows of the embedding table; rows: indices into ids whose final-normed hidden states are returned
   * (default all). options {cache, keepCache} as Engine.forward (the cache is {P, ids, layers, release()}), and the
   * reference's diagnostics (engine.js:313-376):
   *   timestamps: gpu_ms, the GPU time from the embedding to the final norm;
   *   debugLayers: layers[i - 1] = the residual stream x entering layer i >= 1 (f32 [L][D], after the residual add
   *     that opens the layer: the output of layer i - 1), read back between the layers.
   * Returns {hidden: Float32Array(rows.length * D), d: D, kernel (the projection kernel, projectionKernel(L)), cache,
   * fetch_ms (host time of embedRows)[, gpu_ms][, layers]}.
   */
  forward(ids, rows, options) {
    const o = options || {};
    const L = ids.length, D = this.D, I = this.I;
    const cache = pick(o, 'cache', null), keep = !!pick(o, 'keepCache', false);
    const debug = !!pick(o, 'debugLayers', false), stamps = !!pick(o, 'timestamps', false);
    const R = rows ? rows : Array.from({ length: L }, (_, i) => i);
    let maxN = 2 * I;
    Object.keys(this.weights).forEach((k) => { maxN = Math.max(maxN, this.weights[k].N); });
    const t0 = process.hrtime.bigint();
    const tableRows = this.embedRows ? this.embedRows(ids) : ids;
    const fetchMs = Number(process.hrtime.bigint() - t0) / 1e6;
    const bufs = this._work(L, Math.max(R.length, 1), maxN);
    bufs.ids.upload(Uint32Array.from(tableRows));
    const snaps = [], layers = [];
    const timer = stamps ? native.timerCreate(this.device, 2) : null;
    try {
      if (timer) native.timerMark(timer, 0, this.lead._h);
      this._step('embed', () => native.embed(this._w('embed').h._h, L, bufs.ids.ptr, bufs.x.ptr, this.lead._h));
      this.types.forEach((t, i) => {
        const P = 'layers.' + i + '.', S = 'L' + i + '/';
        this._step(S + 'in_norm', () => this._norm(L, L, bufs.x, i > 0 ? bufs.y : null, P + 'in_norm', bufs.h, false,
          null));
        if (debug && i > 0) layers.push(bufs.x.download(new Float32Array(L * D)));
        if (t === 'adapter') {  // x += proj(rms_norm(x)) + bias, the add in the next norm (engine.js:256-261)
          this._matmul(L, bufs.h, P + 'proj', bufs.y, S + 'proj');
          this._step(S + 'bias', () => native.addBias(L, D, bufs.y.ptr, this._v(P + 'bias').ptr, this.device,
            this.lead._h));
          snaps.push(null);
          return;
        }
        const lin = t === 'linear_attention';
        const stride = lin ? this.mixers[i].config.linStride : this.mixers[i].config.fullStride;
        const pname = lin ? 'in_proj' : 'qkv';
        if (this._w(P + pname).N !== stride) {
          throw new Error(P + pname + ' has ' + this._w(P + pname).N + ' columns, the mixer reads rows of ' + stride);
        }
        this._matmul(L, bufs.h, P + pname, bufs.big, S + pname);
        const r = this._step(S + (lin ? 'gdn' : 'attn'), () => this.mixers[i].forward(L, [bufs.big], [bufs.o],
          { cache: cache ? cache.layers[i] : null, keepCache: keep }));
        snaps.push(r.cache);
        this._matmul(L, bufs.o, P + (lin ? 'out_proj' : 'o_proj'), bufs.y, S + (lin ? 'out_proj' : 'o_proj'));
        this._step(S + 'post_norm', () => this._norm(L, L, bufs.x, bufs.y, P + 'post_norm', bufs.h, false, null));
        this._matmul(L, bufs.h, P + 'gate_up', bufs.big, S + 'gate_up');
        this._step(S + 'silu', () => native.siluMul(L, I, bufs.big.ptr, bufs.mid.ptr, this.device, this.lead._h));
        this._matmul(L, bufs.mid, P + 'down', bufs.y, S + 'down');
      });
      const out = new Float32Array(R.length * D);
      if (R.length) {
        bufs.rows.upload(Uint32Array.from(R));
        this._step('final_norm', () => this._norm(R.length, L, bufs.x, bufs.y, 'final_norm', bufs.out, true,
          bufs.rows));
      }
      if (timer) native.timerMark(timer, 1, this.lead._h);
      if (R.length) bufs.out.download(out);  // synchronous on the shared stream
      const c = this.unrotate;  // rotated torso: the original basis is c * FWHT(row) (engine.js:365-366)
      if (c) for (let r = 0; r < R.length; r++) { fwhtHost(out, r * D, D); for (let j = 0; j < D; j++) out[r * D + j] *= c[j]; }
      let snap = null;
      if (keep) {
        snap = { P: (cache ? cache.P : 0) + L, ids: (cache ? cache.ids : []).concat(Array.from(ids)), layers: snaps,
          release: function () { snaps.forEach((s) => { if (s) s.release(); }); } };
      }
      const res = { hidden: out, d: D, kernel: projectionKernel(L), cache: snap, fetch_ms: fetchMs };
      if (timer) res.gpu_ms = native.timerElapsed(timer, 0, 1);
      if (debug) res.layers = layers;
      return res;
    } finally {
      this.lead.synchronize();  // the next call may overwrite the work buffers
      if (timer) native.timerDestroy(timer);
    }
  }
  /*
   * GPU time of every step of a forward over ids (options as forward), summed over the layers by the step's name
   * without its layer prefix (embed, in_norm, in_proj, gdn, out_proj, qkv, attn, o_proj, post_norm, gate_up, silu,
   * down, proj, bias, .../had, final_norm), in ms to 2 decimals, largest first (engine.js:292-307). Diagnostics
   * only: a timestamp pair brackets every step. The reference's `force` (its matmul kernel override) has no
   * counterpart here: there is one projection kernel.
   */
  profile(ids, options) {
    const cap = 2 * (3 + 16 * this.types.length);
    this._prof = { timer: native.timerCreate(this.device, cap), cap: cap, labels: [] };
    try {
      this.forward(ids, [], options);
      const by = {};
      this._prof.labels.forEach((label, k) => {
        const name = label.replace(/^L\d+\//, '');
        by[name] = (by[name] || 0) + native.timerElapsed(this._prof.timer, 2 * k, 2 * k + 1);
      });
      const out = {};
      Object.keys(by).sort((a, b) => by[b] - by[a]).forEach((k) => { out[k] = +by[k].toFixed(2); });
      return out;
    } finally {
      native.timerDestroy(this._prof.timer);
      this._prof = null;
    }
  }
  // Work buffers for L rows and R returned rows, kept between calls and grown when a call needs more (no device
  // allocation on the steady path).
  _work(L, R, maxN) {
    const D = this.D, I = this.I;
    const need = { ids: L * 4, x: L * D * 4, h: L * D * 2, big: L * maxN * 2, o: L * D * 2, y: L * D * 2,
      mid: L * I * 2, rows: R * 4, out: R * D * 4 };
    if (!this._bufs) this._bufs = {};
    Object.keys(need).forEach((k) => {
      const b = this._bufs[k];
      if (!b || b.bytes < need[k]) {
        if (b) b.free();
        this._bufs[k] = this.lead.alloc(need[k]);
      }
    });
    return this._bufs;
  }
  destroy() {
    if (this._bufs) Object.keys(this._bufs).forEach((k) => this._bufs[k].free());
    this._bufs = null;
    Object.keys(this.weights).forEach((k) => this.weights[k].h.destroy());
    Object.keys(this.vectors).forEach((k) => this.vectors[k].free());
    this.weights = {};
    this.vectors = {};
    this.mixers.forEach((m) => { if (m && m !== this.lead) m.destroy(); });
    if (this.lead) this.lead.destroy();
    this.lead = null;
  }
}

module.exports = {
  Engine: Engine,
  Torso: Torso,
  MatMulNBits: MatMulNBits,
  fwht: fwht,
  Snapshot: Snapshot,
  DeviceBuffer: DeviceBuffer,
  DeviceView: DeviceView,
  configFromManifest: configFromManifest,
  F32: F32,
  F16: F16,
  CHUNKED: CHUNKED,
  SEQUENTIAL: SEQUENTIAL,
  CHUNKED_FUSED: CHUNKED_FUSED,
  CHUNKED_SPLIT: CHUNKED_SPLIT,
  CHUNKED_PAIRED: CHUNKED_PAIRED,
  abiVersion: native.abiVersion,
  engineProblems: engineProblems,
  projectionKernel: projectionKernel,
};
