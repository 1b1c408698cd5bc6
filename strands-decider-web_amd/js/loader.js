'use strict';
/*
 * loader.js: an export of the reference's converter (convert/export_engine.py) into a Torso on this GPU, from Node.
 *
 * The export is a directory with manifest.json {config, shards: [{path, start, bytes, wire?}], tensors: {name:
 * {offset, bytes, dtype, shape, N?, K?, bits?, group?, asym?, had?, wire?, u8?}}, embed?} and the shard files
 * (export_engine.py:33-40,83-85). Each shard becomes one device buffer holding the GPU layout: a tensor is the range
 * [offset - start, + bytes) of its shard (Engine.w, engine.js:174-179). A "wire" shard stores its tensors back to back
 * at t.wire with the f16 scale tensors as 8-bit log codes (web/public/engine/wire.js:1-46), rebuilt here.
 * Quantised tensors (<name>.q with <name>.s, <name>.b) become MatMulNBits handles on those ranges; f32 tensors (norms,
 * biases, the mixers' parameters) are read on the host and handed to Torso.setParam.
 *
 * A lazy embedding (manifest.embed: bundled rows + a row file read by byte range, engine.js:113-172) keeps a table of
 * R bundled rows plus `slots` rows filled on first use; Torso.embedRows maps token ids to table rows.
 */
const fs = require('fs');
const path = require('path');
const ha = require('./engine.js');

// f16 bits -> number
function halfToNumber(h) {
  const e = (h >> 10) & 31, f = h & 1023;
  const v = e === 0 ? f * Math.pow(2, -24) : (1024 + f) * Math.pow(2, e - 25);
  return h & 0x8000 ? -v : v;
}

const f32buf = new Float32Array(1), u32buf = new Uint32Array(f32buf.buffer);
// a positive number rounded to f32 (nearest even, by the typed array), then to f16 bits (nearest even)
function toHalfViaF32(x) {
  f32buf[0] = x;
  const b = u32buf[0], exp = (b >>> 23) & 255, man = b & 0x7fffff;
  const e16 = exp - 127 + 15;
  if (e16 >= 31) return 0x7c00;
  if (e16 > 0) {  // normal: keep 10 mantissa bits, round the 13 dropped ones
    let h = (e16 << 10) | (man >>> 13);
    const rest = man & 0x1fff;
    if (rest > 0x1000 || (rest === 0x1000 && (h & 1))) h += 1;  // a carry into the exponent is the right result
    return h;
  }
  // subnormal f16: value in units of 2^-24, rounded to nearest even
  const u = f32buf[0] * Math.pow(2, 24), fl = Math.floor(u), fr = u - fl;
  return fr > 0.5 || (fr === 0.5 && (fl & 1)) ? fl + 1 : fl;
}

/*
 * N rows of G scale codes starting at src[off]: per row m (f16 bits, u16) and j (u16), then the G codes of all rows;
 * code c = sign << 7 | k stands for sign * fp16(f32(m * 2^(-k j / 4096))). Writes f16 bits into dst (Uint16Array).
 */
function decodeScales(src, off, N, G, dst, dstOff) {
  const d0 = dstOff || 0;
  const dv = new DataView(src.buffer, src.byteOffset + off, 4 * N);
  const codes = off + 4 * N;
  for (let r = 0; r < N; r++) {
    const m = halfToNumber(dv.getUint16(4 * r, true)), j = dv.getUint16(4 * r + 2, true);
    const mag = new Int32Array(128).fill(-1);
    for (let g = 0; g < G; g++) {
      const c = src[codes + r * G + g], k = c & 127;
      if (mag[k] < 0) mag[k] = toHalfViaF32(m * Math.pow(2, -(k * j) / 4096));
      dst[d0 + r * G + g] = mag[k] | ((c & 128) << 8);
    }
  }
}

// The GPU layout of shard s (bytes s.bytes) from its wire form: every tensor of the shard at t.offset - s.start.
function unpackShard(wire, s, tensors) {
  const out = new Uint8Array(s.bytes);
  Object.keys(tensors).forEach((name) => {
    const t = tensors[name];
    if (t.wire === undefined || t.offset < s.start || t.offset >= s.start + s.bytes) return;
    if (!t.u8) {
      out.set(wire.subarray(t.wire, t.wire + t.bytes), t.offset - s.start);
      return;
    }
    const N = t.shape[0], G = t.shape[1], d = new Uint16Array(N * G);
    decodeScales(wire, t.wire, N, G, d, 0);
    out.set(new Uint8Array(d.buffer), t.offset - s.start);
  });
  return out;
}

function readFile(dir, p) {
  const b = fs.readFileSync(path.join(dir, p));
  return new Uint8Array(b.buffer, b.byteOffset, b.byteLength);
}

/*
 * loadTorso(dir, {maxCtx, device, readShard, onProgress}) -> Torso. readShard(path) may supply a shard's bytes (for
 * example from a download); by default shards are read from dir. onProgress(path) is called once per shard after it
 * is on the device, as Engine.create calls it (engine.js:83). The reference's `subgroups` option chooses between two
 * WGSL kernels for the same recurrence; there is one implementation here, so it is accepted and has no effect. The
 * torso's buffers are freed by torso.destroy().
 */
function loadTorso(dir, opts) {
  const o = opts || {};
  const manifest = JSON.parse(fs.readFileSync(path.join(dir, 'manifest.json'), 'utf8'));
  const cfg = Object.assign({}, manifest.config);
  if (cfg.rotary_dim && cfg.head_dim && cfg.partial_rotary_factor === undefined) {
    cfg.partial_rotary_factor = cfg.rotary_dim / cfg.head_dim;  // export_engine.py:83 stores rotary_dim
  }
  const torso = new ha.Torso(cfg, { maxCtx: o.maxCtx || 4096, device: o.device || 0 });
  const tensors = manifest.tensors;
  const host = [];  // GPU-layout bytes of each shard, for the host-side f32 tensors
  const shardBufs = manifest.shards.map((s) => {
    const raw = o.readShard ? o.readShard(s.path) : readFile(dir, s.path);
    const data = s.wire ? unpackShard(raw, s, tensors) : raw;
    host.push(data);
    const buf = torso.lead.alloc(Math.max(data.byteLength, 4)).upload(data);
    if (o.onProgress) o.onProgress(s.path);
    return buf;
  });
  const at = (name) => {  // [shard index, byte offset in the shard] of a tensor
    const t = tensors[name];
    const i = manifest.shards.findIndex((s) => t.offset >= s.start && t.offset < s.start + s.bytes);
    if (i < 0) throw new Error('tensor ' + name + ' lies in no shard');
    return [i, t.offset - manifest.shards[i].start];
  };
  // a quantised tensor is a view of its shard's buffer: the weight handle borrows the buffer (its free() is refused
  // while a handle reads it)
  const ptr = (name) => { const [i, off] = at(name); return new ha.DeviceView(shardBufs[i], off); };
  let lazy = null;
  Object.keys(tensors).forEach((name) => {
    const t = tensors[name];
    if (name.endsWith('.s') || name.endsWith('.b')) return;  // with their .q
    if (name.endsWith('.q')) {
      const base = name.slice(0, -2);
      if (base === 'embed' && manifest.embed) return;  // the lazy table below
      torso.setWeight(base, { q: ptr(name), s: ptr(base + '.s'), b: tensors[base + '.b'] ? ptr(base + '.b') : null,
        N: t.N, K: t.K, bits: t.bits || 4, group: t.group || 32, asym: !!t.asym, had: t.had || 0 });
      return;
    }
    if (t.dtype !== 'float32') throw new Error('tensor ' + name + ': unsupported dtype ' + t.dtype);
    const [i, off] = at(name);
    const bytes = host[i].slice(off, off + t.bytes);
    torso.setParam(name, new Float32Array(bytes.buffer, bytes.byteOffset, t.bytes / 4));
  });
  if (manifest.embed) lazy = initLazyEmbed(torso, dir, manifest, o);
  torso.loaded = { manifest: manifest, shards: shardBufs, lazy: lazy };
  const destroy = torso.destroy.bind(torso);
  torso.destroy = function () {
    // the weight handles first (they borrow the shard and table buffers), then those buffers, then the rest of the
    // torso with its engines (a buffer is freed through the engine that allocated it)
    torso.dropWeights();
    shardBufs.forEach((b) => b.free());
    if (lazy) {
      lazy.bufs.forEach((b) => b.free());
      fs.closeSync(lazy.fd);
    }
    destroy();
  };
  return torso;
}

/*
 * The lazy embedding of manifest.embed {bundle, rows, bundled: R, vocab, slots, parts: [[name, bytes per row]...],
 * row_bytes, wire_row_bytes?, u8?} (engine.js:113-172): the bundle file holds R u32 token ids then their R rows; a
 * row of the row file (token t at t * row bytes) holds each part's bytes in order, its scales as 8-bit codes (a
 * 4-byte m, j header then G codes) when u8. Rows land in table rows R .. R + slots - 1 on first use; when those run
 * out, every fetched row is dropped and the table refills.
 */
function initLazyEmbed(torso, dir, manifest, o) {
  const e = manifest.embed, R = e.bundled, RB = e.wire_row_bytes || e.row_bytes;
  const bundle = o.readShard ? o.readShard(e.bundle) : readFile(dir, e.bundle);
  const rowsPath = path.join(dir, e.rows);
  const parts = e.parts.map(([name, bytes]) => ({ name: name, bytes: bytes,
    buf: torso.lead.alloc((R + e.slots) * bytes) }));
  const E = { slot: new Int32Array(e.vocab).fill(-1), next: R, dyn: [], fetched: 0, evictions: 0,
    bufs: parts.map((p) => p.buf) };
  const put = (data, s0, n) => {  // n rows in the row file's layout into table rows s0 ..
    let off = 0;
    parts.forEach((p) => {
      const part = new Uint8Array(n * p.bytes);
      if (e.u8 && p.name === 'embed.s') {
        const G = p.bytes / 2, d = new Uint16Array(part.buffer);
        for (let r = 0; r < n; r++) decodeScales(data, r * RB + off, 1, G, d, r * G);
        off += 4 + G;
      } else {
        for (let r = 0; r < n; r++) part.set(data.subarray(r * RB + off, r * RB + off + p.bytes), r * p.bytes);
        off += p.bytes;
      }
      p.buf.uploadAt(s0 * p.bytes, part);
    });
  };
  const ids = new Uint32Array(bundle.buffer.slice(bundle.byteOffset, bundle.byteOffset + 4 * R));
  put(bundle.subarray(4 * R), 0, R);
  ids.forEach((t, i) => { E.slot[t] = i; });
  const q = manifest.tensors['embed.q'];
  const fmtT = q || {};
  torso.setWeight('embed', { q: parts[0].buf, s: parts[1].buf, b: parts[2] ? parts[2].buf : null,
    N: R + e.slots, K: fmtT.K || manifest.config.hidden_size, bits: fmtT.bits || 4, group: fmtT.group || 32,
    asym: !!fmtT.asym });
  const fd = fs.openSync(rowsPath, 'r');
  E.fd = fd;  // closed by torso.destroy()
  torso.embedRows = function (tokIds) {
    let need = Array.from(new Set(tokIds)).filter((t) => E.slot[t] < 0);
    if (E.next + need.length > R + e.slots) {  // out of slots: drop every fetched row
      E.dyn.forEach((t) => { E.slot[t] = -1; });
      E.dyn = [];
      E.next = R;
      E.evictions++;
      need = Array.from(new Set(tokIds)).filter((t) => E.slot[t] < 0);
    }
    if (need.length > e.slots) throw new Error('one forward needs more embedding rows than the table holds');
    need.sort((x, y) => x - y);
    const rows = new Uint8Array(need.length * RB);
    need.forEach((t, i) => { fs.readSync(fd, rows, i * RB, RB, t * RB); });
    const s0 = E.next;
    need.forEach((t, i) => { E.slot[t] = s0 + i; E.dyn.push(t); });
    E.next += need.length;
    if (need.length) put(rows, s0, need.length);
    E.fetched += need.length;
    return Array.from(tokIds, (t) => E.slot[t]);
  };
  return E;
}

/*
 * Engine.create(base, {onProgress, fetchShard, subgroups, maxCtx, device}) -> Promise<Torso>: the reference's async
 * constructor (engine.js:63-87) over an export at `base`. It throws, as the reference does, when the device cannot run
 * the engine (engineProblems). fetchShard(url, path, wire) may return a shard's bytes or a promise of them (a
 * download, as the reference's option); by default shards are read from `base` on the file system. Every shard and the
 * lazy embedding's bundle are fetched before the torso is built from them (loadTorso), and onProgress(path) is called
 * once per shard after it is on the device. subgroups is accepted and has no effect (one implementation).
 */
const Engine = {
  create: async function (base, opts) {
    const o = opts || {};
    const problems = ha.engineProblems(o.device || 0);
    if (problems.length) throw new Error("this GPU can't run the engine: " + problems.join(', '));
    const manifest = JSON.parse(fs.readFileSync(path.join(base, 'manifest.json'), 'utf8'));
    const fetched = new Map();
    const want = manifest.shards.map((s) => [s.path, s.wire]);
    if (manifest.embed) want.push([manifest.embed.bundle, undefined]);
    for (const [p, wire] of want) {
      const data = o.fetchShard ? await o.fetchShard(base + '/' + p, p, wire) : readFile(base, p);
      fetched.set(p, data instanceof Uint8Array ? data : new Uint8Array(data));
    }
    return loadTorso(base, { maxCtx: o.maxCtx, device: o.device, onProgress: o.onProgress,
      readShard: (p) => {
        if (!fetched.has(p)) throw new Error('shard ' + p + ' was not fetched');
        return fetched.get(p);
      } });
  },
};

module.exports = { Engine: Engine, loadTorso: loadTorso, decodeScales: decodeScales, unpackShard: unpackShard };
