'use strict';
// Drives the MatMulNBits projection API of the Node host (strands-decider-web_amd/js/engine.js) the way the
// reference's Engine.forward drives its matmul dispatch (engine.js:236-246): packed weights and scales uploaded
// once, then y = a x W^T for several row counts M, on the engine's stream. Files in the directory named by the
// first argument: spec.json {N, K, Ms, bits, group, asym}, q.bin (u32 blocks), s.bin (f16 scales), b.bin (f16
// biases, asymmetric only), a.bin (f16 rows, max(Ms) x K); writes y_<M>.bin (f16, M x N) and fwht.bin (the FWHT of
// a's first row block, n = 64).
const fs = require('fs');
const path = require('path');
const ha = require(path.join(__dirname, '..', '..', 'strands-decider-web_amd', 'js', 'engine.js'));

const dir = process.argv[2];
const spec = JSON.parse(fs.readFileSync(path.join(dir, 'spec.json'), 'utf8'));
const engine = ha.Engine.createSync({ layer_types: ['linear_attention'] }, { batch: 1, maxCtx: 64 });

function upload(file) {
  const buf = fs.readFileSync(path.join(dir, file));
  const u8 = new Uint8Array(buf.buffer, buf.byteOffset, buf.byteLength);
  return engine.alloc(u8.byteLength).upload(u8);
}

const q = upload('q.bin');
const s = upload('s.bin');
const b = spec.asym ? upload('b.bin') : null;
const a = upload('a.bin');
const w = new ha.MatMulNBits(engine, spec.N, spec.K, q, s, b, { bits: spec.bits, group: spec.group, asym: spec.asym });
spec.Ms.forEach(function (M) {
  const y = engine.alloc(M * spec.N * 2);
  w.forward(M, a, y);
  const host = new Uint16Array(M * spec.N);
  y.download(host);  // synchronous on the engine's stream, after the matmul
  fs.writeFileSync(path.join(dir, 'y_' + M + '.bin'), Buffer.from(host.buffer));
  y.free();
});
let threw = '';
try { w.forward(0, a, a); } catch (e) { threw = e.code + ' ' + e.message; }
if (threw.indexOf('HA_') !== 0) throw new Error('M = 0 did not throw a status error: ' + threw);
// the handle borrows q and s: freeing them under it is refused, and the handle keeps working
let borrowed = '';
try { q.free(); } catch (e) { borrowed = e.code; }
if (borrowed !== 'HA_BORROWED' || q.ptr === null) throw new Error('free() of a borrowed buffer was not refused');
// a second handle on views of the same buffers borrows them as well
const w2 = new ha.MatMulNBits(engine, spec.N, spec.K, new ha.DeviceView(q, 0), new ha.DeviceView(s, 0),
  b ? new ha.DeviceView(b, 0) : null, { bits: spec.bits, group: spec.group, asym: spec.asym });
w.destroy();
w.destroy();  // idempotent
borrowed = '';
try { s.free(); } catch (e) { borrowed = e.code; }
if (borrowed !== 'HA_BORROWED') throw new Error('free() of a buffer borrowed through a view was not refused');
w2.destroy();
// an engine whose stream another engine borrows cannot be destroyed first
const e2 = ha.Engine.createSync({ layer_types: ['full_attention'] }, { batch: 1, maxCtx: 64 });
const native = require(path.join(__dirname, '..', '..', 'strands-decider-web_amd', 'js', 'ha_napi.node'));
native.shareStream(e2._h, engine._h);
let shared = '';
try { engine.destroy(); } catch (e) { shared = e.code; }
if (shared !== 'HA_STREAM_SHARED' || engine._h === null) throw new Error('destroying a stream owner was not refused');
e2.destroy();
ha.fwht(engine, a, 64, 64);
const f = new Uint16Array(64);
a.download(f);
fs.writeFileSync(path.join(dir, 'fwht.bin'), Buffer.from(f.buffer));
[q, s, a].concat(b ? [b] : []).forEach(function (x) { x.free(); });
engine.destroy();
console.log(JSON.stringify({ ok: true }));
