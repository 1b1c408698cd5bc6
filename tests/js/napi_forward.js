'use strict';
// Drives the Node host API (strands-decider-web_amd/js/engine.js) the way the reference's callers drive
// Engine.forward: a prefix forward that keeps its cache, then a suffix forward resumed from that snapshot, then
// release(). Inputs and outputs are raw little-endian files in a directory named by the first argument:
//   spec.json {kinds, batch, maxCtx, T0, T1, params: [{name: file}...], recurrence (optional)}
//   in_<layer>_<part>.bin  rows in the layer kind's dtype; out_<layer>_<part>.bin written back the same way
//   state_<layer>.bin      snapshot state of linear layers after the prefix
const fs = require('fs');
const path = require('path');
const ha = require(path.join(__dirname, '..', '..', 'strands-decider-web_amd', 'js', 'engine.js'));

const dir = process.argv[2];
const spec = JSON.parse(fs.readFileSync(path.join(dir, 'spec.json'), 'utf8'));
const types = spec.kinds;
const engine = ha.Engine.createSync({ layer_types: types }, { batch: spec.batch, maxCtx: spec.maxCtx });
const c = engine.config;

function readTyped(file, kind) {
  const buf = fs.readFileSync(file);
  const ab = buf.buffer.slice(buf.byteOffset, buf.byteOffset + buf.byteLength);
  return kind === 'f32' ? new Float32Array(ab) : new Uint16Array(ab);
}

types.forEach(function (t, i) {
  Object.keys(spec.params[i]).forEach(function (name) {
    engine.setParam(i, name, readTyped(path.join(dir, spec.params[i][name]), 'f32'));
  });
});

function run(part, L, cache, keep) {
  const ins = [];
  const outs = [];
  const esz = [];
  types.forEach(function (t, i) {
    const lin = t === 'linear_attention';
    const dt = lin ? c.linDtype : c.fullDtype;
    const e = dt === ha.F32 ? 4 : 2;
    const x = readTyped(path.join(dir, 'in_' + i + '_' + part + '.bin'), e === 4 ? 'f32' : 'f16');
    ins.push(engine.alloc(x.byteLength).upload(x));
    outs.push(engine.alloc(spec.batch * L * (lin ? c.H * c.DV : c.HQ * c.HD) * e));
    esz.push(e);
  });
  const r = engine.forward(L, ins, outs, { cache: cache, keepCache: keep, timestamps: true,
    recurrence: spec.recurrence === undefined ? ha.CHUNKED : spec.recurrence });
  outs.forEach(function (o, i) {
    const host = esz[i] === 4 ? new Float32Array(o.bytes / 4) : new Uint16Array(o.bytes / 2);
    o.download(host);
    fs.writeFileSync(path.join(dir, 'out_' + i + '_' + part + '.bin'), Buffer.from(host.buffer));
  });
  ins.concat(outs).forEach(function (b) { b.free(); });
  if (typeof r.gpu_ms !== 'number' || !(r.gpu_ms >= 0)) throw new Error('gpu_ms missing');
  return r;
}

const first = run(0, spec.T0, null, true);
const snap = first.cache;
if (!snap || snap.P !== spec.T0) throw new Error('snapshot P ' + (snap && snap.P));
types.forEach(function (t, i) {
  if (t !== 'linear_attention') return;
  const s = new Float32Array(spec.batch * c.H * c.DK * c.DV);
  snap.read(i, 'state', s);
  fs.writeFileSync(path.join(dir, 'state_' + i + '.bin'), Buffer.from(s.buffer));
});
run(1, spec.T1, snap, false);
snap.release();
snap.release();  // idempotent, as in the reference
let threw = '';
try { run(1, spec.T1, snap, false); } catch (e) { threw = e.code + ' ' + e.message; }
if (threw.indexOf('released') < 0) throw new Error('resume from a released snapshot did not throw: ' + threw);
engine.destroy();
console.log(JSON.stringify({ ok: true, P: spec.T0, layout: 'done' }));
