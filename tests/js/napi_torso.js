'use strict';
// Drives the Node torso API (strands-decider-web_amd/js/engine.js Torso) the way the reference's callers drive
// Engine.forward (engine.js:313-376): a prefix forward of L0 tokens that keeps its cache, then a resumed forward of
// L1 more tokens, returning final-normed hidden rows. Files in the directory named by the first argument:
//   spec.json {types, D, I, L0, L1, rows0, rows1, weights: {name: {N, K}}, vectors: [names], mixer: [[i, name]...]}
//   w_<name>.q / w_<name>.s (u32 blocks, f16 scales), v_<name>.bin (f32), ids0.bin / ids1.bin (u32)
// and writes hidden0.bin / hidden1.bin (f32 rows x D). Then the diagnostics: a forward over ids0 with timestamps and
// debugLayers (layers.bin: the residual stream entering layers 1.., f32 [n-1][L0][D]) and a profile(); prints
// {gpu_ms, n_layers, profile} as JSON.
const fs = require('fs');
const path = require('path');
const ha = require(path.join(__dirname, '..', '..', 'strands-decider-web_amd', 'js', 'engine.js'));

const dir = process.argv[2];
const spec = JSON.parse(fs.readFileSync(path.join(dir, 'spec.json'), 'utf8'));
const raw = (f) => { const b = fs.readFileSync(path.join(dir, f)); return new Uint8Array(b.buffer, b.byteOffset, b.byteLength); };
const f32 = (f) => { const b = fs.readFileSync(path.join(dir, f)); return new Float32Array(b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength)); };
const u32 = (f) => { const b = fs.readFileSync(path.join(dir, f)); return Array.from(new Uint32Array(b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength))); };

const torso = new ha.Torso({ layer_types: spec.types, hidden_size: spec.D, intermediate_size: spec.I }, { maxCtx: 4096 });
const keep = [];
Object.keys(spec.weights).forEach((name) => {
  const q = torso.lead.alloc(raw('w_' + name + '.q').byteLength).upload(raw('w_' + name + '.q'));
  const s = torso.lead.alloc(raw('w_' + name + '.s').byteLength).upload(raw('w_' + name + '.s'));
  keep.push(q, s);
  torso.setWeight(name, { q: q, s: s, N: spec.weights[name].N, K: spec.weights[name].K });
});
spec.vectors.forEach((name) => torso.setParam(name, f32('v_' + name + '.bin')));
spec.mixer.forEach(([i, name]) => torso.setParam('layers.' + i + '.' + name, f32('m_' + i + '_' + name + '.bin')));

const r0 = torso.forward(u32('ids0.bin'), spec.rows0, { keepCache: true });
fs.writeFileSync(path.join(dir, 'hidden0.bin'), Buffer.from(r0.hidden.buffer));
if (!r0.cache || r0.cache.P !== spec.L0) throw new Error('cache P ' + (r0.cache && r0.cache.P));
const r1 = torso.forward(u32('ids1.bin'), spec.rows1, { cache: r0.cache });
fs.writeFileSync(path.join(dir, 'hidden1.bin'), Buffer.from(r1.hidden.buffer));
r0.cache.release();
const rd = torso.forward(u32('ids0.bin'), spec.rows0, { timestamps: true, debugLayers: true });
const stack = new Float32Array(rd.layers.length * spec.L0 * spec.D);
rd.layers.forEach((x, i) => stack.set(x, i * spec.L0 * spec.D));
fs.writeFileSync(path.join(dir, 'layers.bin'), Buffer.from(stack.buffer));
for (let j = 0; j < rd.hidden.length; j++) {
  if (rd.hidden[j] !== r0.hidden[j] && !(Number.isNaN(rd.hidden[j]) && Number.isNaN(r0.hidden[j]))) {
    throw new Error('diagnostics changed the hidden rows');
  }
}
const prof = torso.profile(u32('ids0.bin'));
torso.dropWeights();  // the weight handles borrow these buffers
keep.forEach((b) => b.free());  // the weight buffers live on the torso's lead engine: free them before destroy()
torso.destroy();
console.log(JSON.stringify({ ok: true, gpu_ms: rd.gpu_ms, fetch_ms: rd.fetch_ms, n_layers: rd.layers.length,
  profile: prof }));
