'use strict';
// Loads an export directory (convert/export_engine.py format) with js/loader.js and runs two forwards without a
// cache, the way Engine.create + Engine.forward are used (engine.js:63-84, 313). Arguments: the export directory and
// a work directory holding ids0.bin / ids1.bin (u32) and rows.json; writes hidden0.bin / hidden1.bin (f32).
const fs = require('fs');
const path = require('path');
const loader = require(path.join(__dirname, '..', '..', 'strands-decider-web_amd', 'js', 'loader.js'));
const ha = require(path.join(__dirname, '..', '..', 'strands-decider-web_amd', 'js', 'engine.js'));

// With a third argument "create", the export is loaded through the async Engine.create(base, {onProgress,
// fetchShard}) of loader.js, whose fetchShard hands each shard over a tick later, as a download would.
const [exp, work, how] = process.argv.slice(2);
const u32 = (f) => { const b = fs.readFileSync(path.join(work, f)); return Array.from(new Uint32Array(b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength))); };
const rows = JSON.parse(fs.readFileSync(path.join(work, 'rows.json'), 'utf8'));
const progress = [];
const fetches = [];

async function main() {
  const onProgress = (p) => progress.push(p);
  let torso;
  if (how === 'create') {
    const fetchShard = (url, p, wire) => new Promise((resolve) => setImmediate(() => {
      fetches.push([url, p, !!wire]);
      resolve(fs.readFileSync(path.join(exp, p)));
    }));
    torso = await loader.Engine.create(exp, { maxCtx: 4096, onProgress: onProgress, fetchShard: fetchShard, subgroups: true });
  } else {
    torso = loader.loadTorso(exp, { maxCtx: 4096, onProgress: onProgress });
  }
  const manifest = JSON.parse(fs.readFileSync(path.join(exp, 'manifest.json'), 'utf8'));
  if (JSON.stringify(progress) !== JSON.stringify(manifest.shards.map((s) => s.path))) {
    throw new Error('onProgress saw ' + JSON.stringify(progress));
  }
  if (how === 'create' && fetches.length !== manifest.shards.length + (manifest.embed ? 1 : 0)) {
    throw new Error('fetchShard saw ' + JSON.stringify(fetches));
  }
  const r0 = torso.forward(u32('ids0.bin'), rows[0]);
  fs.writeFileSync(path.join(work, 'hidden0.bin'), Buffer.from(r0.hidden.buffer));
  const r1 = torso.forward(u32('ids1.bin'), rows[1]);
  fs.writeFileSync(path.join(work, 'hidden1.bin'), Buffer.from(r1.hidden.buffer));
  const lazy = torso.loaded.lazy;
  torso.destroy();
  console.log(JSON.stringify({ ok: true, shards: torso.loaded.shards.length, fetched: lazy ? lazy.fetched : 0,
    evictions: lazy ? lazy.evictions : 0, kernels: [r0.kernel, r1.kernel], problems: ha.engineProblems(0) }));
}

main().catch((e) => {
  console.error(e.stack || String(e));
  process.exit(1);
});
