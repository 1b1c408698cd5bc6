'use strict';
// The worker's engine branch (web/public/js/worker.js:186-236) on the MI355X torso: an export loaded by loadTorso,
// a pointer head from a safetensors file, a byte-level tokenizer (one token per UTF-8 byte). Arguments: the export
// directory and a work directory with head.safetensors and cases.json {state, questions: {name: question}, states};
// prints {many, single, lru} as JSON; single[name] also holds the logits and the prompt's ids and option rows.
const fs = require('fs');
const path = require('path');
const js = path.join(__dirname, '..', '..', 'strands-decider-web_amd', 'js');
const { loadTorso } = require(path.join(js, 'loader.js'));
const D = require(path.join(js, 'decider.js'));

const [exp, work] = process.argv.slice(2);
const cases = JSON.parse(fs.readFileSync(path.join(work, 'cases.json'), 'utf8'));
const tok = { encode: (t) => { const b = Buffer.from(t, 'utf8'); return { ids: Array.from(b), tokens: Array.from(b, (x) => String.fromCharCode(x)) }; } };
const torso = loadTorso(exp, { maxCtx: 4096 });
const dec = new D.Decider(torso, D.loadHead(fs.readFileSync(path.join(work, 'head.safetensors'))), tok,
  { temperature: 1.0, temperature_by_kind: { score: 0.5 }, ordinal_smoothing: 0.1, max_length: 4096 });
// one question at a time on a state seen for the first time (whole prompt), then the same questions together
const single = {};
Object.keys(cases.questions).forEach((name) => {
  dec.cache.clear();
  const r = dec.decide(cases.state, cases.questions[name]);
  const b = D.buildInputs(tok, cases.state, cases.questions[name], 4096);
  single[name] = { answer: r.answer, cached: r.cached_state_tokens, logits: r.logits, ids: b.ids, optIdx: b.optIdx };
});
dec.cache.clear();
const many = dec.decideMany(cases.state, cases.questions);
// decide after decideMany: the state's snapshot is cached, only the suffix runs
const again = dec.decide(cases.state, cases.questions[Object.keys(cases.questions)[0]]);
// LRU: four more states evict the first
let released = 0;
const first = dec.cache.entries.values().next().value;
const rel = first.release;
first.release = function () { released++; rel.call(first); };
cases.states.forEach((s) => dec.decideMany(s, { q: cases.questions[Object.keys(cases.questions)[0]] }));
const out = { many: many.answers, single: single, again_cached: again.cached_state_tokens, released: released,
  cache_size: dec.cache.entries.size };
dec.close();
torso.destroy();
console.log(JSON.stringify(out));
