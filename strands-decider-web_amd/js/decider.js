'use strict';
/*
 * decider.js: the worker-level host on top of the MI355X torso (web/public/js/worker.js, prompt.js, head.js of the
 * reference): prompts rendered from a state and a question, their token ids and option positions, the pointer head
 * over the torso's final-normed hidden rows, the answer derived from its probabilities, and the prefix cache of
 * state snapshots (LRU, 4 entries) that lets several questions about one state reuse its forward.
 *
 *   const d = new Decider(torso, head, tokenizer, cfg);   // cfg: the decider config (temperature, temperature_by_kind,
 *   d.decide(state, question)                             //   ordinal_smoothing, max_length)
 *   d.decideMany(state, {name: question, ...})
 *
 * The tokenizer is the caller's: encode(text) -> {ids, tokens}, a byte-level BPE whose token strings hold one
 * character per byte of the input (as the reference's tokenizer).
 */

const KIND_HEADER = {
  noul: 'Decide whether the statement is true of the state.',
  choice: 'Select exactly one option.',
  score: 'Rate the state against the ordered levels below (lowest first).',
};
const NOUL_DEFAULT = { false: 'the statement does not hold for this state', true: 'the statement holds for this state' };

// Text of a state or an instruction: a string trimmed, anything else as indented JSON (prompt.js:12-14).
function renderContent(c) {
  if (typeof c === 'string') return c.trim();
  return JSON.stringify(c, null, 2);
}

function renderState(state) {
  return '<state>\n' + renderContent(state) + '\n</state>\n';
}

/*
 * The question block (prompt.js:21-38): header by kind, the instructions, numbered options "i. name — description"
 * (descriptions with runs of white space collapsed), then "<answer>". Returns the text, the option labels and each
 * option line's [start, end) character span in the text.
 */
function renderQuestion(q) {
  let pairs;
  if (q.type === 'noul') {
    const crit = q.criteria || {};
    pairs = ['false', 'true'].map((l) => [l, crit[l] !== undefined && crit[l] !== null ? crit[l] : NOUL_DEFAULT[l]]);
  } else if (q.type === 'choice') {
    pairs = Array.isArray(q.options) ? q.options.map((o) => [o, '']) : Object.keys(q.options).map((k) => [k, q.options[k]]);
  } else if (q.type === 'score') {
    pairs = q.options.map((desc, i) => [String(i), desc]);
  } else {
    throw new Error('unknown question type ' + q.type);
  }
  const head = '<question type="' + q.type + '">\n' + KIND_HEADER[q.type] + '\n' + renderContent(q.instructions) +
    '\n<options>\n';
  let text = head;
  const spans = [];
  pairs.forEach(([name, desc], i) => {
    const d = String(desc || '').split(/\s+/).filter((w) => w.length > 0).join(' ');
    const line = (i + 1) + '. ' + name + (d ? ' — ' + d : '');
    spans.push([text.length, text.length + line.length]);
    text += line + '\n';
  });
  text += '</options>\n</question>\n<answer>';
  return { text: text, kind: q.type, labels: pairs.map((p) => p[0]), descriptions: pairs.map((p) => p[1]), spans: spans };
}

const utf8len = (s) => Buffer.byteLength(s, 'utf8');

/*
 * Token ids of state + question, tokenised separately, and the position of each option's last token (prompt.js:
 * 48-65): the question keeps up to 3/4 of max_length (its head is cut first), the state fills the rest; an option's
 * position is the last token lying wholly inside its line.
 */
function buildInputs(tokenizer, state, question, maxLength) {
  const maxL = maxLength || 4096;
  const rq = renderQuestion(question);
  const qe = tokenizer.encode(rq.text), se = tokenizer.encode(renderState(state));
  let qIds = Array.from(qe.ids);
  let offs = [];
  let p = 0;
  qe.tokens.forEach((t) => { offs.push([p, p + t.length]); p += t.length; });  // one character per input byte
  const keep = Math.min(qIds.length, Math.max(1, Math.floor(maxL * 0.75)));
  const cut = Math.max(0, qIds.length - keep);
  qIds = qIds.slice(cut);
  offs = offs.slice(cut);
  const sIds = Array.from(se.ids).slice(0, Math.max(1, maxL - keep));
  const optIdx = rq.spans.map(([a, b]) => {
    const A = utf8len(rq.text.slice(0, a)), B = utf8len(rq.text.slice(0, b));
    let last = -1;
    offs.forEach(([lo, hi], j) => { if (hi > lo && lo >= A && hi <= B) last = j; });
    if (last < 0) throw new Error('option truncated out of the prompt');
    return sIds.length + last;
  });
  return { ids: sIds.concat(qIds), optIdx: optIdx, rq: rq, stateLen: sIds.length };
}

// Confidence of an ordinal answer (prompt.js:80-89): 1 at the smallest spread sqrt(eps), 0 at the largest (n-1)/2.
function scoreConfidence(probs, eps) {
  const n = probs.length;
  if (n <= 1) return 1;
  const tot = probs.reduce((a, b) => a + b, 0);
  if (tot <= 0) return 0;
  const p = probs.map((x) => x / tot);
  const mean = p.reduce((s, x, i) => s + i * x, 0);
  const sd = Math.sqrt(p.reduce((s, x, i) => s + x * (i - mean) * (i - mean), 0));
  const hi = (n - 1) / 2, lo = eps > 0 ? Math.sqrt(eps) : 0;
  if (hi <= lo) return sd <= lo ? 1 : 0;
  return Math.min(1, Math.max(0, (hi - sd) / (hi - lo)));
}

// The answer from the option probabilities (prompt.js:68-78).
function readAnswer(rq, probs, ordinalSmoothing) {
  const eps = ordinalSmoothing === undefined ? 0.1 : ordinalSmoothing;
  const by = {};
  rq.labels.forEach((l, i) => { by[l] = probs[i]; });
  if (rq.kind === 'noul') return { type: 'noul', noul: by.true, probabilities: by };
  if (rq.kind === 'choice') {
    const n = probs.length, top = Math.max.apply(null, probs);
    return { type: 'choice', choice: rq.labels[probs.indexOf(top)], probabilities: by,
      confidence: n <= 1 ? 1 : Math.min(1, Math.max(0, (n * top - 1) / (n - 1))) };
  }
  const ordered = rq.labels.map((_, i) => by[String(i)]);
  const mean = ordered.reduce((s, x, i) => s + i * x, 0);
  return { type: 'score', score: mean, probabilities: by, confidence: scoreConfidence(ordered, eps) };
}

/*
 * The pointer head (head.js): f32 tensors of a safetensors file. logits_i = (q . k_i) / sqrt(|q|) / temperature,
 * q = proj_q(LN(h_answer)), k_i = proj_k(LN(h_option_i)), LN with its own weight and bias (eps 1e-5); softmax.
 */
function loadHead(buf) {
  const u8 = buf instanceof Uint8Array ? buf : new Uint8Array(buf);
  const n = Number(new DataView(u8.buffer, u8.byteOffset, 8).getBigUint64(0, true));
  const meta = JSON.parse(Buffer.from(u8.buffer, u8.byteOffset + 8, n).toString('utf8'));
  const H = {};
  Object.keys(meta).forEach((k) => {
    if (k === '__metadata__') return;
    const v = meta[k];
    if (v.dtype !== 'F32') throw new Error('head tensor ' + k + ' is ' + v.dtype);
    const [a, b] = v.data_offsets;
    const bytes = u8.slice(8 + n + a, 8 + n + b);
    H[k] = { data: new Float32Array(bytes.buffer, bytes.byteOffset, (b - a) / 4), shape: v.shape };
  });
  return H;
}

function headProject(H, name, x) {
  const d = x.length;
  let mean = 0;
  for (let j = 0; j < d; j++) mean += x[j];
  mean /= d;
  let v = 0;
  for (let j = 0; j < d; j++) v += (x[j] - mean) * (x[j] - mean);
  const inv = 1 / Math.sqrt(v / d + 1e-5);
  const g = H['norm.weight'].data, be = H['norm.bias'].data;
  const xn = new Float32Array(d);
  for (let j = 0; j < d; j++) xn[j] = (x[j] - mean) * inv * g[j] + be[j];
  const W = H[name + '.weight'], bias = H[name + '.bias'].data, out = new Float32Array(W.shape[0]);
  for (let o = 0; o < W.shape[0]; o++) {
    let s = bias[o];
    const base = o * d;
    for (let j = 0; j < d; j++) s += W.data[base + j] * xn[j];
    out[o] = s;
  }
  return out;
}

// hidden: Float32Array rows of d; logits and probabilities of the options at rows optRows for the answer row.
function pointerLogits(H, hidden, d, answerRow, optRows, temperature) {
  const rowOf = (i) => hidden.subarray(i * d, (i + 1) * d);
  const q = headProject(H, 'q', rowOf(answerRow));
  const scale = 1 / Math.sqrt(q.length);
  const logits = optRows.map((i) => {
    const k = headProject(H, 'k', rowOf(i));
    let s = 0;
    for (let j = 0; j < k.length; j++) s += k[j] * q[j];
    return s * scale / temperature;
  });
  const top = Math.max.apply(null, logits);
  const e = logits.map((l) => Math.exp(l - top));
  const z = e.reduce((a, b) => a + b, 0);
  return { logits: logits, probs: e.map((x) => x / z) };
}

/*
 * Prefix snapshots keyed by the state's token ids, least recently used first out after `capacity` entries (the
 * worker's stateCache, worker.js:17-26); an evicted snapshot is released.
 */
class PrefixCache {
  constructor(capacity) {
    this.capacity = capacity || 4;
    this.map = new Map();
  }
  get(ids) {
    const key = ids.join(',');
    const hit = this.map.get(key);
    if (hit) { this.map.delete(key); this.map.set(key, hit); }
    return { key: key, hit: hit || null };
  }
  put(key, snap) {
    this.map.set(key, snap);
    while (this.map.size > this.capacity) {
      const first = this.map.keys().next().value;
      this.map.get(first).release();
      this.map.delete(first);
    }
  }
  clear() {
    this.map.forEach((s) => s.release());
    this.map.clear();
  }
}

/*
 * The engine branch of the worker's requests (worker.js:186-236): decide runs only the question suffix from a cached
 * state snapshot when the state was seen before, else the whole prompt; decideMany encodes the state once (caching
 * it) and runs each question's suffix from it.
 */
class Decider {
  constructor(torso, head, tokenizer, cfg) {
    this.torso = torso;
    this.head = head;
    this.tokenizer = tokenizer;
    this.cfg = Object.assign({ temperature: 1, temperature_by_kind: {}, ordinal_smoothing: 0.1, max_length: 4096 }, cfg || {});
    this.cache = new PrefixCache(4);
  }
  _answer(rq, hidden, d, answerRow, optRows) {
    const t = this.cfg.temperature_by_kind[rq.kind] !== undefined ? this.cfg.temperature_by_kind[rq.kind] : this.cfg.temperature;
    const r = pointerLogits(this.head, hidden, d, answerRow, optRows, t);
    return { answer: readAnswer(rq, r.probs, this.cfg.ordinal_smoothing), logits: r.logits };
  }
  decide(state, question) {
    const b = buildInputs(this.tokenizer, state, question, this.cfg.max_length);
    const sLen = b.stateLen;
    const { hit } = this.cache.get(b.ids.slice(0, sLen));
    const rows = hit ? b.optIdx.map((i) => i - sLen).concat([b.ids.length - sLen - 1]) : b.optIdx.concat([b.ids.length - 1]);
    const r = hit ? this.torso.forward(b.ids.slice(sLen), rows, { cache: hit }) : this.torso.forward(b.ids, rows);
    const n = b.optIdx.length;
    const out = this._answer(b.rq, r.hidden, r.d, n, b.optIdx.map((_, i) => i));
    return Object.assign(out, { tokens: b.ids.length, cached_state_tokens: hit ? sLen : 0 });
  }
  decideMany(state, questions) {
    const built = Object.keys(questions).map((name) => [name, buildInputs(this.tokenizer, state, questions[name], this.cfg.max_length)]);
    const sLen = built[0][1].stateLen, sIds = built[0][1].ids.slice(0, sLen);
    let { key, hit } = this.cache.get(sIds);
    if (!hit) {
      hit = this.torso.forward(sIds, [], { keepCache: true }).cache;
      this.cache.put(key, hit);
    }
    const answers = {};
    built.forEach(([name, b]) => {
      const suffix = b.ids.slice(sLen);
      const rows = b.optIdx.map((i) => i - sLen).concat([suffix.length - 1]);
      const r = this.torso.forward(suffix, rows, { cache: hit });
      answers[name] = this._answer(b.rq, r.hidden, r.d, b.optIdx.length, b.optIdx.map((_, i) => i)).answer;
    });
    return { answers: answers, tokens: sLen + built.reduce((s, [, b]) => s + b.ids.length - sLen, 0) };
  }
  close() {
    this.cache.clear();
  }
}

module.exports = {
  Decider: Decider, PrefixCache: PrefixCache, renderState: renderState, renderQuestion: renderQuestion,
  buildInputs: buildInputs, readAnswer: readAnswer, loadHead: loadHead, pointerLogits: pointerLogits,
};
