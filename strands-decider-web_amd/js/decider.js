'use strict';
/*
 * decider.js: the worker-level host on top of the MI355X torso. It turns a {state, question} request into one or two
 * torso forwards and an answer, as the engine branch of the reference's worker does (web/public/js/worker.js:17-26,
 * 186-236, with the prompt format of prompt.js and the pointer head of head.js):
 *
 *   const d = new Decider(torso, head, tokenizer, cfg);  // cfg: temperature, temperature_by_kind, ordinal_smoothing,
 *   d.decide(state, question)                            //      max_length (the reference's decider config)
 *   d.decideMany(state, {name: question, ...})
 *
 * What must equal the reference, because the same model reads it and the same decisions must come out: the prompt
 * text (tags, headers, option lines), how the token budget is split, where an option's token sits, the head's
 * arithmetic and the answer formulas. They are implemented here as rules over small tables:
 *   - state block: "<state>\n" + content + "\n</state>\n"; content = a string trimmed, else 2-space-indented JSON;
 *   - question block: '<question type="K">\n' + HEADER[K] + "\n" + content(instructions) + "\n<options>\n" + option
 *     lines joined by "\n" + "\n</options>\n</question>\n<answer>";
 *   - option line n (from 1): "n. label", then " — description" when the description, its white-space runs
 *     collapsed to single spaces, is not empty; labels and descriptions per kind in OPTION_RULES;
 *   - budget: the question keeps its last min(len, max(1, floor(0.75 max_length))) tokens, the state its first
 *     max(1, max_length - that) tokens; the prompt is state then question;
 *   - an option's position is the last kept question token whose bytes lie inside the option line (the tokenizer is
 *     a byte-level BPE: a token string holds one character per input byte);
 *   - the pointer head reads the last prompt row (q) and the option rows (k): LayerNorm (eps 1e-5) with the head's
 *     weight and bias, an affine projection each, logit = q . k / sqrt(dim q) / temperature, softmax;
 *   - answers from the option probabilities per ANSWER_RULES;
 *   - the prefix cache holds the last 4 states' snapshots, least recently used released first.
 * The tokenizer is the caller's: encode(text) -> {ids, tokens}.
 */

const TAGS = {
  stateOpen: '<state>\n',
  stateClose: '\n</state>\n',
  optionsOpen: '\n<options>\n',
  close: '\n</options>\n</question>\n<answer>',
};
const HEADER = {
  noul: 'Decide whether the statement is true of the state.',
  choice: 'Select exactly one option.',
  score: 'Rate the state against the ordered levels below (lowest first).',
};
const NOUL_TEXT = { false: 'the statement does not hold for this state', true: 'the statement holds for this state' };

// [label, description] pairs of a question, by kind
const OPTION_RULES = {
  noul(q) {
    const given = q.criteria || {};
    return ['false', 'true'].map((label) =>
      [label, given[label] === undefined || given[label] === null ? NOUL_TEXT[label] : given[label]]);
  },
  choice(q) {
    if (Array.isArray(q.options)) return q.options.map((label) => [label, '']);
    return Object.entries(q.options);
  },
  score(q) {
    return q.options.map((description, level) => [String(level), description]);
  },
};

function contentText(c) {
  return typeof c === 'string' ? c.trim() : JSON.stringify(c, null, 2);
}

function collapseSpaces(s) {
  return String(s || '').split(/\s+/).filter((word) => word !== '').join(' ');
}

function renderState(state) {
  return TAGS.stateOpen + contentText(state) + TAGS.stateClose;
}

// The question block and, for each option, the [start, end) character range of its line.
function renderQuestion(q) {
  const rule = OPTION_RULES[q.type];
  if (!rule) throw new Error('unknown question type ' + q.type);
  const pairs = rule(q);
  const parts = ['<question type="' + q.type + '">\n', HEADER[q.type], '\n', contentText(q.instructions),
    TAGS.optionsOpen];
  let at = parts.reduce((n, p) => n + p.length, 0);
  const spans = [];
  pairs.forEach((pair, i) => {
    const description = collapseSpaces(pair[1]);
    const line = String(i + 1) + '. ' + pair[0] + (description === '' ? '' : ' — ' + description);
    if (i > 0) {
      parts.push('\n');
      at += 1;
    }
    parts.push(line);
    spans.push([at, at + line.length]);
    at += line.length;
  });
  parts.push(TAGS.close);
  return { text: parts.join(''), kind: q.type, labels: pairs.map((p) => p[0]), descriptions: pairs.map((p) => p[1]),
    spans: spans };
}

// Byte ranges of the tokens of a byte-level BPE, in order.
function tokenByteRanges(tokens) {
  const ranges = new Array(tokens.length);
  let end = 0;
  for (let i = 0; i < tokens.length; i++) {
    ranges[i] = [end, end + tokens[i].length];
    end += tokens[i].length;
  }
  return ranges;
}

// How many question tokens and state tokens a prompt of at most maxLength tokens keeps.
function splitBudget(questionTokens, maxLength) {
  const question = Math.min(questionTokens, Math.max(1, Math.floor(0.75 * maxLength)));
  return { question: question, state: Math.max(1, maxLength - question) };
}

function buildInputs(tokenizer, state, question, maxLength) {
  const rq = renderQuestion(question);
  const qEnc = tokenizer.encode(rq.text);
  const sEnc = tokenizer.encode(renderState(state));
  const budget = splitBudget(qEnc.ids.length, maxLength || 4096);
  const first = qEnc.ids.length - budget.question;
  const qIds = Array.from(qEnc.ids).slice(first);
  const ranges = tokenByteRanges(qEnc.tokens).slice(first);
  const sIds = Array.from(sEnc.ids).slice(0, budget.state);
  const optIdx = rq.spans.map((span) => {
    const lo = Buffer.byteLength(rq.text.slice(0, span[0]), 'utf8');
    const hi = Buffer.byteLength(rq.text.slice(0, span[1]), 'utf8');
    let pos = -1;
    ranges.forEach((r, j) => {
      if (r[1] > r[0] && r[0] >= lo && r[1] <= hi) pos = j;
    });
    if (pos < 0) throw new Error('option truncated out of the prompt');
    return sIds.length + pos;
  });
  return { ids: sIds.concat(qIds), optIdx: optIdx, rq: rq, stateLen: sIds.length };
}

// Confidence of an ordinal answer: 1 when the levels' spread is at most sqrt(eps), 0 at the widest spread (n-1)/2.
function ordinalConfidence(p, eps) {
  const n = p.length;
  if (n <= 1) return 1;
  const total = p.reduce((s, x) => s + x, 0);
  if (total <= 0) return 0;
  const w = p.map((x) => x / total);
  const mean = w.reduce((s, x, i) => s + i * x, 0);
  const spread = Math.sqrt(w.reduce((s, x, i) => s + x * (i - mean) * (i - mean), 0));
  const widest = (n - 1) / 2, floor = eps > 0 ? Math.sqrt(eps) : 0;
  if (widest <= floor) return spread <= floor ? 1 : 0;
  return Math.min(1, Math.max(0, (widest - spread) / (widest - floor)));
}

// Answer of each kind from the option probabilities (in label order) and the probabilities by label.
const ANSWER_RULES = {
  noul(rq, p, byLabel) {
    return { type: 'noul', noul: byLabel.true, probabilities: byLabel };
  },
  choice(rq, p, byLabel) {
    let best = 0;
    for (let i = 1; i < p.length; i++) if (p[i] > p[best]) best = i;
    const n = p.length;
    const confidence = n <= 1 ? 1 : Math.min(1, Math.max(0, (n * p[best] - 1) / (n - 1)));
    return { type: 'choice', choice: rq.labels[best], probabilities: byLabel, confidence: confidence };
  },
  score(rq, p, byLabel, eps) {
    const levels = rq.labels.map((_, i) => byLabel[String(i)]);
    const score = levels.reduce((s, x, i) => s + i * x, 0);
    return { type: 'score', score: score, probabilities: byLabel, confidence: ordinalConfidence(levels, eps) };
  },
};

function readAnswer(rq, probs, ordinalSmoothing) {
  const byLabel = {};
  rq.labels.forEach((label, i) => { byLabel[label] = probs[i]; });
  return ANSWER_RULES[rq.kind](rq, probs, byLabel, ordinalSmoothing === undefined ? 0.1 : ordinalSmoothing);
}

/*
 * The pointer head: the f32 tensors norm.{weight,bias}, q.{weight,bias}, k.{weight,bias} of a safetensors file. A row
 * is layer-normed (population variance, eps 1e-5; sums in double precision, normed values stored as f32) and
 * projected (double-precision sums, f32 results).
 */
class PointerHead {
  constructor(buf) {
    const bytes = buf instanceof Uint8Array ? buf : new Uint8Array(buf);
    const headerLen = Number(new DataView(bytes.buffer, bytes.byteOffset, 8).getBigUint64(0, true));
    const header = JSON.parse(Buffer.from(bytes.buffer, bytes.byteOffset + 8, headerLen).toString('utf8'));
    this.tensors = {};
    for (const name of Object.keys(header)) {
      if (name === '__metadata__') continue;
      const t = header[name];
      if (t.dtype !== 'F32') throw new Error('head tensor ' + name + ' is ' + t.dtype);
      const copy = bytes.slice(8 + headerLen + t.data_offsets[0], 8 + headerLen + t.data_offsets[1]);
      this.tensors[name] = { data: new Float32Array(copy.buffer, copy.byteOffset, copy.byteLength / 4), shape: t.shape };
    }
  }
  normed(x) {
    const d = x.length;
    let sum = 0;
    for (let j = 0; j < d; j++) sum += x[j];
    const mean = sum / d;
    let sq = 0;
    for (let j = 0; j < d; j++) sq += (x[j] - mean) * (x[j] - mean);
    const scale = 1 / Math.sqrt(sq / d + 1e-5);
    const w = this.tensors['norm.weight'].data, b = this.tensors['norm.bias'].data;
    const y = new Float32Array(d);
    for (let j = 0; j < d; j++) y[j] = (x[j] - mean) * scale * w[j] + b[j];
    return y;
  }
  project(which, x) {
    const W = this.tensors[which + '.weight'], bias = this.tensors[which + '.bias'].data;
    const y = this.normed(x), d = y.length, rows = W.shape[0], out = new Float32Array(rows);
    for (let o = 0; o < rows; o++) {
      let acc = bias[o];
      const w = W.data.subarray(o * d, (o + 1) * d);
      for (let j = 0; j < d; j++) acc += w[j] * y[j];
      out[o] = acc;
    }
    return out;
  }
  // hidden: Float32Array rows of d; the logits and probabilities of the option rows for the answer row
  score(hidden, d, answerRow, optionRows, temperature) {
    const row = (i) => hidden.subarray(i * d, (i + 1) * d);
    const q = this.project('q', row(answerRow));
    const norm = 1 / Math.sqrt(q.length);
    const logits = optionRows.map((i) => {
      const k = this.project('k', row(i));
      let dot = 0;
      for (let j = 0; j < k.length; j++) dot += k[j] * q[j];
      return dot * norm / temperature;
    });
    let top = -Infinity;
    logits.forEach((l) => { top = Math.max(top, l); });
    const e = logits.map((l) => Math.exp(l - top));
    const z = e.reduce((s, x) => s + x, 0);
    return { logits: logits, probs: e.map((x) => x / z) };
  }
}

function loadHead(buf) {
  return new PointerHead(buf);
}

function pointerLogits(head, hidden, d, answerRow, optionRows, temperature) {
  return head.score(hidden, d, answerRow, optionRows, temperature);
}

// State snapshots by the state's token ids, at most `capacity`, the least recently used released on overflow.
class PrefixCache {
  constructor(capacity) {
    this.capacity = capacity || 4;
    this.entries = new Map();  // insertion order = use order
  }
  get(ids) {
    const key = ids.join(',');
    const snap = this.entries.get(key) || null;
    if (snap) {
      this.entries.delete(key);
      this.entries.set(key, snap);
    }
    return { key: key, hit: snap };
  }
  put(key, snap) {
    this.entries.set(key, snap);
    for (const k of this.entries.keys()) {
      if (this.entries.size <= this.capacity) break;
      this.entries.get(k).release();
      this.entries.delete(k);
    }
  }
  clear() {
    for (const snap of this.entries.values()) snap.release();
    this.entries.clear();
  }
}

/*
 * decide: when the state's snapshot is cached, only the question tokens run, resumed from it; otherwise the whole
 * prompt (the state is not cached by decide). decideMany: the state runs once (or comes from the cache), is cached,
 * and each question's tokens run resumed from it. The requested rows are the option tokens and the last token.
 */
class Decider {
  constructor(torso, head, tokenizer, cfg) {
    this.torso = torso;
    this.head = head instanceof PointerHead ? head : new PointerHead(head);
    this.tokenizer = tokenizer;
    this.cfg = Object.assign({ temperature: 1, temperature_by_kind: {}, ordinal_smoothing: 0.1, max_length: 4096 },
      cfg || {});
    this.cache = new PrefixCache(4);
  }
  _temperature(kind) {
    const t = this.cfg.temperature_by_kind[kind];
    return t === undefined ? this.cfg.temperature : t;
  }
  // forward of `ids` (resumed from `snap` when given) returning the option rows then the answer row
  _run(ids, optionRows, snap) {
    const rows = optionRows.concat([ids.length - 1]);
    return snap ? this.torso.forward(ids, rows, { cache: snap }) : this.torso.forward(ids, rows);
  }
  _answer(rq, r, nOptions) {
    const s = this.head.score(r.hidden, r.d, nOptions, Array.from({ length: nOptions }, (_, i) => i),
      this._temperature(rq.kind));
    return { answer: readAnswer(rq, s.probs, this.cfg.ordinal_smoothing), logits: s.logits };
  }
  decide(state, question) {
    const b = buildInputs(this.tokenizer, state, question, this.cfg.max_length);
    const snap = this.cache.get(b.ids.slice(0, b.stateLen)).hit;
    const offset = snap ? b.stateLen : 0;
    const r = this._run(b.ids.slice(offset), b.optIdx.map((i) => i - offset), snap);
    const out = this._answer(b.rq, r, b.optIdx.length);
    out.tokens = b.ids.length;
    out.cached_state_tokens = offset;
    return out;
  }
  decideMany(state, questions) {
    const names = Object.keys(questions);
    const built = names.map((n) => buildInputs(this.tokenizer, state, questions[n], this.cfg.max_length));
    const sLen = built[0].stateLen;
    const look = this.cache.get(built[0].ids.slice(0, sLen));
    let snap = look.hit;
    if (!snap) {
      snap = this.torso.forward(built[0].ids.slice(0, sLen), [], { keepCache: true }).cache;
      this.cache.put(look.key, snap);
    }
    const answers = {};
    let tokens = sLen;
    built.forEach((b, i) => {
      const r = this._run(b.ids.slice(sLen), b.optIdx.map((j) => j - sLen), snap);
      answers[names[i]] = this._answer(b.rq, r, b.optIdx.length).answer;
      tokens += b.ids.length - sLen;
    });
    return { answers: answers, tokens: tokens };
  }
  close() {
    this.cache.clear();
  }
}

module.exports = {
  Decider: Decider, PrefixCache: PrefixCache, PointerHead: PointerHead, renderState: renderState,
  renderQuestion: renderQuestion, buildInputs: buildInputs, readAnswer: readAnswer, loadHead: loadHead,
  pointerLogits: pointerLogits,
};
