'use strict';
// Token choice for the token loop, with quipullm's sampler semantics (web/js/sampling.js), in llama.cpp's order:
// penalties -> top_k -> top_p -> min_p -> temperature.
//
//  - penalties (sampling.js:27-37): repetition / frequency / presence over the last 64 history tokens, applied to
//    the logits in place (a Float32Array store rounds each result to float);
//  - temperature <= 0 (sampling.js:38-42): the first index with the largest logit (strict '>' from -Infinity:
//    ties go to the lowest index, NaN is never chosen);
//  - otherwise (sampling.js:43-81): the top_k candidates by a min-heap over the logits in index order (every
//    token when top_k <= 0 or >= V), a stable sort by descending logit, softmax without temperature for the top_p
//    and min_p cuts, then weights exp((l - max) / T) and one uniform draw from mulberry32(seed) (Math.random
//    without a seed).
//
// The float steps run in doubles exactly as the reference's JavaScript does; the heap keeps the reference's
// comparisons, which decide the order of equal logits.  muestrear() takes an already selected candidate list, so
// the device top-k (transformer.js, candidatosDispositivo) can replace the heap when it proves there are no ties.

function def(v, d) { return v === undefined || v === null ? d : v; }

// mulberry32 (reference sampling.js:3-10): 32-bit state, one output per call in [0, 1).
function mulberry32(semilla) {
  let a = semilla | 0;
  return function () {
    a = (a + 0x6D2B79F5) | 0;
    let t = Math.imul(a ^ (a >>> 15), a | 1);
    t = (t + Math.imul(t ^ (t >>> 7), t | 61)) ^ t;
    return ((t ^ (t >>> 14)) >>> 0) / 4294967296;
  };
}

class Muestreador {
  constructor(p) {
    p = p || {};
    this.temp = def(p.temperature, 0.8);
    this.topK = def(p.top_k, 40);
    this.topP = def(p.top_p, 0.95);
    this.minP = def(p.min_p, 0.05);
    this.rep = def(p.repeat_penalty, 1.0);
    this.freq = def(p.frequency_penalty, 0);
    this.pres = def(p.presence_penalty, 0);
    this.ventana = 64;
    this.rand = p.seed !== null && p.seed !== undefined ? mulberry32(p.seed) : Math.random;
  }

  // True when elegir() reduces to a plain argmax, so the device-side greedy loop can be used.
  esVoraz() { return !(this.temp > 0) && !this.penaliza(); }

  penaliza() { return this.rep !== 1 || !!this.freq || !!this.pres; }

  // [token, count] over the penalty window, in first-occurrence order (sampling.js:28-29).
  conteos(historial) {
    const cuenta = new Map();
    for (const t of historial.slice(-this.ventana)) cuenta.set(t, (cuenta.get(t) || 0) + 1);
    return Array.from(cuenta);
  }

  penalizar(logits, historial) {
    if (!historial || !historial.length || !this.penaliza()) return;
    const V = logits.length;
    for (const par of this.conteos(historial)) {
      const t = par[0], n = par[1];
      if (t >= V) continue;
      let l = logits[t];
      if (this.rep !== 1) l = l > 0 ? l / this.rep : l * this.rep;
      l -= n * this.freq + this.pres;
      logits[t] = l;
    }
  }

  elegir(logits, historial) {
    this.penalizar(logits, historial || []);
    return this.elegirPenalizado(logits);
  }

  // The choice from logits that already carry the penalties.
  elegirPenalizado(logits) {
    if (!(this.temp > 0)) return argmax(logits);
    const cand = candidatosHeap(logits, this.topK);
    const val = new Float64Array(cand.length);
    for (let i = 0; i < cand.length; i++) val[i] = logits[cand[i]];
    return this.muestrear(cand, val);
  }

  // The device path applies to: stochastic, 1 <= top_k <= 128 and below the vocabulary, and partial lists that
  // fit the device merge (ceil(V / 2048) chunks of top_k + 1 keys, at most 16384).
  usaCandidatosDispositivo(V) {
    return this.temp > 0 && this.topK >= 1 && this.topK <= 128 && this.topK < V &&
      Math.ceil(V / 2048) * (this.topK + 1) <= 16384;
  }

  // sampling.js:58-81 from candidate ids `cand` and their logits `val` (same order).
  muestrear(cand, val) {
    const n0 = cand.length;
    const orden = new Array(n0);
    for (let i = 0; i < n0; i++) orden[i] = i;
    orden.sort(function (a, b) { return val[b] - val[a]; });   // stable: equal logits keep the candidate order
    const ids = orden.map(function (i) { return cand[i]; });
    const v = orden.map(function (i) { return val[i]; });
    const max = v[0];
    const probs = new Array(n0);
    let s = 0;
    for (let i = 0; i < n0; i++) { probs[i] = Math.exp(v[i] - max); }
    for (let i = 0; i < n0; i++) s += probs[i];
    for (let i = 0; i < n0; i++) probs[i] = probs[i] / s;
    let n = n0;
    if (this.topP < 1) {
      let acum = 0;
      for (let i = 0; i < n; i++) { acum += probs[i]; if (acum >= this.topP) { n = i + 1; break; } }
    }
    if (this.minP > 0) {
      const lim = probs[0] * this.minP;
      let m = 1;
      while (m < n && probs[m] >= lim) m++;
      n = m;
    }
    const pt = new Array(n);
    let tot = 0;
    for (let i = 0; i < n; i++) pt[i] = Math.exp((v[i] - max) / this.temp);
    for (let i = 0; i < n; i++) tot += pt[i];
    let r = this.rand() * tot;
    for (let i = 0; i < n; i++) { r -= pt[i]; if (r <= 0) return ids[i]; }
    return ids[n - 1];
  }
}

// Top-k candidate ids in the reference's min-heap order (sampling.js:44-57); every id when k <= 0 or k >= V.
function candidatosHeap(logits, topK) {
  const V = logits.length;
  const k = topK > 0 ? Math.min(topK, V) : V;
  if (k >= V) {
    const todos = new Array(V);
    for (let i = 0; i < V; i++) todos[i] = i;
    return todos;
  }
  const h = [];
  const cambia = function (i, j) { const t = h[i]; h[i] = h[j]; h[j] = t; };
  for (let i = 0; i < V; i++) {
    if (h.length < k) {
      h.push(i);
      let c = h.length - 1;            // sift up: stop at a parent that is not larger
      while (c > 0) {
        const p = (c - 1) >> 1;
        if (logits[h[p]] <= logits[h[c]]) break;
        cambia(p, c);
        c = p;
      }
    } else if (logits[i] > logits[h[0]]) {
      h[0] = i;
      let c = 0;                       // sift down to the strictly smaller child
      for (;;) {
        const l = 2 * c + 1, r = l + 1;
        let m = c;
        if (l < h.length && logits[h[l]] < logits[h[m]]) m = l;
        if (r < h.length && logits[h[r]] < logits[h[m]]) m = r;
        if (m === c) break;
        cambia(m, c);
        c = m;
      }
    }
  }
  return h;
}

function argmax(v) {
  let mejor = 0, mv = -Infinity;
  for (let i = 0; i < v.length; i++) if (v[i] > mv) { mv = v[i]; mejor = i; }
  return mejor;
}

module.exports = { Muestreador: Muestreador, argmax: argmax, mulberry32: mulberry32, candidatosHeap: candidatosHeap };
