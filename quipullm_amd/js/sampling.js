'use strict';
// Token choice for the token loop.
//
// Greedy selection follows quipullm's sampler (web/js/sampling.js:25-42): optional repetition / frequency /
// presence penalties over the last 64 history tokens, then, at temperature 0, the first index with the largest
// logit (a strict '>' scan from -Infinity, so ties go to the lowest index and NaN is never chosen).
// Stochastic sampling (top-k/top-p/min-p/temperature) is not part of this backend yet: a positive temperature
// raises an error instead of silently sampling differently.

class Muestreador {
  constructor(p) {
    p = p || {};
    this.temp = p.temperature !== undefined && p.temperature !== null ? p.temperature : 0.8;
    this.rep = p.repeat_penalty !== undefined && p.repeat_penalty !== null ? p.repeat_penalty : 1.0;
    this.freq = p.frequency_penalty || 0;
    this.pres = p.presence_penalty || 0;
    this.ventana = 64;
    if (this.temp > 0) throw new Error('stochastic sampling (temperature > 0) is not supported by this backend yet');
  }

  // True when elegir() reduces to a plain argmax, so the device-side greedy loop can be used.
  esVoraz() { return !(this.temp > 0) && this.rep === 1 && !this.freq && !this.pres; }

  penalizar(logits, historial) {
    if (!historial.length || (this.rep === 1 && !this.freq && !this.pres)) return;
    const V = logits.length, cuenta = new Map();
    for (const t of historial.slice(-this.ventana)) cuenta.set(t, (cuenta.get(t) || 0) + 1);
    for (const par of cuenta) {
      const t = par[0], n = par[1];
      if (t >= V) continue;
      let l = logits[t];
      if (this.rep !== 1) l = l > 0 ? l / this.rep : l * this.rep;
      logits[t] = l - (n * this.freq + this.pres);
    }
  }

  elegir(logits, historial) {
    this.penalizar(logits, historial || []);
    return argmax(logits);
  }
}

function argmax(v) {
  let mejor = 0, mv = -Infinity;
  for (let i = 0; i < v.length; i++) if (v[i] > mv) { mv = v[i]; mejor = i; }
  return mejor;
}

module.exports = { Muestreador: Muestreador, argmax: argmax };
