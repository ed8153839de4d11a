'use strict';
// GGUF header reader producing the model `meta` object of quipullm's engine protocol.
//
// Same result as the reference server's leer_gguf + meta_json (server.py:404-441, 797-815): key/values,
// tensor infos {nombre, dims (ggml order, dims[0] = K), tipo, offset, bytes, tipo_nombre, abs} with `bytes`
// from the block table (server.py:353-355) and abs = data_start + offset, data_start aligned to
// general.alignment.  Reads a local file instead of fetching over HTTP.
const fs = require('fs');

const GGML_TIPOS = { 0: 'F32', 1: 'F16', 2: 'Q4_0', 3: 'Q4_1', 6: 'Q5_0', 7: 'Q5_1', 8: 'Q8_0', 9: 'Q8_1',
  10: 'Q2_K', 11: 'Q3_K', 12: 'Q4_K', 13: 'Q5_K', 14: 'Q6_K', 15: 'Q8_K', 16: 'IQ2_XXS', 17: 'IQ2_XS',
  18: 'IQ3_XXS', 19: 'IQ1_S', 20: 'IQ4_NL', 21: 'IQ3_S', 22: 'IQ2_S', 23: 'IQ4_XS', 24: 'I8', 25: 'I16',
  26: 'I32', 27: 'I64', 28: 'F64', 29: 'IQ1_M', 30: 'BF16' };
// (elements per block, bytes per block)
const GGML_BLOQUES = { 0: [1, 4], 1: [1, 2], 2: [32, 18], 3: [32, 20], 6: [32, 22], 7: [32, 24], 8: [32, 34],
  9: [32, 36], 10: [256, 84], 11: [256, 110], 12: [256, 144], 13: [256, 176], 14: [256, 210], 15: [256, 292],
  20: [32, 18], 30: [1, 2] };

class Lector {
  constructor(fd) { this.fd = fd; this.pos = 0; this.buf = Buffer.alloc(1 << 20); this.b0 = 0; this.b1 = 0; }
  _need(n) {
    if (this.pos >= this.b0 && this.pos + n <= this.b1) return;
    const size = Math.max(n, this.buf.length);
    if (size > this.buf.length) this.buf = Buffer.alloc(size);
    const got = fs.readSync(this.fd, this.buf, 0, size, this.pos);
    if (got < n) throw new Error('GGUF: unexpected end of file');
    this.b0 = this.pos; this.b1 = this.pos + got;
  }
  take(n) { this._need(n); const o = this.pos - this.b0; this.pos += n; return this.buf.subarray(o, o + n); }
  u8() { return this.take(1).readUInt8(0); }
  i8() { return this.take(1).readInt8(0); }
  u16() { return this.take(2).readUInt16LE(0); }
  i16() { return this.take(2).readInt16LE(0); }
  u32() { return this.take(4).readUInt32LE(0); }
  i32() { return this.take(4).readInt32LE(0); }
  f32() { return this.take(4).readFloatLE(0); }
  f64() { return this.take(8).readDoubleLE(0); }
  u64() { const b = this.take(8); return b.readUInt32LE(0) + b.readUInt32LE(4) * 4294967296; }
  i64() { const b = this.take(8); return b.readUInt32LE(0) + b.readInt32LE(4) * 4294967296; }
  str() { const n = this.u64(); return n ? this.take(n).toString('utf8') : ''; }
  valor(t) {
    switch (t) {
      case 0: return this.u8(); case 1: return this.i8(); case 2: return this.u16(); case 3: return this.i16();
      case 4: return this.u32(); case 5: return this.i32(); case 6: return this.f32(); case 7: return this.u8() !== 0;
      case 8: return this.str(); case 10: return this.u64(); case 11: return this.i64(); case 12: return this.f64();
      case 9: {
        const sub = this.u32(), n = this.u64();
        const out = new Array(n);
        for (let i = 0; i < n; i++) out[i] = this.valor(sub);
        return out;
      }
      default: throw new Error('GGUF: unknown value type ' + t);
    }
  }
}

// leerGGUF(path) -> {kv, tensors, data_start}
function leerGGUF(ruta) {
  const fd = fs.openSync(ruta, 'r');
  try {
    const r = new Lector(fd);
    if (r.take(4).toString('latin1') !== 'GGUF') throw new Error('not a GGUF file');
    const version = r.u32();
    if (version < 2) throw new Error('GGUF version ' + version + ' not supported');
    const nt = r.u64(), nkv = r.u64();
    const kv = {};
    for (let i = 0; i < nkv; i++) { const k = r.str(); kv[k] = r.valor(r.u32()); }
    const tensors = [];
    for (let i = 0; i < nt; i++) {
      const nombre = r.str();
      const nd = r.u32();
      const dims = [];
      for (let d = 0; d < nd; d++) dims.push(r.u64());
      const tipo = r.u32();
      const offset = r.u64();
      tensors.push({ nombre: nombre, dims: dims, tipo: tipo, offset: offset });
    }
    const alin = kv['general.alignment'] || 32;
    const inicio = Math.ceil(r.pos / alin) * alin;
    for (const t of tensors) {
      const n = t.dims.reduce(function (a, b) { return a * b; }, 1);
      const eb = GGML_BLOQUES[t.tipo];
      t.bytes = eb ? Math.floor(n / eb[0]) * eb[1] : null;
      t.tipo_nombre = GGML_TIPOS[t.tipo] || String(t.tipo);
      t.abs = inicio + t.offset;
    }
    return { kv: kv, tensors: tensors, data_start: inicio };
  } finally {
    fs.closeSync(fd);
  }
}

// The engine's meta object (server.py:797-815) for a local file; `manifiesto` is the web/arch manifest.
function metaDe(ruta, opciones) {
  opciones = opciones || {};
  const g = leerGGUF(ruta);
  const man = opciones.manifiesto || {};
  return {
    id: opciones.id || ruta, kv: g.kv, tensors: g.tensors, data_start: g.data_start,
    ctx: opciones.ctx || 4096, overrides: opciones.overrides || {}, arch_options: man.options || {},
    options: Object.assign({ tiled_prefill: true, prompt_cache: true }, opciones.options || {}),   // server.py:808-809 defaults
  };
}

module.exports = { leerGGUF: leerGGUF, metaDe: metaDe, GGML_TIPOS: GGML_TIPOS, GGML_BLOQUES: GGML_BLOQUES };
