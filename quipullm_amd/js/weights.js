'use strict';
// Loading of GGUF tensors into device buffers, from a local file or from the server's file URL by ranges.
//
// Same interface as quipullm's CargadorPesos (web/js/weights.js:15-139): existe(name), info(name),
// f32(name) -> buffer, matriz(name) -> {tipo, N, K, w} ({tipo:'q8' | 'iq4nl', N, K, qs, ds} for Q8_0, IQ4_NL: qs and
// ds are the quant and scale planes of one buffer).  The device layout behind a handle is this backend's own:
// K-quant blocks, Q8_0 and IQ4_NL repacked on the device into planar arrays (quants | scales) so every lane load is
// a 16-byte vector load.
// Source: a path (read synchronously), or {url} (the reference engine's /engine/file/<id>, web/js/weights.js:51):
// then the caller awaits precargar(names) before the synchronous calls that use those tensors.
const fs = require('fs');
const { despachar, vista } = require('./gpu');
const { rango } = require('./http');

// GGUF K-quant types: name, GGUF block bytes, device bytes per block (Q3_K padded to 112)
const K_QUANTS = { 10: { nombre: 'q2k', bytes: 84, disp: 84 }, 11: { nombre: 'q3k', bytes: 110, disp: 112 },
  12: { nombre: 'q4k', bytes: 144, disp: 144 }, 13: { nombre: 'q5k', bytes: 176, disp: 176 },
  14: { nombre: 'q6k', bytes: 210, disp: 210 } };

const F16 = (function () {
  const t = new Float32Array(65536);
  for (let h = 0; h < 65536; h++) {
    const s = h & 0x8000 ? -1 : 1, e = (h >> 10) & 0x1f, f = h & 0x3ff;
    if (e === 0) t[h] = s * Math.pow(2, -14) * (f / 1024);
    else if (e === 31) t[h] = f ? NaN : s * Infinity;
    else t[h] = s * Math.pow(2, e - 15) * (1 + f / 1024);
  }
  return t;
})();

class CargadorPesos {
  constructor(gpu, meta, fuente, progreso) {
    this.gpu = gpu;
    this.meta = meta;
    this.url = typeof fuente === 'string' ? null : fuente.url;
    this.progreso = progreso || function () {};
    this.tensores = new Map(meta.tensors.map(function (t) { return [t.nombre, t]; }));
    this.totalBytes = meta.tensors.reduce(function (a, t) { return a + (t.bytes || 0); }, 0);
    this.leidos = 0;
    this.buffers = [];
    this.previos = new Map();   // tensors fetched by precargar (URL source), taken by bytes()
    this.fd = this.url ? null : fs.openSync(fuente, 'r');
  }

  cerrar() { if (this.fd !== null) { fs.closeSync(this.fd); this.fd = null; } this.previos.clear(); }

  // URL source: fetches the named tensors that exist (one range request each, in turn); a path source needs nothing.
  async precargar(nombres) {
    if (!this.url) return;
    for (const n of nombres) {
      const t = this.tensores.get(n);
      if (!t || this.previos.has(n) || t.bytes === null || t.bytes === undefined) continue;
      this.previos.set(n, await rango(this.url, t.abs, t.bytes));
    }
  }

  existe(nombre) { return this.tensores.has(nombre); }

  info(nombre) {
    const t = this.tensores.get(nombre);
    if (!t) throw new Error('missing tensor ' + nombre);
    return t;
  }

  bytes(t) {
    if (t.bytes === null || t.bytes === undefined) throw new Error('unsupported tensor type (' + t.tipo_nombre + ') in ' + t.nombre);
    let b;
    if (this.url) {
      b = this.previos.get(t.nombre);
      if (!b) throw new Error('tensor ' + t.nombre + ' was not fetched from ' + this.url);
      this.previos.delete(t.nombre);
    } else {
      b = Buffer.allocUnsafe(t.bytes);
      let got = 0;
      while (got < t.bytes) {
        const n = fs.readSync(this.fd, b, got, Math.min(t.bytes - got, 1 << 30), t.abs + got);
        if (n <= 0) throw new Error('incomplete read of ' + t.nombre);
        got += n;
      }
    }
    this.leidos += t.bytes;
    this.progreso(this.leidos / this.totalBytes, t.nombre);
    return new Uint8Array(b.buffer, b.byteOffset, b.length);
  }

  // Vector or matrix as f32 on the device (reference weights.js:72-92).
  f32(nombre) {
    const t = this.info(nombre);
    const u8 = this.bytes(t);
    let f;
    if (t.tipo === 0) f = new Float32Array(u8.buffer.slice(u8.byteOffset, u8.byteOffset + u8.length));
    else if (t.tipo === 1) {
      const s = new Uint16Array(u8.buffer.slice(u8.byteOffset, u8.byteOffset + u8.length));
      f = new Float32Array(s.length);
      for (let i = 0; i < s.length; i++) f[i] = F16[s[i]];
    } else if (t.tipo === 30) {
      const s = new Uint16Array(u8.buffer.slice(u8.byteOffset, u8.byteOffset + u8.length));
      f = new Float32Array(s.length);
      const v = new Uint32Array(f.buffer);
      for (let i = 0; i < s.length; i++) v[i] = s[i] << 16;
    } else if (t.tipo === 8) {
      const nb = u8.length / 34;
      f = new Float32Array(nb * 32);
      const dv = new DataView(u8.buffer, u8.byteOffset, u8.length);
      for (let b = 0; b < nb; b++) {
        const d = F16[dv.getUint16(b * 34, true)];
        for (let i = 0; i < 32; i++) f[b * 32 + i] = dv.getInt8(b * 34 + 2 + i) * d;
      }
    } else throw new Error(nombre + ': type ' + t.tipo_nombre + ' not supported as f32');
    const b = this.gpu.subir(f, nombre);
    this.buffers.push(b);
    return b;
  }

  // Raw blocks -> device layout, repacked on the device (K-quant row chunk planes, Q8_0 planar).
  _subirRepack(u8, op, nblocks, K, etiqueta, bytesDisp) {
    const gpu = this.gpu;
    const staging = gpu.subir(u8, etiqueta + '.raw');
    const dst = gpu.buffer(bytesDisp || u8.length, undefined, etiqueta);
    const lo = nblocks % 4294967296, hi = Math.floor(nblocks / 4294967296);
    despachar(null, gpu.grupo(op, [gpu.uniforme([['u', lo], ['u', hi], ['u', K]]), null, staging, dst]), 1);
    gpu.liberar([staging]);
    return dst;
  }

  // Weight matrix [N][K] (reference weights.js:96-139).  Stacked expert tensors give N = E * rows.
  matriz(nombre) {
    const t = this.info(nombre);
    const K = t.dims[0], N = t.dims.slice(1).reduce(function (a, b) { return a * b; }, 1);
    if (K_QUANTS[t.tipo]) {
      const info = K_QUANTS[t.tipo];
      if (K % 256) throw new Error(nombre + ': K=' + K + ' is not a multiple of 256 (' + info.nombre + ')');
      const u8 = this.bytes(t);
      const w = this._subirRepack(u8, 'repack_' + info.nombre, N * K / 256, K, nombre, N * K / 256 * info.disp);
      this.buffers.push(w);
      return { tipo: info.nombre, N: N, K: K, w: w };
    }
    if (t.tipo === 8) {
      if (K % 32) throw new Error(nombre + ': K=' + K + ' is not a multiple of 32');
      const u8 = this.bytes(t);
      const w = this._subirRepack(u8, 'repack_q8', N * K / 32, K, nombre);
      this.buffers.push(w);
      return { tipo: 'q8', N: N, K: K, w: w, qs: w, ds: vista(w, N * K) };
    }
    if (t.tipo === 20) {
      // IQ4_NL (reference weights.js:110-116): the nibble bytes as they are (16 per block) then the f16 scales,
      // 18 bytes per 32 weights as in the file; the reference's qs / dh pair is the two planes of one buffer
      if (K % 32) throw new Error(nombre + ': K=' + K + ' is not a multiple of 32');
      const u8 = this.bytes(t);
      const w = this._subirRepack(u8, 'repack_iq4nl', N * K / 32, K, nombre);
      this.buffers.push(w);
      return { tipo: 'iq4nl', N: N, K: K, w: w, qs: w, ds: vista(w, N * K / 2) };
    }
    if (t.tipo === 0 || t.tipo === 1 || t.tipo === 30) {
      const w = this.f32(nombre);
      return { tipo: 'f32', N: N, K: K, w: w };
    }
    throw new Error(nombre + ': quantization ' + t.tipo_nombre + ' not supported yet (supported: Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, IQ4_NL, F16, BF16, F32)');
  }
}

module.exports = { CargadorPesos: CargadorPesos, F16: F16 };
