'use strict';
// GPU facade over the gfx950 backend (libquipu through the quipu_napi addon).
//
// Same surface as quipullm's WebGPU facade (web/js/gpu.js:1167-1282): GPU.crear, pipeline/prepararPipelines,
// buffer/subir/uniforme/grupo/liberar, despachar and dim2, with the reference's kernel names and binding
// lists (binding 0 = the uniform struct P, binding 1 = the Paso step record, then the storage buffers).
// Buffers are device addresses (BigInt).  A "pass" is the backend's single in-order stream, so despachar's
// first argument is accepted and ignored.  Node 12 syntax (CommonJS, no ?? or ?.).
const path = require('path');

// QP_ADDON selects another build of the addon (the profiling build in lib/timeline/)
const ADDON = process.env.QP_ADDON ? path.resolve(process.env.QP_ADDON) : path.join(__dirname, '..', 'lib', 'quipu_napi.node');
let native = null;
function addon() {
  if (!native) {
    try {
      native = require(ADDON);
    } catch (e) {
      throw new Error('quipu: native addon not built (' + ADDON + '): ' + e.message);
    }
  }
  return native;
}

const TB = 32;   // tokens per prefill pass of the dense model class (reference transformer.js:10)

// Packs [[type, value], ...] ('u' = u32, 'f' = f32) into 16-byte-padded bytes (reference gpu.js:1248-1256).
function empaquetar(valores) {
  const n = Math.max(4, Math.ceil(valores.length / 4) * 4);
  const ab = new ArrayBuffer(n * 4);
  const u = new Uint32Array(ab), f = new Float32Array(ab);
  valores.forEach(function (tv, i) {
    if (tv[0] === 'f') f[i] = tv[1]; else u[i] = tv[1] >>> 0;
  });
  return new Uint8Array(ab);
}

class Buffer {
  constructor(h, tam, label) { this.h = h; this._tam = tam; this.label = label; }
  get size() { return this._tam; }   // bytes, as WebGPU's GPUBuffer.size
}

class GPU {
  static crear(log, device) {
    addon().init(device || 0);
    return Promise.resolve(new GPU(log));
  }

  constructor(log) {
    this.n = addon();
    this.log = log || function () {};
    const i = JSON.parse(this.n.info());
    this.info = {
      summary: 'AMD ' + i.arch + ' (' + i.cus + ' CUs, ' + (i.hbm_bytes / 1e9).toFixed(0) + ' GB)',
      maxBuffer: i.max_buffer, maxBufferSize: i.max_buffer, vendor: 'amd', arquitectura: i.arch, cus: i.cus,
    };
    this.pipelines = {};
    this.perdido = false;
  }

  get bytesUsados() { return this.n.bytesUsed(); }

  _vigilar(fn) {
    try { return fn(); } catch (e) {
      if (this.n.lost()) { this.perdido = true; this.log('GPU lost: ' + e.message); }
      throw e;
    }
  }

  // Named op -> id (reference compiles a WGSL pipeline here, gpu.js:1197-1212).
  pipeline(nombre) {
    if (this.pipelines[nombre] !== undefined) return Promise.resolve(this.pipelines[nombre]);
    const id = this.n.opId(nombre);
    if (id < 0) return Promise.reject(new Error('quipu: unknown op ' + nombre));
    this.pipelines[nombre] = id;
    return Promise.resolve(id);
  }

  prepararPipelines(extra) {
    const self = this;
    return Promise.all((extra || []).map(function (n) { return self.pipeline(n); }));
  }

  buffer(bytes, uso, label) {
    const tam = Math.max(16, Math.ceil(bytes / 4) * 4);
    if (tam > this.info.maxBuffer) throw new Error("buffer '" + label + "' of " + (tam / 1e6).toFixed(0) + ' MB exceeds the GPU');
    const self = this;
    const h = this._vigilar(function () { return self.n.alloc(tam); });
    return new Buffer(h, tam, label || '');
  }

  subir(typed, label) {
    const b = this.buffer(typed.byteLength, undefined, label);
    this.escribir(b, 0, typed);
    return b;
  }

  // queue.writeBuffer(buffer, offset, data)
  escribir(b, offset, typed) {
    const self = this;
    const bytes = typed instanceof Uint8Array ? typed : new Uint8Array(typed.buffer, typed.byteOffset, typed.byteLength);
    this._vigilar(function () { self.n.upload(b.h, offset, bytes); });
  }

  leer(b, offset, into) {
    const self = this;
    this._vigilar(function () { self.n.download(b.h, offset, into); });
    return into;
  }

  copiar(dst, dOff, src, sOff, n) {
    const self = this;
    this._vigilar(function () { self.n.copy(dst.h, dOff, src.h, sOff, n); });
  }

  uniforme(valores) { return { uniforme: true, bytes: empaquetar(valores) }; }

  // Bind group: recursos[0] is the uniform, the rest device buffers (or sub-buffer views {h, off}, or null).
  grupo(nombre, recursos) {
    if (this.pipelines[nombre] === undefined) {
      const id = this.n.opId(nombre);
      if (id < 0) throw new Error('quipu: unknown op ' + nombre);
      this.pipelines[nombre] = id;
    }
    const u = recursos[0] && recursos[0].uniforme ? recursos[0].bytes : new Uint8Array(16);
    const resto = recursos[0] && recursos[0].uniforme ? recursos.slice(1) : recursos;
    const bufs = new BigUint64Array(resto.length);
    resto.forEach(function (r, i) { bufs[i] = r ? (typeof r === 'bigint' ? r : r.h) : 0n; });
    return { op: this.pipelines[nombre], nombre: nombre, u: u, bufs: bufs, gpu: this };
  }

  liberar(buffers) {
    for (const b of buffers) {
      if (b && b.h) { this.n.free(b.h); b.h = 0n; }
    }
  }

  sincronizar() { const self = this; this._vigilar(function () { self.n.sync(); }); }

  // HIP graph capture of the dispatches issued by fn(); returns a replayable graph handle.
  capturar(fn) {
    this.n.graphBegin();
    try { fn(); } catch (e) { try { this.n.graphEnd(); } catch (e2) { /* capture already broken */ } throw e; }
    return this.n.graphEnd();
  }

  reproducir(g, veces) { const self = this; this._vigilar(function () { self.n.graphLaunch(g, veces || 1); }); }
  liberarGrafo(g) { this.n.graphFree(g); }
  evento() { return this.n.eventCreate(); }
  marcar(e) { this.n.eventRecord(e); }
  msEntre(e0, e1) { return this.n.eventElapsed(e0, e1); }
}

// despachar(pass, grupo, x, y, z) -- reference gpu.js:1270-1274.
function despachar(pass, g, x, y, z) {
  const gpu = g.gpu;
  gpu._vigilar(function () { gpu.n.dispatch(g.op, g.u, g.bufs, x || 1, y || 1, z || 1); });
}

// 2-D split under the 65535-per-dimension limit (reference gpu.js:1278-1282).
function dim2(n) {
  if (n <= 65535) return [n, 1];
  const y = Math.ceil(n / 65535);
  return [Math.ceil(n / y), y];
}

// View of a sub-range of a device buffer (a binding that starts `off` bytes in).
function vista(b, off) { return { h: b.h + BigInt(off) }; }

module.exports = { GPU: GPU, despachar: despachar, dim2: dim2, vista: vista, empaquetar: empaquetar, TB: TB, addon: addon };
