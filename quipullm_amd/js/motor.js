'use strict';
// The engine side of quipullm's server protocol, so this Node.js process can take the place of the browser tab
// behind the unchanged server (reference web/js/engine.js:56-80, 226-322, 386-465; the server side is its Puente
// and the /engine/api routes, server.py:1545-1657, 2056-2110):
//
//   POST /engine/api/hello  {motor, gpu, version, recarga}           -> {ok, version}
//   GET  /engine/api/next?motor=ID   (long poll, answered within 20 s) -> job | {accion: "nada"} | {accion: "cerrar"}
//   POST /engine/api/event  {motor, tipo, ...}                       -> {cancelar?}
//   GET  <job.modelo.meta_url>   the model's meta object; GET <job.modelo.archivo_url> with Range: tensor bytes
//
// Jobs: {id, accion, params, prompt, modelo: {id, arch, meta_url, archivo_url, ctx, bytes}}.  accion "generar":
// events inicio {prompt_tokens}, progreso {fase} per prompt chunk when the prompt is longer than one chunk, token
// {texto, n} per generated token (the reply may ask to cancel), fin {razon, prompt_tokens, completion_tokens, tps,
// ttft, tps_prompt, diag}; "cargar" / "descargar": load or free the model, then fin; failures: error {mensaje,
// codigo}.  State: estado {modelo_cargado, estado, info}.  Prompts are tokenized by a pluggable tokenizer
// (tokenizador.js); params.prompt_ids, when present, are used as the prompt's ids.
const { pedirJSON, dormir } = require('./http');
const engine = require('./engine');
const { TokenizadorIds } = require('./tokenizador');

const VERSION_MOTOR = 'quipullm-amd-engine-1';

class Motor {
  // op: servidor (base URL), id, opciones (this engine's model options: kv_f16, batch, ...), cargar(meta, fuente,
  // opciones) -> model (default: engine.cargarDesdeMeta), crearTokenizador(meta), info (the GPU summary the server
  // shows), log(text), espera (ms to wait after a failed request).
  constructor(op) {
    this.servidor = op.servidor.replace(/\/$/, '');
    this.id = op.id || ('m' + Date.now().toString(36) + Math.floor(Math.random() * 1e6).toString(36));
    this.opciones = op.opciones || {};
    this.cargar = op.cargar || function (meta, fuente, o) { return engine.cargarDesdeMeta(meta, fuente, o); };
    this.crearTokenizador = op.crearTokenizador || function (meta) { return new TokenizadorIds(meta); };
    this.info = op.info || null;
    this.log = op.log || function (m) { process.stderr.write('motor: ' + m + '\n'); };
    this.espera = op.espera || 2000;
    this.modelo = null;
    this.modeloId = null;
    this.tok = null;
    this.ocupado = false;
  }

  post(ruta, datos) { return pedirJSON(this.servidor + ruta, 'POST', datos, 60000); }

  // Events reach the server in the order they are made: each is posted after the previous one completed (progress
  // events are not awaited by the generation loop, so without the chain two of them could overtake each other).
  evento(d) {
    const self = this, cuerpo = Object.assign({ motor: this.id }, d);
    const p = (this.cadena || Promise.resolve()).then(function () { return self.post('/engine/api/event', cuerpo); });
    this.cadena = p.catch(function () {});
    return p;
  }

  informarEstado(estado) {
    return this.evento({ tipo: 'estado', modelo_cargado: this.modeloId, estado: estado, info: this.info });
  }

  async gpuInfo() {
    if (this.info) return this.info;
    const g = await engine.gpu();
    this.info = g.info;
    return this.info;
  }

  async descargarModelo() {
    if (this.modelo) this.modelo.free();
    this.modelo = null;
    this.modeloId = null;
    this.tok = null;
  }

  // The job's model in memory (loaded from the server's meta object and file route when it is another one).
  async asegurarModelo(m, jobId) {
    if (!m || !m.id) {
      const e = new Error('the job names no model');
      e.codigo = 400;
      throw e;
    }
    if (this.modelo && this.modeloId === m.id) return;
    await this.descargarModelo();
    await this.informarEstado('cargando ' + m.id);
    const t0 = Date.now();
    const meta = await pedirJSON(this.servidor + m.meta_url, 'GET', undefined, 300000);
    if (m.ctx && !meta.ctx) meta.ctx = m.ctx;
    const self = this;
    let ultimo = 0;
    const progreso = function (f) {
      if (f - ultimo >= 0.1 || f >= 1) {
        ultimo = f;
        self.evento({ tipo: 'progreso', id: jobId, fase: 'cargando modelo ' + Math.round(100 * f) + '%' }).catch(function () {});
      }
    };
    this.modelo = await this.cargar(meta, { url: this.servidor + m.archivo_url }, { options: this.opciones, progreso: progreso });
    this.modeloId = m.id;
    this.tok = this.crearTokenizador(meta);
    this.log('model ' + m.id + ' loaded in ' + (Date.now() - t0) + ' ms');
    await this.informarEstado('listo');
  }

  // accion "generar" (reference engine.js:226-322)
  async generar(job) {
    const p = job.params || {};
    const tJob = Date.now();
    await this.asegurarModelo(job.modelo, job.id);
    const tok = this.tok, modelo = this.modelo, self = this;
    const t0 = Date.now();
    const diag = { modelo_ms: t0 - tJob, tok_ms: 0, lotes_ms: [] };
    if (p.imagenes && p.imagenes.length) {
      const e = new Error('images are not supported by this engine');
      e.codigo = 400;
      throw e;
    }
    const ids = Array.isArray(p.prompt_ids) ? p.prompt_ids.map(function (x) { return x | 0; })
      : tok.codificar(job.prompt || '', { addBos: p.add_bos === false ? false : null });
    if (!ids.length) throw new Error('the prompt is empty');
    diag.tok_ms = Date.now() - t0;
    await this.evento({ tipo: 'inicio', id: job.id, prompt_tokens: ids.length });
    const ctx = modelo.ctx;
    if (ids.length >= ctx) {
      const e = new Error('the prompt has ' + ids.length + ' tokens and the model context is ' + ctx);
      e.codigo = 400;
      throw e;
    }
    const maxTok = p.max_tokens > 0 ? Math.min(p.max_tokens, ctx - ids.length) : ctx - ids.length;
    const dec = tok.decodificadorIncremental();
    let tLote = null;
    const params = Object.assign({}, p, {
      max_tokens: maxTok,
      esFin: function (id) { return tok.esFin(id); },
      alLote: function (fin, total) {
        const ahora = Date.now();
        if (tLote !== null) diag.lotes_ms.push(ahora - tLote);
        tLote = ahora;
        if (total > modelo.batch)
          self.evento({ tipo: 'progreso', id: job.id, fase: 'procesando prompt ' + fin + '/' + total }).catch(function () {});
      },
      // the last token of a generation cut by length is counted but its text is not sent (engine.js:297)
      alToken: async function (id, k) {
        if (k >= maxTok) return false;
        const r = await self.evento({ tipo: 'token', id: job.id, texto: dec.agregar(id), n: 1 });
        return !!(r && r.cancelar);
      },
      bloque: p.bloque || 8,
    });
    const tGen = Date.now();
    const r = await engine.generar(modelo, ids, params);
    const tPrompt = tGen + r.prompt_ms;
    if (tLote !== null) diag.lotes_ms.push(tPrompt - tLote);
    diag.reutilizados = r.reutilizados;
    const cola = dec.terminar();
    if (cola) await this.evento({ tipo: 'token', id: job.id, texto: cola, n: 0 });
    const n = r.ids.length, seg = r.decode_ms / 1000, ttft = (tPrompt - t0) / 1000;
    const tps = n > 0 && seg > 0 ? +(n / seg).toFixed(2) : null;
    const tpsPrompt = +((ids.length - r.reutilizados) / Math.max(ttft, 1e-3)).toFixed(1);
    this.log('done: ' + ids.length + ' prompt tokens (' + tpsPrompt + ' tok/s), ' + n + ' generated (' + tps + ' tok/s)');
    await this.evento({ tipo: 'fin', id: job.id, razon: r.razon, prompt_tokens: ids.length, completion_tokens: n, tps: tps,
      ttft: +ttft.toFixed(3), tps_prompt: tpsPrompt, diag: diag });
  }

  // reference engine.js:386-405
  async atender(job) {
    this.ocupado = true;
    try {
      if (job.accion === 'generar') await this.generar(job);
      else if (job.accion === 'cargar') {
        await this.asegurarModelo(job.modelo, job.id);
        await this.evento({ tipo: 'fin', id: job.id, razon: 'stop' });
      } else if (job.accion === 'descargar') {
        await this.descargarModelo();
        await this.informarEstado('listo');
        await this.evento({ tipo: 'fin', id: job.id, razon: 'stop' });
      } else {
        const e = new Error("action '" + job.accion + "' is not supported by this engine");
        e.codigo = 400;
        throw e;
      }
    } catch (e) {
      this.log('error: ' + e.message);
      if (this.modelo && this.modelo.invalidar) this.modelo.invalidar();
      await this.evento({ tipo: 'error', id: job.id, mensaje: e.message, codigo: e.codigo || 500 }).catch(function () {});
      if (this.modelo && this.modelo.gpu && this.modelo.gpu.perdido) {
        this.modelo = null;
        this.modeloId = null;
      }
    } finally {
      this.ocupado = false;
    }
  }

  // The engine loop (reference engine.js:416-465).  Returns when the server answers "cerrar" (another engine took
  // over) or when op.parar() says so between jobs.
  async correr(op) {
    op = op || {};
    let saludado = false, avisado = false;
    for (;;) {
      if (op.parar && op.parar()) return 'parado';
      try {
        if (!saludado) {
          const info = await this.gpuInfo();
          await this.post('/engine/api/hello', { motor: this.id, gpu: info, version: VERSION_MOTOR, recarga: true,
            userAgent: 'node ' + process.version });
          await this.informarEstado('listo');
          saludado = true;
        }
        // the server answers within 20 s: cut at 35 s and ask again (a hung connection)
        let job;
        try {
          job = await pedirJSON(this.servidor + '/engine/api/next?motor=' + encodeURIComponent(this.id), 'GET', undefined, 35000);
        } catch (e) {
          if (e && e.name === 'AbortError') { this.log('the request to the server hung; retrying'); continue; }
          throw e;
        }
        avisado = false;
        if (!job || !job.accion || job.accion === 'nada') continue;
        if (job.accion === 'cerrar') {
          this.log('another engine took over; this one stops');
          await this.descargarModelo();
          return 'cerrado';
        }
        await this.atender(job);
      } catch (e) {
        if (!avisado) { this.log('no connection to the server, or error: ' + e.message); avisado = true; }
        await dormir(this.espera);
      }
    }
  }
}

module.exports = { Motor: Motor, VERSION_MOTOR: VERSION_MOTOR };
