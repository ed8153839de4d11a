'use strict';
// Token loop of the engine on the gfx950 backend.
//
// Architecture registry: manifests in ./arch/*.json map general.architecture to a base model class, as
// quipullm's web/arch manifests do (engine.js:14-34, server.py:64-101).  generar() is the reference's
// generation loop (engine.js:226-322); the HTTP job protocol around it is motor.js.  The prompt is processed in
// chunks of modelo.batch tokens (only the last chunk asks for logits), then tokens are chosen until max_tokens.  With
// greedy parameters the decode runs on the device (one captured graph per token, argmax on the device);
// otherwise each step reads the logits back and the host sampler chooses.
const fs = require('fs');
const path = require('path');
const { GPU } = require('./gpu');
const { metaDe } = require('./gguf');
const { ModeloTransformer } = require('./transformer');
const { Muestreador, argmax } = require('./sampling');

const BASES = { transformer: ModeloTransformer };
const DIR_ARCH = path.join(__dirname, 'arch');

function cargarRegistro() {
  const reg = {};
  for (const f of fs.readdirSync(DIR_ARCH).sort()) {
    if (!f.endsWith('.json')) continue;
    const man = JSON.parse(fs.readFileSync(path.join(DIR_ARCH, f), 'utf8'));
    if (!man.id || !Array.isArray(man.arch) || !man.arch.length) throw new Error('invalid manifest ' + f);
    if (!!man.base === !!man.module) throw new Error(f + ": define exactly one of 'base' or 'module'");
    const Clase = man.base ? BASES[man.base] : require(path.join(DIR_ARCH, man.module));
    if (typeof Clase !== 'function') throw new Error(f + ': unknown base ' + man.base);
    for (const a of man.arch) reg[a] = { Clase: Clase, manifiesto: man };
  }
  return reg;
}

let gpuGlobal = null;
async function gpu() {
  if (!gpuGlobal) gpuGlobal = await GPU.crear(null);
  return gpuGlobal;
}

// Loads a GGUF model: reads the header, picks the class from the registry, uploads the weights.
async function cargarModelo(ruta, opciones) {
  opciones = opciones || {};
  const reg = cargarRegistro();
  const cab = metaDe(ruta, {});
  const a = cab.kv['general.architecture'];
  if (!reg[a]) throw new Error("architecture '" + a + "' is not supported by this engine (see quipullm_amd/js/arch)");
  const meta = metaDe(ruta, { manifiesto: reg[a].manifiesto, ctx: opciones.ctx, options: opciones.options });
  const modelo = new reg[a].Clase(await gpu(), meta);
  await modelo.load(ruta, opciones.progreso);
  return modelo;
}

// Loads a model from the server's meta object (server.py meta_json: kv, tensors, data_start, ctx, overrides,
// arch_options, options) with its weights from `fuente` (a path, or {url} of /engine/file/<id>).  opciones.options
// are this engine's own settings (kv_f16, batch, ...), merged over the server's options.
async function cargarDesdeMeta(meta, fuente, opciones) {
  opciones = opciones || {};
  const reg = cargarRegistro();
  const a = meta.kv['general.architecture'];
  if (!reg[a]) {
    const e = new Error("architecture '" + a + "' is not supported by this engine (see quipullm_amd/js/arch)");
    e.codigo = 400;
    throw e;
  }
  const m = Object.assign({}, meta, { options: Object.assign({}, reg[a].manifiesto.options || {}, meta.options || {},
    opciones.options || {}) });
  const modelo = new reg[a].Clase(await gpu(), m);
  await modelo.load(fuente, opciones.progreso);
  return modelo;
}

// Prompt processing in chunks of modelo.batch from id `desde` (reference engine.js:253-288); returns the last
// logits.  desde = 0 resets the model.  alLote(fin, total), if given, is called before each chunk.
async function prefill(modelo, ids, desde, alLote) {
  desde = desde || 0;
  if (!desde) modelo.reset();
  const TL = modelo.batch;
  let logits = null;
  for (let i = desde; i < ids.length; i += TL) {
    const fin = Math.min(i + TL, ids.length);
    if (alLote) alLote(fin, ids.length);
    logits = await modelo.forward(ids.slice(i, fin), fin >= ids.length);
  }
  return logits;
}

// Generation (reference engine.js:226-322).  Returns {ids, razon, prompt_ms, decode_ms, tps, reutilizados}; tps is
// computed as the reference does (generated / (t_end - t_after_prompt), engine.js:315-316); razon is 'stop' (end
// token, or alToken asked to stop) or 'length' (max_tokens or the context).
// params: the sampler's (sampling.js), max_tokens, esFin(id), onToken(id) (synchronous), alToken(id, k) (async,
// awaited per token k = 1, 2, ...; a true result stops the generation: the reference's `cancelar`), alLote(fin,
// total) (per prompt chunk), host_loop, bloque (greedy: tokens per device run between host readbacks).
async function generar(modelo, ids, params) {
  params = params || {};
  if (!ids.length) throw new Error('the prompt is empty');
  const ctx = modelo.ctx;
  if (ids.length >= ctx) {
    const e = new Error('the prompt has ' + ids.length + ' tokens and the model context is ' + ctx);
    e.codigo = 400;
    throw e;
  }
  const maxTok = params.max_tokens > 0 ? Math.min(params.max_tokens, ctx - ids.length) : ctx - ids.length;
  const esFin = params.esFin || function () { return false; };
  const porToken = params.onToken || function () {};
  const mu = new Muestreador(params);
  const t0 = Date.now();
  // prompt cache (reference engine.js:254-256): the ids already in the model's state are not computed again
  const saltar = modelo.cacheOn && modelo.reutilizar && params.prompt_cache !== false ? modelo.reutilizar(ids) : 0;
  let logits = await prefill(modelo, ids, saltar, params.alLote);
  const tPrompt = Date.now();
  const hist = ids.slice();
  const out = [];
  let razon = 'length';
  // records token t; true when the generation must stop after it
  const emitir = async function (t) {
    out.push(t);
    porToken(t);
    if (params.alToken && await params.alToken(t, out.length)) { razon = 'stop'; return true; }
    return false;
  };
  if (mu.esVoraz() && modelo.decodificarVoraz && !params.host_loop) {
    const primero = argmax(logits);
    if (esFin(primero)) razon = 'stop';
    else if (!(await emitir(primero))) {
      const resto = maxTok - 1;
      const bloque = params.bloque || resto;
      let hechos = 0;
      while (hechos < resto) {
        const n = Math.min(bloque, resto - hechos);
        const nuevos = modelo.decodificarVoraz(out[out.length - 1], n);
        let parar = false;
        for (const t of nuevos) {
          if (esFin(t)) { razon = 'stop'; parar = true; break; }
          if (await emitir(t)) { parar = true; break; }
        }
        hechos += n;
        if (parar) break;
      }
    }
  } else if (modelo.pasoMuestreado && !params.host_loop) {
    // each step on the fused one-token plan; penalties and top-k candidates on the device where the sampler
    // allows, the draw on the host (the first token from the prefill's logits)
    let id = mu.elegir(logits, hist);
    while (out.length < maxTok) {
      if (esFin(id)) { razon = 'stop'; break; }
      hist.push(id);
      if (await emitir(id)) break;
      if (out.length >= maxTok) break;
      id = modelo.pasoMuestreado(id, mu, hist);
    }
  } else {
    while (out.length < maxTok) {
      const id = mu.elegir(logits, hist);
      if (esFin(id)) { razon = 'stop'; break; }
      hist.push(id);
      if (await emitir(id)) break;
      if (out.length >= maxTok) break;
      logits = await modelo.forward([id], true);
    }
  }
  const tEnd = Date.now();
  const seg = (tEnd - tPrompt) / 1000;
  return { ids: out, razon: razon, prompt_ms: tPrompt - t0, decode_ms: tEnd - tPrompt,
    tps: out.length && seg > 0 ? out.length / seg : null, reutilizados: saltar };
}

module.exports = { cargarRegistro: cargarRegistro, cargarModelo: cargarModelo, cargarDesdeMeta: cargarDesdeMeta,
  prefill: prefill, generar: generar, gpu: gpu };
