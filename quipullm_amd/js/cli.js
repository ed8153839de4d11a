'use strict';
// Command-line driver of the engine, for tests and the benchmark.
//
//   node cli.js generate --model M.gguf --prompt-file ids.json --n 128 [--mode fast|ref|engine|sample] [--kv f16|f32]
//                        [--ctx N] [--batch N] [--no-tiled] [--no-fused-ffn] [--no-ffn-planes] [--no-norm-planes] [--logits-out file.f32] [--kv-out file]
//                        [--force-ids ids.json]
//                        [--repeat-penalty R] [--frequency-penalty F] [--presence-penalty P] [--host-loop]
//                        [--temperature T] [--top-k K] [--top-p P] [--min-p M] [--seed S]
//   node cli.js bench    --model M.gguf --prompt-file ids.json --n 256 [--kv f16] [--ctx N] [--batch N]
//                        [--warmup W] [--prefill P1,P2] [--eager] [--sample] [--keys-per-split N]
//                        [--no-moe-grouped] [--no-moe-planes] [--no-fused-ffn] [--no-ffn-planes] [--no-norm-planes] [--no-merged-attention] [--attn-block] [--no-moe-router]
//   node cli.js motor    --servidor http://127.0.0.1:PORT [--id ID] [--kv f16] [--batch N]   (the server's engine)
//                        [--check-prompt-file ids.json --check-n N --check-logits file.f32]
//
// generate prints one JSON line {ids, prompt_ms, decode_ms, tps}; with --logits-out the logits each token was
// chosen from are appended to the file as float32 (vocab floats per token).  mode "ref" runs the reference op
// sequence (prompt pass included: no fused gate/up/SwiGLU) with a host argmax per token; "fast" runs the captured one-token graph with the device argmax;
// "engine" runs engine.generar with the given sampler parameters (no logits file); "sample" the sampled
// continuation with the host cross-check of every token (result field `control`).
// bench prefills the prompt, then times n decode steps (device events around the graph replays, and the wall
// clock) and prints {decode_tok_s, ms_per_token, ...}; with --check-prompt-file it first generates --check-n
// greedy tokens from that prompt on the fused path (ids in check_ids, logits to --check-logits) for a parity
// check by the caller.
const fs = require('fs');
const engine = require('./engine');
const { argmax, Muestreador } = require('./sampling');

function args(argv) {
  const o = { _: [] };
  for (let i = 0; i < argv.length; i++) {
    const a = argv[i];
    if (a.startsWith('--')) {
      const k = a.slice(2);
      if (i + 1 < argv.length && !argv[i + 1].startsWith('--')) o[k] = argv[++i]; else o[k] = true;
    } else o._.push(a);
  }
  return o;
}

async function cargar(o) {
  const options = { tiled_prefill: !o['no-tiled'], kv_f16: o.kv === 'f16' };
  if (o.batch) options.batch = parseInt(o.batch, 10);
  if (o['max-gen']) options.max_gen = parseInt(o['max-gen'], 10);
  if (o.eager) options.eager_decode = true;
  if (o['keys-per-split']) options.attn_keys_per_split = parseInt(o['keys-per-split'], 10);
  if (o['no-moe-grouped']) options.moe_grouped = false;
  // the reference's op sequence keeps gate, up and SwiGLU as three ops in the prompt pass too
  if (o['no-fused-ffn'] || o.mode === 'ref') options.fused_ffn = false;
  if (o['no-ffn-planes']) options.ffn_planes = false;
  if (o['no-norm-planes']) options.norm_planes = false;
  if (o['no-moe-planes']) options.moe_planes = false;
  if (o['no-merged-attention']) options.merged_attention = false;
  if (o['attn-block']) options.attn_block = true;
  if (o['no-moe-router']) options.moe_router = false;
  return engine.cargarModelo(o.model, { ctx: o.ctx ? parseInt(o.ctx, 10) : undefined, options: options });
}

async function generate(o) {
  const modelo = await cargar(o);
  const ids = JSON.parse(fs.readFileSync(o['prompt-file'], 'utf8'));
  const n = parseInt(o.n || '16', 10);
  const out = o['logits-out'] ? fs.openSync(o['logits-out'], 'w') : null;
  const escribe = function (lg) { if (out !== null) fs.writeSync(out, Buffer.from(lg.buffer, lg.byteOffset, lg.byteLength)); };
  const t0 = Date.now();
  const logits = await engine.prefill(modelo, ids);
  const tPrompt = Date.now();
  const toks = [];
  const extra = {};
  if (o.mode === 'engine') {
    // the engine's generation loop with sampler parameters (penalties -> host loop, greedy -> device loop)
    const params = { temperature: 0, max_tokens: n, host_loop: !!o['host-loop'] };
    for (const k of ['repeat_penalty', 'frequency_penalty', 'presence_penalty', 'temperature', 'top_k', 'top_p', 'min_p',
      'seed']) {
      const v = o[k.replace(/_/g, '-')];
      if (v !== undefined) params[k] = parseFloat(v);
    }
    const r = await engine.generar(modelo, ids, params);
    for (const t of r.ids) toks.push(t);
  } else if (o.mode === 'sample') {
    if (!modelo.pasoMuestreado) throw new Error('this model has no fused one-token plan for the sampled mode');
    // sampled continuation on the fused one-token plan (device penalties and top-k candidates, host draw); each
    // token is also chosen on the host from the same logits by a second sampler of the same seed (the reference's
    // procedure over the whole array), and the disagreements are counted
    const params = {};
    for (const k of ['repeat_penalty', 'frequency_penalty', 'presence_penalty', 'temperature', 'top_k', 'top_p', 'min_p',
      'seed']) {
      const v = o[k.replace(/_/g, '-')];
      if (v !== undefined) params[k] = parseFloat(v);
    }
    const mu = new Muestreador(params);
    const control = { mu: new Muestreador(params), penalizacion: 0, distintos: 0, candidatos: 0 };
    const hist = ids.slice();
    let id = mu.elegir(Float32Array.from(logits), hist);
    if (control.mu.elegir(Float32Array.from(logits), hist) !== id) control.distintos++;
    while (toks.length < n) {
      toks.push(id); hist.push(id);
      if (toks.length >= n) break;
      id = modelo.pasoMuestreado(id, mu, hist, control);
    }
    delete control.mu;
    extra.control = control;
  } else if (o.mode === 'ref' || !modelo.decodificarVoraz) {
    // the reference's loop (also the fast mode of models without the fused one-token plan)
    let lg = logits;
    while (toks.length < n) {
      escribe(lg);
      const t = argmax(lg);
      toks.push(t);
      if (toks.length >= n) break;
      lg = await modelo.forward([t], true);
    }
  } else if (o['force-ids']) {
    // teacher forcing on the fused one-token plan: step i consumes forced[i - 1] (step 0 is the prompt's last
    // token) and its logits and the device's argmax are recorded, so a checker that has the forced sequence can
    // compare every step even after a near tie sent the free-running sequences apart
    const forzados = JSON.parse(fs.readFileSync(o['force-ids'], 'utf8'));
    if (forzados.length < n) throw new Error('--force-ids holds ' + forzados.length + ' ids, fewer than --n');
    escribe(logits);
    toks.push(argmax(logits));
    if (n > 1) {
      const nuevos = modelo.decodificarVoraz(forzados[0], n - 1,
        { forzar: forzados.slice(1, n - 1), porPaso: function (i, t, lg) { escribe(lg); } });
      for (const t of nuevos) toks.push(t);
    }
    extra.forced = true;
  } else {
    escribe(logits);
    toks.push(argmax(logits));
    if (n > 1) {
      const nuevos = modelo.decodificarVoraz(toks[0], n - 1, out !== null ? { porPaso: function (i, t, lg) { if (i < n - 1) escribe(lg); } } : {});
      for (const t of nuevos) toks.push(t);
    }
  }
  const tEnd = Date.now();
  if (out !== null) fs.closeSync(out);
  if (o['kv-out']) modelo.volcarKV(o['kv-out']);
  const r = Object.assign({ ids: toks, prompt_ms: tPrompt - t0, decode_ms: tEnd - tPrompt, pos: modelo.pos }, extra);
  modelo.free();
  process.stdout.write(JSON.stringify(r) + '\n');
}

// One decode measurement after prefilling the first P ids: warm-up steps (then the position is rewound; the KV
// slots they wrote are overwritten by the timed run), then n timed steps.
async function medir(modelo, ids, P, n, warm, eager, muestreo) {
  const gpu = modelo.gpu;
  const tp0 = Date.now();
  const logits = await engine.prefill(modelo, ids.slice(0, P));
  gpu.sincronizar();
  const prefillMs = Date.now() - tp0;
  const primero = argmax(logits);
  const pos0 = modelo.pos;
  if (warm > 0) {
    modelo.decodificarVoraz(primero, warm);
    gpu.sincronizar();
    modelo.pos = pos0;
    modelo.hist.length = Math.min(modelo.hist.length, pos0);
  }
  const tiempos = {};
  const tw0 = process.hrtime.bigint();
  const toks = modelo.decodificarVoraz(primero, n, { tiempos: tiempos, eager: eager });
  const wallMs = Number(process.hrtime.bigint() - tw0) / 1e6;
  const r = {
    prompt_tokens: P, n: n, decode_tok_s: n / (tiempos.ms / 1000), ms_per_token: tiempos.ms / n,
    device_ms: tiempos.ms, wall_ms: wallMs, wall_tok_s: n / (wallMs / 1000), prefill_ms: prefillMs,
    prefill_tok_s: P / (prefillMs / 1000), first_ids: [primero].concat(toks.slice(0, 7)),
  };
  if (muestreo) {
    // the same n steps from the same position with the reference's default sampler (temperature 0.8, top_k 40,
    // top_p 0.95, min_p 0.05) and a fixed seed: one graph step, the device top-k and the host draw per token,
    // timed on the wall clock (the host takes part in every token)
    modelo.pos = pos0;
    modelo.hist.length = Math.min(modelo.hist.length, pos0);
    const mu = new Muestreador({ seed: 1 });
    const hist = [primero];
    let id = primero;
    const ts0 = process.hrtime.bigint();
    for (let i = 0; i < n; i++) { id = modelo.pasoMuestreado(id, mu, hist); hist.push(id); }
    gpu.sincronizar();
    const ms = Number(process.hrtime.bigint() - ts0) / 1e6;
    r.sampled_tok_s = n / (ms / 1000);
    r.sampled_ms_per_token = ms / n;
    r.sampled_first_ids = hist.slice(0, 8);
  }
  return r;
}

// Greedy generation of n tokens from `ids` on the fused path, with the logits each token was chosen from
// written to `archivo` (float32, vocab per token).  Returns the ids.
async function chequeo(modelo, ids, n, archivo) {
  const out = fs.openSync(archivo, 'w');
  const escribe = function (lg) { fs.writeSync(out, Buffer.from(lg.buffer, lg.byteOffset, lg.byteLength)); };
  const logits = await engine.prefill(modelo, ids);
  escribe(logits);
  const toks = [argmax(logits)];
  if (n > 1) {
    const nuevos = modelo.decodificarVoraz(toks[0], n - 1, { porPaso: function (i, t, lg) { escribe(lg); } });
    for (const t of nuevos) toks.push(t);
  }
  fs.closeSync(out);
  return toks;
}

async function bench(o) {
  const tLoad = Date.now();
  const modelo = await cargar(o);
  const loadMs = Date.now() - tLoad;
  let check = null;
  if (o['check-prompt-file']) {
    const cids = JSON.parse(fs.readFileSync(o['check-prompt-file'], 'utf8'));
    check = await chequeo(modelo, cids, parseInt(o['check-n'] || '8', 10), o['check-logits']);
  }
  const ids = JSON.parse(fs.readFileSync(o['prompt-file'], 'utf8'));
  const n = parseInt(o.n || '256', 10);
  const warm = parseInt(o.warmup || '8', 10);
  const prefills = (o.prefill ? String(o.prefill) : String(ids.length)).split(',').map(function (x) { return parseInt(x, 10); });
  const runs = [];
  for (const P of prefills) {
    if (P > ids.length) throw new Error('prompt file has ' + ids.length + ' ids, ' + P + ' requested');
    runs.push(await medir(modelo, ids, P, n, warm, !!o.eager, !!o.sample));
  }
  const r = { runs: runs, load_ms: loadMs, ctx: modelo.ctx, nsplit: modelo.nsplit, kv_f16: modelo.kvF16,
    batch: modelo.batch, bytes_on_gpu: modelo.gpu.bytesUsados, check_ids: check };
  modelo.free();
  process.stdout.write(JSON.stringify(r) + '\n');
}

// The engine of quipullm's server (motor.js): hello, then jobs from the long poll until the server says "cerrar".
async function motor(o) {
  const { Motor } = require('./motor');
  const opciones = { kv_f16: o.kv === 'f16' };
  if (o.batch) opciones.batch = parseInt(o.batch, 10);
  if (o['max-gen']) opciones.max_gen = parseInt(o['max-gen'], 10);
  if (o['keys-per-split']) opciones.attn_keys_per_split = parseInt(o['keys-per-split'], 10);
  const m = new Motor({ servidor: o.servidor || 'http://127.0.0.1:8080', id: o.id, opciones: opciones });
  const r = await m.correr();
  process.stdout.write(JSON.stringify({ fin: r }) + '\n');
}

const o = args(process.argv.slice(2));
const cmd = o._[0];
const fn = { generate: generate, bench: bench, motor: motor }[cmd];
if (!fn) {
  process.stderr.write('usage: node cli.js generate|bench --model M.gguf --prompt-file ids.json ... | motor --servidor URL\n');
  process.exit(2);
}
fn(o).catch(function (e) {
  process.stderr.write('error: ' + (e && e.stack ? e.stack : e) + '\n');
  process.exit(1);
});
