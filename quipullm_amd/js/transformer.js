'use strict';
// Llama-style decoder on the gfx950 backend: the dense architectures (llama, qwen3) and the GQA
// mixture-of-experts variant (qwen3moe).
//
// Plugin interface of quipullm's model classes (docs/ARCH_GUIDE.md:52-65, used by engine.js:104-125 and
// 265-312): new Clase(gpu, meta); load(path, progress); reset(); forward(ids, wantLogits) -> Float32Array |
// null; free(); properties nLayers, D, ctx, batch, vocab.  forward() issues the reference's op sequence
// (transformer.js:252-336; the MoE FFN of deepseek2.js:374-386 without shared experts) through the named-op
// facade.  decodificarVoraz() is this backend's fast path for greedy decoding: the whole one-token step is
// captured once in a HIP graph with fused kernels (norm folded into the GEMVs, split-K attention with RoPE and
// the KV append, SwiGLU folded into the gate/up GEMV, residual adds in the epilogues) and the argmax stays on
// the device, feeding the next step's token id.
const { despachar, dim2, vista } = require('./gpu');
const { CargadorPesos } = require('./weights');

const ROPE_NEOX = new Set(['qwen2', 'qwen3', 'qwen3moe', 'phi3', 'gemma', 'gemma2', 'gemma3', 'stablelm', 'olmo2']);
const KQ = new Set(['q2k', 'q3k', 'q4k', 'q5k', 'q6k']);
const MEZCLA = new Set(['q4k', 'q6k']);    // formats whose GEMV segments may share one launch
const EG = new Set(['q2k', 'q3k', 'q4k', 'q5k', 'q6k', 'q8', 'f32', 'iq4nl']);   // grouped expert matmul (matmul_<fmt>_eg)
// handles bound as two buffers (quants, scales): Q8_0 and IQ4_NL
function plano(W) { return W.tipo === 'q8' || W.tipo === 'iq4nl'; }
// moe_group lists at most 65535 jobs (16-bit counts) of at most 256 experts: a batch whose jobs (tokens x
// experts used) exceed that takes the ungrouped per-job expert path instead of failing.
const MOE_GROUP_JOBS = 65535, MOE_GROUP_EXPERTS = 256;
function agrupable(formatos, batch, nUsados, nExp) {
  return formatos && batch * nUsados <= MOE_GROUP_JOBS && nExp <= MOE_GROUP_EXPERTS;
}
const FMT_ID = { f32: 0, q8: 8, q2k: 10, q3k: 11, q4k: 12, q5k: 13, q6k: 14, iq4nl: 20 };
// gemv segment modes (qp_args.h)
const STORE = 0, ACC = 1, SWIGLU = 2, ARGMAX = 3;
const AMAX_WG = 512;   // workgroups of the fused output GEMV = partial maxima for the device argmax

class ModeloTransformer {
  constructor(gpu, meta) {
    this.gpu = gpu;
    this.meta = meta;
    const kv = meta.kv, a = kv['general.architecture'];
    this.arch = a;
    const g = function (k, d) { return kv[a + '.' + k] !== undefined ? kv[a + '.' + k] : d; };
    this.nLayers = g('block_count');
    this.D = g('embedding_length');
    this.nh = g('attention.head_count');
    const hkv = g('attention.head_count_kv', this.nh);
    if (Array.isArray(hkv)) throw new Error('per-layer KV head counts are not supported by this backend');
    this.nkv = hkv;
    this.hd = g('attention.key_length', this.D / this.nh);
    this.eps = g('attention.layer_norm_rms_epsilon', 1e-5);
    this.base = g('rope.freq_base', 10000);
    this.nrot = g('rope.dimension_count', this.hd);
    const oa = meta.arch_options || {};
    this.neox = oa.rope ? (oa.rope === 'neox' ? 1 : 0) : (ROPE_NEOX.has(a) ? 1 : 0);
    this.escAtt = g('attention.scale', 0) || 1 / Math.sqrt(this.hd);
    // scales (0: none) and soft-capping of the logits, as the reference reads them (transformer.js:35-45)
    this.escEmb = g('embedding_scale', 0) || 0;
    this.escRes = g('residual_scale', 0) || 0;
    this.escLogit = g('logit_scale', 0) || 0;
    if (oa.embedding_scale === 'sqrt_d') this.escEmb = Math.fround(Math.sqrt(this.D));
    else if (typeof oa.embedding_scale === 'number') this.escEmb = oa.embedding_scale;
    this.softcap = g('final_logit_softcapping', 0) || 0;
    // gemma3 (transformer.js:46-54): sliding windows on all but every `patron`-th layer, their own RoPE base, the
    // global layers' linear RoPE scaling, sqrt(D) embedding scale, GeGLU
    this.gemma = a === 'gemma3';
    this.ventana = 0;
    if (this.gemma) {
      this.ventana = g('attention.sliding_window', 0) || 0;
      this.patron = g('attention.sliding_window_pattern', 6) || 6;
      this.baseSwa = g('rope.freq_base_swa', 10000);
      const fac = g('rope.scaling.factor', 1);
      this.escalaGlobal = g('rope.scaling.type', '') === 'linear' && fac > 0 ? 1 / fac : 1;
      this.escEmb = Math.fround(Math.sqrt(this.D));
      this.escAtt = this.nLayers === 62 ? 1 / Math.sqrt(this.D / this.nh) : 1 / Math.sqrt(this.hd);
    }
    this.ctx = meta.ctx || 4096;
    this.vocab = kv['tokenizer.ggml.tokens'].length;
    this.nExp = g('expert_count', 0);
    this.nUsados = g('expert_used_count', 0);
    this.ffe = g('expert_feed_forward_length', 0);
    this.normExp = !!g('expert_weights_norm', false);
    this.escExp = g('expert_weights_scale', 1) || 1;
    if (this.nExp > 1024 || this.nUsados > this.nExp) throw new Error(a + ': expert count not supported');
    if (this.hd !== 64 && this.hd !== 128) throw new Error('head_dim ' + this.hd + ' not supported (64 or 128)');
    if (this.nh % this.nkv || this.nh / this.nkv > 8) throw new Error('GQA group ' + this.nh + '/' + this.nkv + ' not supported');
    const op = meta.options || {};
    this.batch = op.batch || 32;                 // tokens per prefill pass (reference transformer.js:10 uses 32)
    this.kvF16 = !!op.kv_f16;                    // f16 KV cache (the reference keeps it in f32)
    this.eagerDecode = !!op.eager_decode;        // fused step dispatched op by op instead of a captured graph
    // decode attention: keys per workgroup at full context: 256 (two 32-key tiles per wavefront) while that still
    // gives at least 64 workgroups (nkv x splits), else 128
    this.attnPorSplit = op.attn_keys_per_split || (this.nkv * Math.ceil(this.ctx / 256) >= 64 ? 256 : 128);
    this.baldosa = op.tiled_prefill !== false;   // config.json "tiled_prefill"
    // MoE prompt batches of 8 or more tokens grouped by expert on the matrix cores (moe_group + matmul_*_eg, the
    // reference's deepseek2.js:353-378); false: one job per (token, expert) on the expert GEMV
    this.agrupado = op.moe_grouped !== false;
    // dense FFN of prompt chunks of 256 tokens or more: gate, up and SwiGLU as one matrix-core launch
    // (matmul_<fmt>_t_swiglu, the same results as the reference's matmul_<fmt>_t, matmul_<fmt>_t, swiglu of
    // transformer.js:311-313); false: those three ops
    this.ffnFusionada = op.fused_ffn !== false;
    // with K-quant down weights that launch writes the down matmul's input planes itself (matmul_<fmt>_t_swiglu
    // P[2] = 1, matmul_<fmt>_t P[4] = 2: the same planes qp_split_bf16 makes of its f32 outputs, without the f32 round
    // trip and the split launch); false: f32 outputs, split by the down matmul
    this.planosFfn = op.ffn_planes !== false;
    // prompt chunks of 256 tokens or more: the attention (and dense FFN) norm writes the bf16 input planes of the
    // K-quant matmuls that read it (rmsnorm_planes; Q, K, V with P[4] = 2, the fused gate/up with P[3] = 1) instead
    // of f32 rows that each matmul splits; false: rmsnorm
    this.planosNorma = op.norm_planes !== false;
    // MoE prompt batches grouped by expert: each expert matmul's input split into bf16 planes once (matmul_<fmt>_eg
    // P[4] = rows per token: 1 for gate and up, the top-k count for down; up reuses gate's planes, P[5] = 1) instead
    // of in every tile that reads a row; the same sums bit for bit.  false: f32 rows split in the tiles
    this.planosMoe = op.moe_planes !== false;
    // one-token step: the split-K attention's partials merged by the last workgroup of each grid column in the same
    // launch (dec_attn P[12] = 1) instead of a dec_attn_comb launch.  A column takes at most 4 query heads: groups of
    // 8 or more query heads are split over gsplit columns per KV head (P[13]; each column streams its KV head's keys
    // and merges its own heads), as long as the columns fit the 8 XCDs.  Measured: 8B decode 449 -> 455 tok/s; MoE
    // (8 query heads per KV head): one workgroup merging all 8 cost more than the launch it saved (400 -> 396),
    // two columns of 4 heads each 402 -> 421 tok/s; false: the separate merge
    const grupoQ = this.nh / this.nkv;
    this.gsplitAtt = 1;
    while (grupoQ / this.gsplitAtt > 4 && this.gsplitAtt < 8) this.gsplitAtt *= 2;
    this.atencionUnida = op.merged_attention !== false && this.nkv * this.gsplitAtt <= 8 &&
      grupoQ % this.gsplitAtt === 0 && grupoQ / this.gsplitAtt <= 4;
    // one-token step: each layer's Q/K/V GEMV, attention, KV append and split merge as one launch (dec_attn_block,
    // eight head groups on the eight XCDs meeting at barriers in their L2) where the layer fits it (_bloqueAtt).
    // Off unless asked: measured no faster than the separate launches (8B at ctx 4096 450 against 455 tok/s, MoE
    // at ctx 2048 398 against 397): the chain of dependent memory round trips is as long with barriers as with
    // launch boundaries.
    this.bloqueAtt = op.attn_block === true;
    // one-token MoE step: the router GEMV and the routing in one launch (moe_router; f32 routers); false: the router
    // GEMV, with the routing computed by every workgroup of the gate/up kernel
    this.enrutador = op.moe_router !== false;
    this.bufs = [];
    this.pos = 0;
    this.grafo = null;
    // prompt cache (the reference's interface, engine.js:254-290 / lfm2.js:205-245): the ids whose KV rows are
    // written, in order; hist.length === pos whenever the cache is usable
    this.cacheOn = op.prompt_cache !== false;
    this.hist = [];
    this.intervaloCP = 64;
    // The fused one-token plan (decodificarVoraz, pasoMuestreado) covers the llama / qwen families; models with
    // scales, soft-capping or gemma3's post norms, GeGLU and windows decode through forward(), the reference's op
    // sequence, one token at a time (engine.generar takes that path when the fused methods are absent).
    this.fusion = !this.gemma && !this.escEmb && !this.escRes && !this.escLogit && !this.softcap;
    if (!this.fusion) {
      this.decodificarVoraz = null;
      this.pasoMuestreado = null;
    }
  }

  esSwa(i) { return this.ventana > 0 && (i % this.patron) < this.patron - 1; }

  // fuente: the GGUF path, or {url} of the server's file route (tensors fetched by ranges, layer by layer)
  async load(fuente, progreso) {
    const gpu = this.gpu, c = new CargadorPesos(gpu, this.meta, fuente, progreso);
    this.cargador = c;
    try {
      if (c.existe('rope_freqs.weight')) throw new Error('this model uses rope_freqs.weight (scaled RoPE), which is not supported');
      await c.precargar(['token_embd.weight', 'output.weight', 'output_norm.weight']);
      this.emb = c.matriz('token_embd.weight');
      this.vocab = this.emb.N;
      this.salida = c.existe('output.weight') ? c.matriz('output.weight') : this.emb;
      this.normFinal = c.f32('output_norm.weight');
      this.capas = [];
      let F = 0, ceros = null;
      for (let i = 0; i < this.nLayers; i++) {
        const p = 'blk.' + i + '.';
        for (const n of ['attn_q.bias', 'attn_k.bias', 'attn_v.bias', 'attn_output.bias'])
          if (c.existe(p + n)) throw new Error(p + n + ': biases are not supported by this backend');
        await c.precargar(['attn_norm', 'attn_q', 'attn_k', 'attn_v', 'attn_output', 'attn_q_norm', 'attn_k_norm',
          'ffn_norm', 'ffn_gate_inp', 'ffn_gate_exps', 'ffn_up_exps', 'ffn_down_exps', 'ffn_gate', 'ffn_up',
          'ffn_down'].map(function (n) { return p + n + '.weight'; }));
        const capa = {};
        capa.attnNorm = c.f32(p + 'attn_norm.weight');
        capa.wq = c.matriz(p + 'attn_q.weight');
        capa.wk = c.matriz(p + 'attn_k.weight');
        capa.wv = c.matriz(p + 'attn_v.weight');
        capa.wo = c.matriz(p + 'attn_output.weight');
        capa.qNorm = c.existe(p + 'attn_q_norm.weight') ? c.f32(p + 'attn_q_norm.weight') : null;
        capa.kNorm = c.existe(p + 'attn_k_norm.weight') ? c.f32(p + 'attn_k_norm.weight') : null;
        capa.ffnNorm = c.f32(p + 'ffn_norm.weight');
        // outputs normalized before the residual add (gemma3; transformer.js:100-101, 218-226)
        capa.postAtt = c.existe(p + 'post_attention_norm.weight') ? c.f32(p + 'post_attention_norm.weight') : null;
        capa.postFfn = c.existe(p + 'post_ffw_norm.weight') ? c.f32(p + 'post_ffw_norm.weight') : null;
        if (this.nExp && (capa.postAtt || capa.postFfn || this.escRes))
          throw new Error('layer ' + i + ': post norms and residual scales are not supported with experts');
        if (capa.postAtt || capa.postFfn) {
          this.fusion = false;
          this.decodificarVoraz = null;
          this.pasoMuestreado = null;
        }
        if (this.nExp) {
          capa.router = c.matriz(p + 'ffn_gate_inp.weight');
          capa.eg = c.matriz(p + 'ffn_gate_exps.weight');
          capa.eu = c.matriz(p + 'ffn_up_exps.weight');
          capa.ed = c.matriz(p + 'ffn_down_exps.weight');
          if (capa.eg.N !== this.nExp * this.ffe || capa.ed.N !== this.nExp * this.D)
            throw new Error('layer ' + i + ': unexpected expert dimensions');
        } else {
          capa.gate = c.matriz(p + 'ffn_gate.weight');
          capa.up = c.matriz(p + 'ffn_up.weight');
          capa.down = c.matriz(p + 'ffn_down.weight');
          F = Math.max(F, capa.gate.N);
        }
        const kvd = this.nkv * this.hd, eb = this.kvF16 ? 2 : 4;
        // windowed layers keep a ring of window + batch slots (transformer.js:106-111): position p in slot p % cap
        // holds the window of every token of a batch as it is processed
        capa.swa = this.esSwa(i) ? this.ventana : 0;
        capa.anillo = capa.swa && this.ctx > capa.swa + this.batch ? capa.swa + this.batch : 0;
        capa.slots = capa.anillo || this.ctx;
        capa.kc = gpu.buffer(capa.slots * kvd * eb, undefined, 'kcache' + i);
        // the f16 value cache is stored in whole tiles of 32 slots, read whole by the decode attention: it starts
        // zeroed so that slots not yet written hold finite values (they are weighted by 0)
        const vBytes = (this.kvF16 ? Math.ceil(capa.slots / 32) * 32 : capa.slots) * kvd * eb;
        capa.vc = gpu.buffer(vBytes, undefined, 'vcache' + i);
        if (!ceros || ceros.length < vBytes) ceros = new Uint8Array(vBytes);
        gpu.escribir(capa.vc, 0, ceros.subarray(0, vBytes));
        this.bufs.push(capa.kc, capa.vc);
        this.capas.push(capa);
      }
      this.F = F;
    } finally {
      c.cerrar();
    }
    const B = (n, l) => { const b = gpu.buffer(n, undefined, l); this.bufs.push(b); return b; };
    const TB = this.batch, D = this.D, qd = this.nh * this.hd, kvd = this.nkv * this.hd;
    // the bf16 input planes the norms and the attention write for prompt chunks of 256 tokens or more (256-token
    // rows of the wider of the model and attention widths)
    this.xsPl = TB >= 256 ? B(4 * Math.ceil(TB / 256) * 256 * Math.max(D, qd), 'x_planes') : null;
    const FF = this.nExp ? this.nUsados * this.ffe : this.F;
    this.bPaso = B(16, 'paso');
    this.bIds = B(4 * TB, 'ids');
    gpu.escribir(this.bIds, 0, new Uint32Array(TB));   // device memory starts undefined; ids index the embeddings
    this.x = B(4 * TB * D, 'x');
    this.xn = B(4 * TB * D, 'xn');
    this.q = B(4 * TB * qd, 'q');
    this.k = B(4 * TB * kvd, 'k');
    this.v = B(4 * TB * kvd, 'v');
    this.att = B(4 * TB * qd, 'att');
    // (dense FFN: room for the down matmul's input planes, 256-token rows, that the fused gate/up writes here)
    this.g = B(4 * (this.nExp ? TB : Math.ceil(TB / 256) * 256) * FF, 'g');
    this.u = B(4 * TB * FF, 'u');
    if (this.nExp) {
      this.rl = B(4 * TB * this.nExp, 'router_logits');
      this.sel = B(4 * TB * this.nUsados, 'sel');
      this.wts = B(4 * TB * this.nUsados, 'wts');
      this.de = B(4 * TB * this.nUsados * D, 'de');
      this.lst = B(4 * TB * this.nUsados, 'lst');
      this.off = B(4 * (this.nExp + 1), 'off');
    }
    if (!this.fusion) this.tmp = B(4 * TB * D, 'tmp');   // a block's output before its norm / scaled add
    this.xl = B(4 * D, 'xlast');
    this.logits = B(4 * this.vocab, 'logits');
    // decode fast path
    // split-K decode attention: workgroups per KV head (each covers ctx / nsplit keys at the longest context)
    this.nsplit = Math.max(1, Math.min(256, Math.ceil(this.ctx / this.attnPorSplit)));
    this.partO = B(4 * this.nh * this.nsplit * this.hd, 'attn_part_o');
    this.partML = B(8 * this.nh * this.nsplit, 'attn_part_ml');
    // the merged attention's arrival counters (kept at zero by it) and its error word at byte 1024
    this.attCnt = B(8 * 128 + 128, 'attn_counters');
    gpu.escribir(this.attCnt, 0, new Uint8Array(8 * 128 + 128));
    // dec_attn_block: 64 workgroups per head group (two per CU of an XCD: every wavefront then has at most one
    // unit of the Q/K/V GEMV), their partials, and the op's sync words (barrier counters, XCD words, error word),
    // zero at allocation and touched by that op only
    const cusXcd = Math.max(1, Math.floor((gpu.info.cus || 256) / 8));
    this.nsBloque = 1;
    while (this.nsBloque * 2 <= Math.min(64, 2 * cusXcd, (this.nh / 8) * this.hd)) this.nsBloque *= 2;
    this.partOB = B(4 * this.nh * this.nsBloque * this.hd, 'block_part_o');
    this.partMLB = B(8 * this.nh * this.nsBloque, 'block_part_ml');
    this.syncBloque = B(2304, 'block_sync');
    gpu.escribir(this.syncBloque, 0, new Uint8Array(2304));
    if (this.nExp) {
      // moe_router: workgroups (a power of two, four router rows each, at most two per CU of an XCD) and their
      // arrival counter, zero at allocation and touched by that op only
      this.nwRouter = 1;
      while (this.nwRouter * 4 < this.nExp && this.nwRouter * 2 <= 2 * cusXcd) this.nwRouter *= 2;
      this.routerCnt = B(8, 'router_counter');   // arrival counter, then the error word
      gpu.escribir(this.routerCnt, 0, new Uint8Array(8));
    }
    this.ropeFreq = B(4 * Math.max(1, this.nrot / 2), 'rope_freq');
    gpu.escribir(this.ropeFreq, 0, tablaRope(this.base, this.nrot));
    this.amax = B(8 * AMAX_WG, 'argmax_partials');
    gpu.escribir(this.amax, 0, new Uint8Array(8 * AMAX_WG));
    this.maxGen = op_max_gen(this.meta);
    this.tokens = B(4 * this.maxGen, 'tokens');
    // sampling on the device: top-k partials (ceil(V/2048) chunks x (k + 1) keys, k <= 128, plus a flag each),
    // the candidates read back, and the penalty window's (token, count) pairs
    const nParte = Math.ceil(this.vocab / 2048);
    this.candParte = B(nParte * 129 * 8 + nParte * 4, 'topk_partials');
    this.candSalida = B(4 * (2 + 2 * 128), 'topk_candidates');
    this.penPares = B(4 * 2 * 64, 'penalty_pairs');
    this.contador = B(16, 'step_counter');
    this._armarGrupos();
    if (this.fusion) this.prepararDecode();
    this.reset();
    return Promise.resolve();
  }

  // ---------------------------------------------------------------- reference op sequence
  // matmul of the reference facade: one token -> matmul_<t>_1; T >= 8 with a K-quant and tiling -> _t; else _4
  // (transformer.js:268-284).
  // reusa: x is the input of the matmul dispatched just before (Q, K, V): the tiled form may reuse the bf16 planes
  // that matmul split it into (P[4] = 1, an addition of this backend's; the reference's P has four words).
  // planos: x holds those planes already, written by the fused gate/up (P[4] = 2; the tiled form only).
  _mm(W, x, y, acc, reusa, planos) {
    const gpu = this.gpu;
    const u = gpu.uniforme([['u', W.N], ['u', W.K], ['u', acc ? 1 : 0], ['u', 0]]);
    const wb = plano(W) ? [W.qs, W.ds] : [W.w];
    const b = [u, this.bPaso].concat(wb, [x, y]);
    const modo = planos ? 2 : reusa && this.fusion ? 1 : 0;
    const bt = modo ? [gpu.uniforme([['u', W.N], ['u', W.K], ['u', acc ? 1 : 0], ['u', 0], ['u', modo]]),
      this.bPaso].concat(wb, [x, y]) : b;
    return {
      uno: gpu.grupo('matmul_' + W.tipo + '_1', b), lote: gpu.grupo('matmul_' + W.tipo + '_4', b),
      baldosa: this.baldosa && KQ.has(W.tipo) ? gpu.grupo('matmul_' + W.tipo + '_t', bt) : null, filas: W.N,
    };
  }

  _mmE(W, x, y, tfijo, filasTok, reusa) {
    const gpu = this.gpu;
    const u = gpu.uniforme([['u', W.N / this.nExp], ['u', W.K], ['u', 0], ['u', tfijo], ['u', this.nExp]]);
    const wb = plano(W) ? [W.qs, W.ds] : [W.w];
    // grouped by expert (the reference's matmul_<fmt>_eg: P{N, K, acc, tfijo}; [paso, w, x, y, lst, off])
    const ug = gpu.uniforme([['u', W.N / this.nExp], ['u', W.K], ['u', 0], ['u', tfijo]].concat(
      this.planosMoe ? [['u', filasTok], ['u', reusa ? 1 : 0]] : []));
    const gg = EG.has(W.tipo) ? gpu.grupo('matmul_' + W.tipo + '_eg', [ug, this.bPaso].concat(wb, [x, y, this.lst, this.off])) : null;
    return { g: gpu.grupo('matmul_' + W.tipo + '_e', [u, this.bPaso].concat(wb, [x, y, this.sel])), gg: gg, filas: W.N / this.nExp };
  }

  _embedGrupo(ids, y) {
    const gpu = this.gpu, E = this.emb;
    const u = gpu.uniforme([['u', this.D], ['u', E.N]]);
    const wb = plano(E) ? [E.qs, E.ds] : [E.w];
    return gpu.grupo('embed_' + E.tipo, [u, this.bPaso].concat(wb, [ids, y]));
  }

  _armarGrupos() {
    const gpu = this.gpu, D = this.D, P = this.bPaso;
    const G = {};
    G.embed = this._embedGrupo(this.bIds, this.x);
    if (this.escEmb) G.escEmb = gpu.grupo('escalar', [gpu.uniforme([['u', D], ['f', this.escEmb]]), P, this.x]);
    const uNorm = gpu.uniforme([['u', D], ['u', 0], ['f', this.eps], ['u', 0]]);
    const dummy = this.normFinal;
    const f16 = this.kvF16 ? 1 : 0;
    const kvd = this.nkv * this.hd;
    const resid = this.escRes || 1;
    // a block's output into the residual (transformer.js:218-233): added by the matmul itself (acc = 1), or, with
    // a post norm or a residual scale, written to tmp, normalized, then x += resid * it (suma_esc)
    const directo = (W, x, post, planos) => {
      if (!post && resid === 1) return { mm: this._mm(W, x, this.x, 1, false, planos) };
      return {
        mm: this._mm(W, x, this.tmp, 0, false, planos),
        norma: post ? gpu.grupo('rmsnorm', [uNorm, P, this.tmp, post, this.xn]) : null,
        suma: gpu.grupo('suma_esc', [gpu.uniforme([['u', D], ['f', resid]]), P, this.x, post ? this.xn : this.tmp]),
      };
    };
    G.capas = this.capas.map((c) => {
      const baseCapa = this.gemma && c.swa ? this.baseSwa : this.base;
      const tablaCapa = baseCapa === this.base ? [this.ropeFreq] : [];
      const escRope = this.gemma && !c.swa ? this.escalaGlobal : 1;
      const ur = (nh, norm) => gpu.uniforme([['u', this.hd], ['u', nh], ['u', norm ? 1 : 0], ['u', this.neox],
        ['f', this.eps], ['f', baseCapa], ['u', this.nrot], ['f', escRope === 1 ? 0 : escRope]]);
      const gc = {
        attnNorm: gpu.grupo('rmsnorm', [uNorm, P, this.x, c.attnNorm, this.xn]),
        ffnNorm: gpu.grupo('rmsnorm', [uNorm, P, this.x, c.ffnNorm, this.xn]),
        wq: this._mm(c.wq, this.xn, this.q, 0), wk: this._mm(c.wk, this.xn, this.k, 0, true),
        wv: this._mm(c.wv, this.xn, this.v, 0, true),
        // (the layer's frequency table when it has the model's base: no power evaluated in the kernel)
        ropeQ: gpu.grupo('norm_rope', [ur(this.nh, !!c.qNorm), P, this.q, c.qNorm || dummy].concat(tablaCapa)),
        ropeK: gpu.grupo('norm_rope', [ur(this.nkv, !!c.kNorm), P, this.k, c.kNorm || dummy].concat(tablaCapa)),
        kvw: gpu.grupo('kv_write', [gpu.uniforme([['u', kvd], ['u', c.anillo], ['u', f16], ['u', c.slots]]), P, this.k, this.v,
          c.kc, c.vc]),
        att: gpu.grupo('atencion', [gpu.uniforme([['u', this.hd], ['u', this.nh], ['u', this.nkv], ['u', c.swa],
          ['f', this.escAtt], ['u', c.anillo], ['u', 0], ['u', 0], ['u', f16], ['u', c.slots]]), P, this.q, c.kc, c.vc, this.att]),
        wo: directo(c.wo, this.att, c.postAtt),
      };
      // the attention norm as input planes of Q, K and V (all K-quant, tiled)
      const uPl = gpu.uniforme([['u', D], ['f', this.eps]]);
      const pl = this.planosNorma && this.fusion && this.baldosa && this.xsPl && D % 32 === 0;
      if (pl && KQ.has(c.wq.tipo) && KQ.has(c.wk.tipo) && KQ.has(c.wv.tipo)) {
        gc.attnNormPl = gpu.grupo('rmsnorm_planes', [uPl, P, this.x, c.attnNorm, this.xsPl]);
        gc.wqPl = this._mm(c.wq, this.xsPl, this.q, 0, false, true);
        gc.wkPl = this._mm(c.wk, this.xsPl, this.k, 0, false, true);
        gc.wvPl = this._mm(c.wv, this.xsPl, this.v, 0, false, true);
      }
      // the attention's output as wo's input planes (the matrix-core attention: f16 cache, no window or ring)
      const grupoQ = this.nh / this.nkv, qd = this.nh * this.hd;
      if (pl && KQ.has(c.wo.tipo) && f16 && !c.swa && !c.anillo && [1, 2, 4, 8].includes(grupoQ) && qd % 32 === 0) {
        gc.attPl = gpu.grupo('atencion', [gpu.uniforme([['u', this.hd], ['u', this.nh], ['u', this.nkv], ['u', c.swa],
          ['f', this.escAtt], ['u', c.anillo], ['u', 0], ['u', 0], ['u', f16], ['u', c.slots], ['u', 1]]), P, this.q,
          c.kc, c.vc, this.xsPl]);
        gc.woPl = directo(c.wo, this.xsPl, c.postAtt, true);
      }
      if (this.nExp) {
        const K = this.nUsados;
        gc.router = this._mm(c.router, this.xn, this.rl, 0);
        gc.topk = gpu.grupo('moe_topk', [gpu.uniforme([['u', this.nExp], ['u', K], ['u', this.normExp ? 1 : 0],
          ['f', this.escExp]]), P, this.rl, this.sel, this.wts]);
        gc.eg = this._mmE(c.eg, this.xn, this.g, K, 1, false);
        gc.eu = this._mmE(c.eu, this.xn, this.u, K, 1, true);
        gc.eact = gpu.grupo('swiglu', [gpu.uniforme([['u', K * this.ffe]]), P, this.g, this.u]);
        gc.ed = this._mmE(c.ed, this.g, this.de, 1, K, false);
        gc.comb = gpu.grupo('moe_comb', [gpu.uniforme([['u', D], ['u', K]]), P, this.x, this.de, this.wts]);
        gc.grupar = gpu.grupo('moe_group', [gpu.uniforme([['u', this.nExp], ['u', K]]), P, this.sel, this.lst, this.off]);
        gc.agrupado = agrupable(!!(gc.eg.gg && gc.eu.gg && gc.ed.gg), this.batch, K, this.nExp);
      } else {
        gc.gate = this._mm(c.gate, this.xn, this.g, 0);
        gc.up = this._mm(c.up, this.xn, this.u, 0);
        if (this.ffnFusionada && this.fusion && this.baldosa && KQ.has(c.gate.tipo) && c.up.tipo === c.gate.tipo &&
            c.up.N === c.gate.N && c.up.K === c.gate.K) {
          // with K-quant down weights the fused gate/up writes the down matmul's input planes (no split between them)
          const yp = KQ.has(c.down.tipo) && c.down.K === c.gate.N && this.planosFfn;
          gc.glu = gpu.grupo('matmul_' + c.gate.tipo + '_t_swiglu', [gpu.uniforme([['u', c.gate.N], ['u', c.gate.K],
            ['u', yp ? 1 : 0]]), P, c.gate.w, c.up.w, this.xn, this.g]);
          if (yp) gc.downPl = directo(c.down, this.g, c.postFfn, true);
          // the FFN norm as the fused launch's input planes
          if (pl) {
            gc.ffnNormPl = gpu.grupo('rmsnorm_planes', [uPl, P, this.x, c.ffnNorm, this.xsPl]);
            gc.gluPl = gpu.grupo('matmul_' + c.gate.tipo + '_t_swiglu', [gpu.uniforme([['u', c.gate.N],
              ['u', c.gate.K], ['u', yp ? 1 : 0], ['u', 1]]), P, c.gate.w, c.up.w, this.xsPl, this.g]);
          }
        }
        gc.swiglu = gpu.grupo(this.gemma ? 'geglu' : 'swiglu', [gpu.uniforme([['u', c.gate.N]]), P, this.g, this.u]);
        gc.F = c.gate.N;
        gc.down = directo(c.down, this.g, c.postFfn);
      }
      return gc;
    });
    G.normFinal = gpu.grupo('rmsnorm', [gpu.uniforme([['u', D], ['u', 1], ['f', this.eps], ['u', 0]]), P, this.x, this.normFinal, this.xl]);
    G.salida = this._mm(this.salida, this.xl, this.logits, 0);
    G.argmax = gpu.grupo('argmax', [gpu.uniforme([['u', this.vocab]]), P, this.logits, this.bIds]);
    this.G = G;
  }

  reset() {
    this.pos = 0;   // the KV cache is overwritten by position (reference transformer.js:243-245)
    this.hist = [];
  }

  // Prompt cache: how many leading ids of a new prompt are already in the KV cache (pos is set there), or 0 (the
  // caller then resets).  The KV rows are written by position and depend only on the ids before them, so the
  // longest common prefix with the processed history stays valid and no state snapshot is needed (unlike the
  // reference's LFM2 convolution states).  The last id is always recomputed: its logits are the result.
  reutilizar(ids) {
    if (!this.cacheOn || !this.hist.length || this.pos !== this.hist.length) return 0;
    const h = this.hist, m = Math.min(h.length, ids.length - 1);
    let n = 0;
    while (n < m && h[n] === ids[n]) n++;
    // a ring of cap slots still holds the keys the recomputed positions need (from n + 1 - window on) only while
    // no later position has taken their slots: the history may not reach the first of them plus cap
    for (const c of this.capas) if (c.anillo && h.length > Math.max(0, n + 1 - c.swa) + c.anillo) n = 0;
    h.length = n;
    this.pos = n;
    return n;
  }

  // The reference engine saves recurrent-state checkpoints here; a KV cache needs none.
  guardarPunto() {}

  _despacharCapas(T) {
    const G = this.G, self = this;
    const mm = function (g, uno) {
      if (uno === undefined) uno = T === 1;
      if (!uno && g.baldosa && T >= 8) { despachar(null, g.baldosa, Math.ceil(g.filas / 64), 1, Math.ceil(T / 32)); return; }
      const xy = dim2(Math.ceil(g.filas / 8));
      despachar(null, uno ? g.uno : g.lote, xy[0], xy[1], uno ? 1 : Math.ceil(T / 4));
    };
    const filas = function (n) { return Math.ceil(T * n / 256); };
    despachar(null, G.embed, filas(this.D));
    if (G.escEmb) despachar(null, G.escEmb, filas(this.D));
    const salida = function (d) {
      mm(d.mm);
      if (!d.suma) return;
      if (d.norma) despachar(null, d.norma, T);
      despachar(null, d.suma, filas(self.D));
    };
    for (const gc of G.capas) {
      if (gc.attnNormPl && T >= 256) {
        despachar(null, gc.attnNormPl, Math.ceil(T / 8));
        mm(gc.wqPl); mm(gc.wkPl); mm(gc.wvPl);
      } else {
        despachar(null, gc.attnNorm, T);
        mm(gc.wq); mm(gc.wk); mm(gc.wv);
      }
      despachar(null, gc.ropeQ, this.nh, T);
      despachar(null, gc.ropeK, this.nkv, T);
      despachar(null, gc.kvw, Math.ceil(T * this.nkv * this.hd / 256));
      if (gc.attPl && T >= 256) {
        despachar(null, gc.attPl, this.nh, T);
        salida(gc.woPl);
      } else {
        despachar(null, gc.att, this.nh, T);
        salida(gc.wo);
      }
      const gluPl = !this.nExp && gc.gluPl && T >= 256;
      if (gluPl) despachar(null, gc.ffnNormPl, Math.ceil(T / 8));
      else despachar(null, gc.ffnNorm, T);
      if (this.nExp) {
        mm(gc.router);
        despachar(null, gc.topk, Math.ceil(T / 64));
        const gr = T >= 8 && gc.agrupado && this.agrupado;
        if (gr) despachar(null, gc.grupar, 1);
        const e = function (m) {
          if (gr) { despachar(null, m.gg, Math.ceil(m.filas / 64), self.nExp, Math.ceil(T / 32)); return; }
          const xy = dim2(Math.ceil(m.filas / 8));
          despachar(null, m.g, xy[0], xy[1], T * self.nUsados);
        };
        e(gc.eg); e(gc.eu);
        despachar(null, gc.eact, filas(this.nUsados * this.ffe));
        e(gc.ed);
        despachar(null, gc.comb, filas(this.D));
      } else {
        if (gc.glu && T >= 256) {
          despachar(null, gluPl ? gc.gluPl : gc.glu, Math.ceil(gc.F / 64), 1, Math.ceil(T / 32));
          salida(gc.downPl || gc.down);
        } else {
          mm(gc.gate); mm(gc.up);
          despachar(null, gc.swiglu, filas(gc.F));
          salida(gc.down);
        }
      }
    }
    return mm;
  }

  // Processes up to `batch` tokens from the current position; with conLogits returns the logits of the last
  // one (reference transformer.js:252-336).
  forward(ids, conLogits) {
    const T = ids.length;
    if (T < 1 || T > this.batch) return Promise.reject(new Error('invalid batch'));
    if (this.pos + T > this.ctx) return Promise.reject(new Error('context exceeded (' + this.ctx + ' tokens)'));
    for (const id of ids) if (!(id >= 0 && id < this.vocab)) return Promise.reject(new Error('token id ' + id + ' outside the vocabulary'));
    const gpu = this.gpu;
    gpu.escribir(this.bPaso, 0, new Uint32Array([T, this.pos, 0, 0]));
    gpu.escribir(this.bIds, 0, new Uint32Array(ids));
    const mm = this._despacharCapas(T);
    if (conLogits) {
      despachar(null, this.G.normFinal, 1);
      mm(this.G.salida, true);
    }
    this.pos += T;
    for (const id of ids) this.hist.push(id);
    if (!conLogits) return Promise.resolve(null);
    const out = new Float32Array(this.vocab);
    gpu.leer(this.logits, 0, out);
    // on the host, as the reference (transformer.js:333-334)
    if (this.escLogit) { const k = 1 / this.escLogit; for (let i = 0; i < out.length; i++) out[i] *= k; }
    if (this.softcap) { const c = this.softcap; for (let i = 0; i < out.length; i++) out[i] = c * Math.tanh(out[i] / c); }
    return Promise.resolve(out);
  }

  // ---------------------------------------------------------------- fused greedy decode
  _gemv(segs, x, norm, K, opts) {
    opts = opts || {};
    const gpu = this.gpu;
    const fmt = FMT_ID[segs[0].W.tipo];
    const u = [['u', segs.length], ['u', K], ['f', this.eps], ['u', opts.last ? 1 : 0], ['u', opts.R || 0],
      ['u', opts.maxWg || 0], ['u', fmt], ['u', 0]];
    const b = [this.bPaso, x, norm || null, opts.amax || null];
    for (const s of segs) {
      const f = FMT_ID[s.W.tipo];
      if (f !== fmt && !(MEZCLA.has(s.W.tipo) && MEZCLA.has(segs[0].W.tipo))) throw new Error('gemv segments must share one format');
      u.push(['u', s.mode | ((f !== fmt ? f : 0) << 8)], ['u', s.W.N], ['u', 0], ['u', s.W.N]);
      b.push(s.W.w, s.W2 ? s.W2.w : null, s.y);
    }
    return gpu.grupo('gemv', [gpu.uniforme(u)].concat(b));
  }

  // GEMV segments in as few launches as possible: K-quant formats (Q4_K, Q6_K) share one launch, any other
  // format gets its own.
  _gemvPorFormato(segs, x, norm, K) {
    const porFmt = new Map();
    for (const s of segs) {
      const clave = MEZCLA.has(s.W.tipo) ? 'kq' : s.W.tipo;
      if (!porFmt.has(clave)) porFmt.set(clave, []);
      porFmt.get(clave).push(s);
    }
    const out = [];
    for (const lista of porFmt.values()) out.push(this._gemv(lista, x, norm, K));
    return out;
  }

  // Whether the fused MoE decode ops take this layer: Q4_K/Q6_K experts with gate and up in one format, at most 256
  // experts to route, and inputs the kernels stage whole (D and kused * ffe at most 16384).
  _moeFusionable(c) {
    const kq = function (t) { return t === 'q4k' || t === 'q6k'; };
    return kq(c.eg.tipo) && c.eg.tipo === c.eu.tipo && kq(c.ed.tipo) && this.nExp <= 256 && this.nUsados <= 64 &&
      this.D <= 16384 && this.nUsados * this.ffe <= 16384 && this.ffe % 256 === 0 && this.D % 256 === 0;
  }

  // Whether dec_attn_block takes layer c: f16 cache, Q4_K q and k with Q4_K or Q6_K v, head_dim 64 or 128, 1, 2,
  // 4 or 8 KV heads and a multiple of 8 query heads (1, 2 or 4 per head group; 1 or 4 at head_dim 64), a model
  // width the GEMV stages whole (a multiple of 256, at most 8192).
  _bloqueAtt(c) {
    const gp = this.nh / 8;
    return this.bloqueAtt && this.kvF16 && c.wq.tipo === 'q4k' && c.wk.tipo === 'q4k' &&
      (c.wv.tipo === 'q4k' || c.wv.tipo === 'q6k') && (this.hd === 64 || this.hd === 128) &&
      [1, 2, 4, 8].indexOf(this.nkv) >= 0 && this.nh % 8 === 0 &&
      (gp === 1 || gp === 4 || (gp === 2 && this.hd === 128)) && this.D % 256 === 0 && this.D <= 8192;
  }

  // The sync words of the fused step's launches that share counters in one XCD's L2: the error word of
  // dec_attn_block (a barrier wait past its bound, or a head group seen on two XCDs), the merged attention's
  // counters and error word and the MoE router's (a grid column found on more than one XCD, or an arrival count
  // left over).  The decode results are then invalid.
  _comprobarBloque() {
    const e = new Uint32Array(1);
    if (this.usaBloque) {
      this.gpu.leer(this.syncBloque, 2112, e);
      if (e[0]) {
        throw new Error('dec_attn_block: ' + ((e[0] & 1) ? 'a barrier wait ran past its bound; ' : '') +
          ((e[0] & 2) ? 'a head group ran on more than one XCD; ' : '') + 'the decode results are invalid');
      }
    }
    if (this.usaMerged) {
      const w = new Uint32Array(8 * 32 + 1);
      this.gpu.leer(this.attCnt, 0, w);
      let resto = 0;
      for (let i = 0; i < 8; i++) resto |= w[32 * i];
      if (w[256] || resto) {
        this.gpu.escribir(this.attCnt, 0, new Uint8Array(8 * 128 + 128));   // the next launch starts clean
        throw new Error('dec_attn (merged): ' + (w[256] ? 'a column of workgroups ran on more than one XCD; ' : '') +
          (resto ? 'arrival counters left non-zero; ' : '') + 'the decode results are invalid');
      }
    }
    if (this.usaRouter) {
      const w = new Uint32Array(2);
      this.gpu.leer(this.routerCnt, 0, w);
      if (w[0] || w[1]) {
        this.gpu.escribir(this.routerCnt, 0, new Uint8Array(8));
        throw new Error('moe_router: ' + (w[1] ? 'its workgroups ran on more than one XCD; ' : '') +
          (w[0] ? 'arrival counter left non-zero; ' : '') + 'the routing is invalid');
      }
    }
  }

  _armarDecode() {
    const gpu = this.gpu, P = this.bPaso, D = this.D, qd = this.nh * this.hd, self = this;
    const plan = [];
    plan.push([this._embedGrupo(this.bIds, this.x), Math.ceil(D / 256)]);
    const uAtt = gpu.uniforme([['u', this.hd], ['u', this.nh], ['u', this.nkv], ['u', this.nsplit], ['f', this.escAtt],
      ['f', this.eps], ['f', this.base], ['u', 0], ['u', this.nrot], ['u', this.neox], ['u', this.kvF16 ? 1 : 0], ['u', this.ctx]]);
    const uComb = gpu.uniforme([['u', this.hd], ['u', this.nh], ['u', this.nsplit]]);
    const uAttM = gpu.uniforme([['u', this.hd], ['u', this.nh], ['u', this.nkv], ['u', this.nsplit], ['f', this.escAtt],
      ['f', this.eps], ['f', this.base], ['u', 0], ['u', this.nrot], ['u', this.neox], ['u', this.kvF16 ? 1 : 0], ['u', this.ctx],
      ['u', 1], ['u', this.gsplitAtt]]);
    this.usaBloque = this.usaMerged = this.usaRouter = false;
    for (let i = 0; i < this.capas.length; i++) {
      const c = this.capas[i], gc = this.G.capas[i];
      if (this._bloqueAtt(c)) {
        this.usaBloque = true;
        const uB = gpu.uniforme([['u', this.hd], ['u', this.nh], ['u', this.nkv], ['u', this.nsBloque], ['f', this.escAtt],
          ['f', this.eps], ['f', this.base], ['u', 0], ['u', this.nrot], ['u', this.neox], ['u', this.ctx], ['u', D],
          ['u', FMT_ID[c.wq.tipo]], ['u', FMT_ID[c.wk.tipo]], ['u', FMT_ID[c.wv.tipo]], ['u', 0]]);
        plan.push([gpu.grupo('dec_attn_block', [uB, P, this.x, c.attnNorm, c.wq.w, c.wk.w, c.wv.w, this.q, this.k, this.v,
          c.kc, c.vc, c.qNorm, c.kNorm, this.partOB, this.partMLB, this.ropeFreq, this.att, this.syncBloque]), 1]);
      } else {
      for (const g of this._gemvPorFormato([{ W: c.wq, mode: STORE, y: this.q }, { W: c.wk, mode: STORE, y: this.k },
        { W: c.wv, mode: STORE, y: this.v }], this.x, c.attnNorm, D)) plan.push([g, 1]);
      if (this.atencionUnida) {
        this.usaMerged = true;
        plan.push([gpu.grupo('dec_attn', [uAttM, P, this.q, this.k, this.v, c.kc, c.vc, c.qNorm, c.kNorm, this.partO,
          this.partML, this.ropeFreq, this.att, this.attCnt]), 1]);
      } else {
        plan.push([gpu.grupo('dec_attn', [uAtt, P, this.q, this.k, this.v, c.kc, c.vc, c.qNorm, c.kNorm, this.partO, this.partML,
          this.ropeFreq]), 1]);
        plan.push([gpu.grupo('dec_attn_comb', [uComb, P, this.partO, this.partML, this.att]), 1]);
      }
      }
      plan.push([this._gemv([{ W: c.wo, mode: ACC, y: this.x }], this.att, null, qd), 1]);
      if (this.nExp && this._moeFusionable(c)) {
        // routing, gate/up with SwiGLU, down and the weighted combine in two launches (the norm is fused in both
        // the router GEMV and the gate/up kernel)
        const K = this.nUsados, E = this.nExp;
        const u = function (n, k) {
          return gpu.uniforme([['u', n], ['u', k], ['u', E], ['u', K], ['f', self.eps], ['f', self.escExp],
            ['u', self.normExp ? 1 : 0]]);
        };
        if (this.enrutador && c.router.tipo === 'f32') {
          // the router GEMV and the routing in one launch (moe_router), so that the gate/up kernel reads the chosen
          // experts instead of routing in every workgroup
          this.usaRouter = true;
          plan.push([gpu.grupo('moe_router', [gpu.uniforme([['u', E], ['u', D], ['u', K], ['u', this.nwRouter], ['f', self.eps],
            ['f', self.escExp], ['u', self.normExp ? 1 : 0]]), P, c.router.w, this.x, c.ffnNorm, this.rl, this.sel, this.wts,
            this.routerCnt]), 1]);
          plan.push([gpu.grupo('moe_gate_up_' + c.eg.tipo, [gpu.uniforme([['u', this.ffe], ['u', D], ['u', E], ['u', K],
            ['f', self.eps], ['f', self.escExp], ['u', self.normExp ? 1 : 0], ['u', 1]]), P, c.eg.w, c.eu.w, this.x,
            c.ffnNorm, this.rl, this.g, this.sel, this.wts]), 1]);
        } else {
          // the router (E rows): one row per wavefront, so that the short tensor spreads over more workgroups
          plan.push([this._gemv([{ W: c.router, mode: STORE, y: this.rl }], this.x, c.ffnNorm, D, { R: 1 }), 1]);
          plan.push([gpu.grupo('moe_gate_up_' + c.eg.tipo, [u(this.ffe, D), P, c.eg.w, c.eu.w, this.x, c.ffnNorm, this.rl,
            this.g, this.sel, this.wts]), 1]);
        }
        plan.push([gpu.grupo('moe_down_' + c.ed.tipo, [u(D, this.ffe), P, c.ed.w, this.g, this.x, this.sel, this.wts]), 1]);
      } else if (this.nExp) {
        plan.push([gc.ffnNorm, 1]);
        plan.push([this._gemv([{ W: c.router, mode: STORE, y: this.rl }], this.xn, null, D), 1]);
        plan.push([gc.topk, 1]);
        const K = this.nUsados, E = this.nExp;
        const eg = c.eg, eu = c.eu, ed = c.ed;
        if (eg.tipo === eu.tipo) {
          const wb = plano(eg) ? [eg.qs, eg.ds] : [eg.w];
          plan.push([gpu.grupo('matmul_' + eg.tipo + '_e_swiglu', [gpu.uniforme([['u', this.ffe], ['u', D], ['u', 0], ['u', K], ['u', E]]),
            P].concat(wb, [eu.w, this.xn, this.g, this.sel])), [1, 1, K]]);
        } else {
          plan.push([gc.eg.g, [1, 1, K]]); plan.push([gc.eu.g, [1, 1, K]]); plan.push([gc.eact, Math.ceil(K * this.ffe / 256)]);
        }
        plan.push([gc.ed.g, [1, 1, K]]);
        plan.push([gc.comb, Math.ceil(D / 256)]);
      } else if (c.gate.tipo === c.up.tipo) {
        plan.push([this._gemv([{ W: c.gate, W2: c.up, mode: SWIGLU, y: this.g }], this.x, c.ffnNorm, D), 1]);
        plan.push([this._gemv([{ W: c.down, mode: ACC, y: this.x }], this.g, null, this.F), 1]);
      } else {
        for (const g of this._gemvPorFormato([{ W: c.gate, mode: STORE, y: this.g }, { W: c.up, mode: STORE, y: this.u }], this.x, c.ffnNorm, D)) plan.push([g, 1]);
        plan.push([gc.swiglu, Math.ceil(this.F / 256)]);
        plan.push([this._gemv([{ W: c.down, mode: ACC, y: this.x }], this.g, null, this.F), 1]);
      }
    }
    const S = this.salida;
    const rOut = S.tipo === 'q6k' ? 2 : 4;
    this.amaxWg = Math.min(AMAX_WG, Math.ceil(this.vocab / (4 * rOut)));
    plan.push([this._gemv([{ W: S, mode: ARGMAX, y: this.logits }], this.x, this.normFinal, D,
      { R: rOut, maxWg: this.amaxWg, amax: this.amax }), 1]);
    plan.push([gpu.grupo('argmax_fin', [gpu.uniforme([['u', this.amaxWg], ['u', 1], ['u', this.maxGen]]), P, this.amax, this.bIds,
      this.tokens, this.contador]), 1]);
    return plan;
  }

  _ejecutar(plan) {
    for (const it of plan) {
      const d = Array.isArray(it[1]) ? it[1] : [it[1], 1, 1];
      despachar(null, it[0], d[0], d[1], d[2]);
    }
  }

  // Builds and captures the fused one-token step.  Called from load(): the eager validation run writes KV slot 0
  // of every layer, which the first prefill overwrites.
  prepararDecode() {
    if (this.planDecode && (this.grafo || this.eagerDecode)) return;
    this.planDecode = this._armarDecode();
    const self = this;
    // one eager run validates every op's bindings before capture (a failed op inside a capture is harder to read)
    this.gpu.escribir(this.bPaso, 0, new Uint32Array([1, 0, 0, 0]));
    this.gpu.escribir(this.bIds, 0, new Uint32Array([0]));
    this.gpu.escribir(this.contador, 0, new Uint32Array([0, 0, 0, 0]));
    this._ejecutar(this.planDecode);
    this.gpu.sincronizar();
    if (!this.eagerDecode) this.grafo = this.gpu.capturar(function () { self._ejecutar(self.planDecode); });
  }

  // k one-token steps of the fused plan: graph replays, or the same ops dispatched one by one (eager_decode).
  _pasos(k) {
    if (this.eagerDecode) for (let i = 0; i < k; i++) this._ejecutar(this.planDecode);
    else this.gpu.reproducir(this.grafo, k);
  }

  // Greedy continuation on the device: `primero` is the token chosen from the last logits; runs `n` one-token
  // steps (each consumes the previous token and picks the next with the reference's argmax: strict '>', lowest
  // index on ties) and returns the n new token ids.  Positions advance by n.  With porPaso, each step's logits
  // are passed to porPaso(i, token, logits) (one readback per step, for checks).  With forzar (n - 1 ids, and
  // porPaso), step i > 0 consumes forzar[i - 1] instead of the token chosen at step i - 1 (teacher forcing for
  // checks): the same replays, with the step's input id written from the host; the returned ids are still the
  // device's choices.
  decodificarVoraz(primero, n, opciones) {
    opciones = opciones || {};
    if (n < 1) return [];
    if (n > this.maxGen) throw new Error('at most ' + this.maxGen + ' tokens per call');
    if (this.pos + n > this.ctx) throw new Error('context exceeded (' + this.ctx + ' tokens)');
    if (!(primero >= 0 && primero < this.vocab)) throw new Error('token id ' + primero + ' outside the vocabulary');
    this.prepararDecode();
    const gpu = this.gpu;
    gpu.escribir(this.bPaso, 0, new Uint32Array([1, this.pos, 0, 0]));
    gpu.escribir(this.bIds, 0, new Uint32Array([primero]));
    gpu.escribir(this.contador, 0, new Uint32Array([0, 0, 0, 0]));
    const forzar = opciones.forzar || null;
    if (forzar && (!opciones.porPaso || forzar.length < n - 1)) throw new Error('forzar needs porPaso and n - 1 ids');
    if (opciones.porPaso) {
      const lg = new Float32Array(this.vocab), t = new Uint32Array(1);
      for (let i = 0; i < n; i++) {
        if (forzar && i > 0) {
          if (!(forzar[i - 1] >= 0 && forzar[i - 1] < this.vocab)) throw new Error('forced id outside the vocabulary');
          gpu.escribir(this.bIds, 0, new Uint32Array([forzar[i - 1]]));
        }
        this._pasos(1);
        gpu.leer(this.logits, 0, lg);
        gpu.leer(this.bIds, 0, t);
        opciones.porPaso(i, t[0], lg);
      }
    } else if (opciones.tiempos) {
      const e0 = gpu.evento(), e1 = gpu.evento();
      gpu.marcar(e0);
      if (opciones.eager) for (let i = 0; i < n; i++) this._ejecutar(this.planDecode);   // same ops, no graph
      else this._pasos(n);
      gpu.marcar(e1);
      opciones.tiempos.ms = gpu.msEntre(e0, e1);
    } else {
      this._pasos(n);
    }
    const out = new Uint32Array(n);
    gpu.leer(this.tokens, 0, out);
    this._comprobarBloque();
    this.pos += n;
    this.hist.push(primero);                                    // the n processed ids: primero and out[0..n-2]
    for (let i = 0; i + 1 < n; i++) this.hist.push(forzar ? forzar[i] : out[i]);
    return Array.from(out);
  }

  // ---------------------------------------------------------------- sampled decode
  // One step of the fused plan from token `id` (a graph replay), then the next token chosen by the sampler `mu`
  // (sampling.js) with the history `historial`: when mu allows it, the penalties and the top-k candidates on the
  // device and only the draw on the host; otherwise, or when the candidates tie, from the whole logits on the
  // host, exactly as the reference.  The position advances by one.
  // control (checks): {mu: a second sampler with the same parameters and seed, penalizacion, distintos,
  // candidatos: counters}; the same logits are also read back and the host's choice made with control.mu, which
  // must agree bit for bit on the penalized logits and on the token.
  pasoMuestreado(id, mu, historial, control) {
    if (this.pos + 1 > this.ctx) throw new Error('context exceeded (' + this.ctx + ' tokens)');
    if (!(id >= 0 && id < this.vocab)) throw new Error('token id ' + id + ' outside the vocabulary');
    this.prepararDecode();
    const gpu = this.gpu;
    gpu.escribir(this.bPaso, 0, new Uint32Array([1, this.pos, 0, 0]));
    gpu.escribir(this.bIds, 0, new Uint32Array([id]));
    this._pasos(1);
    this._comprobarBloque();
    this.pos += 1;
    this.hist.push(id);
    const lg = new Float32Array(this.vocab);
    let ref = null;
    if (control) {
      gpu.leer(this.logits, 0, lg);
      ref = Float32Array.from(lg);
      control.mu.penalizar(ref, historial);
    }
    let t;
    if (mu.usaCandidatosDispositivo(this.vocab)) {
      this.penalizarDispositivo(mu, historial);
      if (control) {
        gpu.leer(this.logits, 0, lg);
        const a = new Uint32Array(lg.buffer), b = new Uint32Array(ref.buffer);
        for (let i = 0; i < a.length; i++) if (a[i] !== b[i]) { control.penalizacion++; break; }
      }
      const c = this.candidatosDispositivo(mu.topK);
      if (c) {
        if (control) control.candidatos++;
        t = mu.muestrear(c.ids, c.vals);
      } else {
        gpu.leer(this.logits, 0, lg);
        t = mu.elegirPenalizado(lg);
      }
    } else {
      gpu.leer(this.logits, 0, lg);
      t = mu.elegir(lg, historial);
    }
    if (control && control.mu.elegirPenalizado(ref) !== t) control.distintos++;
    return t;
  }

  // The sampler's penalties (sampling.js:27-37) applied to the logits buffer in place.
  penalizarDispositivo(mu, historial) {
    if (!historial || !historial.length || !mu.penaliza()) return;
    const pares = mu.conteos(historial);
    const d = new Float64Array([mu.rep, mu.freq, mu.pres]), w = new Uint32Array(d.buffer);
    const flat = new Uint32Array(2 * pares.length);
    pares.forEach(function (p, i) { flat[2 * i] = p[0] >>> 0; flat[2 * i + 1] = p[1]; });
    const gpu = this.gpu;
    gpu.escribir(this.penPares, 0, flat);
    despachar(null, gpu.grupo('penalizar', [gpu.uniforme([['u', pares.length], ['u', this.vocab], ['u', w[0]], ['u', w[1]],
      ['u', w[2]], ['u', w[3]], ['u', w[4]], ['u', w[5]]]), this.logits, this.penPares]), 1);
  }

  // The k largest logits {ids, vals} in descending order, or null when two of the k + 1 largest are equal (the
  // candidate set or order would then depend on the reference's heap) or a logit is NaN.
  candidatosDispositivo(k) {
    const gpu = this.gpu;
    despachar(null, gpu.grupo('topk_cand', [gpu.uniforme([['u', this.vocab], ['u', k]]), this.logits, this.candParte,
      this.candSalida]), 1);
    const o = new Uint32Array(2 + 2 * k);
    gpu.leer(this.candSalida, 0, o);
    if (o[0] !== 0) return null;
    const bits = new Uint32Array(k), ids = new Array(k);
    for (let i = 0; i < k; i++) { bits[i] = o[2 + 2 * i]; ids[i] = o[3 + 2 * i]; }
    return { ids: ids, vals: Float64Array.from(new Float32Array(bits.buffer)) };
  }

  // Greedy argmax of the current logits buffer on the device (same tie rule as the reference).
  argmaxDispositivo() {
    despachar(null, this.G.argmax, 1);
    const t = new Uint32Array(1);
    this.gpu.leer(this.bIds, 0, t);
    return t[0];
  }

  // The KV cache as this backend holds it, for checking against the CPU oracle: per layer the K cache bytes then
  // the V cache bytes ([ctx][kvd] f32 or f16 rows; the f16 V cache in its 32-slot tiles), written to `ruta`.
  volcarKV(ruta) {
    const fs = require('fs');
    const fd = fs.openSync(ruta, 'w');
    try {
      for (const c of this.capas)
        for (const b of [c.kc, c.vc]) {
          const u = new Uint8Array(b.size);
          this.gpu.leer(b, 0, u);
          fs.writeSync(fd, u);
        }
    } finally {
      fs.closeSync(fd);
    }
  }

  free() {
    if (this.grafo) { this.gpu.liberarGrafo(this.grafo); this.grafo = null; }
    const todos = this.bufs.concat(this.cargador ? this.cargador.buffers : []);
    this.gpu.liberar(todos);
    this.bufs = [];
  }
}

// RoPE frequencies base^(-2j/nrot) for j < nrot/2, each rounded once to float: the exponent is the float
// quotient of the reference's formula (gpu.js:436), the power is evaluated in double.
function tablaRope(base, nrot) {
  const t = new Float32Array(Math.max(1, nrot / 2));
  for (let j = 0; j < nrot / 2; j++) t[j] = Math.fround(Math.pow(base, Math.fround((-2 * j) / nrot)));
  return t;
}

function op_max_gen(meta) {
  const op = meta.options || {};
  return op.max_gen || 4096;
}

module.exports = { ModeloTransformer: ModeloTransformer, tablaRope: tablaRope, agrupable: agrupable };
