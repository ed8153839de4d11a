'use strict';
// Tokenizer interface of the engine (the methods quipullm's engine calls on its tokenizer: web/js/engine.js:235,
// 292-311): codificar(texto, {addBos}) -> ids, decodificadorIncremental() -> {agregar(id) -> text, terminar() ->
// text}, esFin(id).  Text tokenization (quipullm's tokenizer.js: BPE / SentencePiece from the GGUF vocabulary) is
// outside this backend; a real tokenizer plugs into motor.js through its crearTokenizador option.
//
// TokenizadorIds is the built-in stand-in: a prompt is the token ids written as decimal numbers separated by
// white space ("128000 9906 1917"), and a token's text is " <id>".  esFin follows the GGUF end-of-text ids
// (tokenizer.ggml.eos_token_id and eot_token_id), as the reference's does.

class TokenizadorIds {
  constructor(meta) {
    const kv = (meta && meta.kv) || {};
    const t = kv['tokenizer.ggml.tokens'];
    this.vocab = Array.isArray(t) ? t.length : null;   // the model's own size is checked by forward()
    this.fines = new Set();
    for (const k of ['tokenizer.ggml.eos_token_id', 'tokenizer.ggml.eot_token_id'])
      if (typeof kv[k] === 'number') this.fines.add(kv[k]);
    this.bos = typeof kv['tokenizer.ggml.bos_token_id'] === 'number' ? kv['tokenizer.ggml.bos_token_id'] : null;
  }

  codificar(texto, opciones) {
    const partes = String(texto).trim().split(/\s+/).filter(function (p) { return p.length; });
    const ids = partes.map(function (p) {
      if (!/^\d+$/.test(p)) {
        const e = new Error('this engine takes prompts as token ids (decimal numbers); got "' + p.slice(0, 20) + '"');
        e.codigo = 400;
        throw e;
      }
      return parseInt(p, 10);
    });
    if (opciones && opciones.addBos === true && this.bos !== null && ids[0] !== this.bos) ids.unshift(this.bos);
    return ids;
  }

  decodificadorIncremental() {
    return { agregar: function (id) { return ' ' + id; }, terminar: function () { return ''; } };
  }

  esFin(id) { return this.fines.has(id); }
}

module.exports = { TokenizadorIds: TokenizadorIds };
