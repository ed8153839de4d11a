"""End-to-end parity of the token loop on the GPU: the JavaScript engine (Node.js over the N-API addon) generates
greedily from seeded synthetic GGUF files and is compared with the CPU oracle on the same files.

Bars: the greedy ids are identical for every generated token, and the logits each token was chosen from
agree within 1e-3 relative (max |a - b| / max |b|).  Modes: "ref" is the reference op sequence (one op per
reference shader, host argmax), "fast" the captured one-token graph with fused kernels and the device argmax,
"engine" the engine's generation loop.  KV cache in f32 (the reference's) and f16 (checked against the oracle
with the same f16 rounding of the cache).

Node is started through the spawner of conftest.py, never from this (GPU-using) process.
"""
import ctypes
import json
import os

import numpy as np
import pytest

import refs
from conftest import ROOT, run
from quipullm_amd import build, synth

pytestmark = pytest.mark.gpu

CLI = os.path.join(ROOT, "quipullm_amd", "js", "cli.js")

MINI = ["mini_llama_q4km_c", "mini_llama_q5km_c", "mini_qwen3moe_q5k_c", "mini_llama_q3k_c", "mini_llama_q2k_c",
        "mini_llama_q8_c", "mini_qwen3_q4km_c", "mini_llama_iq4nl_c", "mini_qwen3moe_iq4nl_c",
        "mini_qwen3moe_q4k_c", "mini_llama_q4km",
        "mini_qwen3moe_q4k", "mini_llama_f16_c"]


@pytest.fixture(scope="module", autouse=True)
def native():
    if not build.built() or not os.path.exists(build.NAPI):
        pytest.fail("native parts not built: run __graft_entry__.build() first")


def rel(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def generate(path, prompt, n, mode, kv, tmp, extra=(), kv_out=None, ctx=256):
    pf = os.path.join(tmp, "prompt.json")
    lf = os.path.join(tmp, "logits.f32")
    with open(pf, "w") as f:
        json.dump([int(t) for t in prompt], f)
    if os.path.exists(lf):
        os.remove(lf)
    cmd = ["timeout", "-k", "5", "110", "node", CLI, "generate", "--model", path, "--prompt-file", pf, "--n", str(n),
           "--mode", mode, "--kv", kv, "--ctx", str(ctx)] + (["--logits-out", lf] if mode in ("fast", "ref") else []) + \
        (["--kv-out", kv_out] if kv_out else []) + list(extra)
    print("node generate", os.path.basename(path), mode, kv, flush=True)
    rc, out, err = run(cmd, timeout=120)
    assert rc == 0, err[-3000:]
    r = json.loads(out.strip().splitlines()[-1])
    lg = np.fromfile(lf, np.float32) if mode in ("fast", "ref") else None
    return r, lg


def oracle_run(oracle, path, prompt, n, kv_f16, kv_ref=None, ctx=256):
    m = oracle.Model(path, ctx=ctx, kv_f16=kv_f16)
    if kv_ref is not None:
        m.set_kv_reference(*kv_ref)
    ids, lgs = m.generate(prompt, n)
    m.close()
    return ids, lgs


read_kv_f16 = refs.read_kv_f16


@pytest.mark.parametrize("name", ["mini_llama_q4km_c", "mini_llama_q5km_c", "mini_llama_q3k_c", "mini_llama_q2k_c",
                                  "mini_llama_q8_c", "mini_qwen3_q4km_c",
                                  "mini_qwen3moe_q4k_c", "mini_qwen3moe_q5k_c", "mini_llama_iq4nl_c",
                                  "mini_qwen3moe_iq4nl_c", "mini_gemma3_q4km_c", "mini_llama_f16_c"])
@pytest.mark.parametrize("plen", [150, 300])
def test_long_prefill_on_matrix_cores_matches_oracle(oracle, models_dir, tmp_path, name, plen):
    """A 150- or 300-token prompt in one chunk runs the prefill matmuls on MFMA (bf16 hi/lo products; from 256
    tokens on the 256-token tiles and, for the dense K-quant models, gate, up and SwiGLU fused into one launch);
    the logits of the prompt's last token and the greedy continuation must still match the oracle."""
    path = synth.ensure_model(name, models_dir)
    vocab = oracle.GGUF(path).tensors["token_embd.weight"]["dims"][1]
    prompt = synth.random_prompt(vocab, plen, 2)
    n = 8
    ctx = 256 if plen + n <= 256 else 320
    want_ids, want_lg = oracle_run(oracle, path, prompt, n, False, ctx=ctx)
    r, lg = generate(path, prompt, n, "fast", "f32", str(tmp_path), ["--batch", str(plen + 10)], ctx=ctx)
    lg = lg.reshape(-1, vocab)
    errs = [rel(a, b) for a, b in zip(lg, want_lg)]
    assert r["ids"] == want_ids, (r["ids"], want_ids, errs)
    assert max(errs) < 1e-3, errs


@pytest.mark.parametrize("name", MINI)
@pytest.mark.parametrize("kv", ["f32", "f16"])
def test_greedy_matches_oracle(oracle, models_dir, tmp_path, name, kv):
    """Greedy ids identical to the oracle's, logits within 1e-3 relative at every step.  With the f16 cache the
    oracle is given the GPU's own f16 cache rows (downloaded after the run, the value cache converted from its
    32-slot tiles): each side rounds its own float32 K/V to f16, and an element near a rounding boundary would
    otherwise land one f16 step apart, a discrete difference of the two caches rather than of the arithmetic."""
    path = synth.ensure_model(name, models_dir)
    g = oracle.GGUF(path)
    vocab = g.tensors["token_embd.weight"]["dims"][1]
    prompt = synth.random_prompt(vocab, 40, 1)
    n = 24
    if kv == "f32":
        want_ids, want_lg = oracle_run(oracle, path, prompt, n, False)
    for mode in ("ref", "fast"):
        kvf = os.path.join(str(tmp_path), "kv.bin") if kv == "f16" else None
        r, lg = generate(path, prompt, n, mode, kv, str(tmp_path), kv_out=kvf)
        lg = lg.reshape(-1, vocab)
        assert len(lg) == n
        if kv == "f16":
            c = synth.CONFIGS[name]
            ref = read_kv_f16(kvf, c.n_layers, 256, c.nkv * c.hd, len(prompt) + n - 1)
            want_ids, want_lg = oracle_run(oracle, path, prompt, n, True, ref)
        errs = [rel(a, b) for a, b in zip(lg, want_lg)]
        assert r["ids"] == want_ids, (mode, r["ids"], want_ids, errs)
        over = [(i, "%.2e" % e) for i, e in enumerate(errs) if not e < 1e-3]
        assert not over, (mode, over)
        assert r["pos"] == len(prompt) + n - 1


@pytest.mark.parametrize("name", ["mini_llama_q4km_c", "mini_qwen3_q4km_c", "mini_qwen3moe_q4k_c"])
def test_attention_block_matches_oracle(oracle, models_dir, tmp_path, name):
    """The fused one-token step with dec_attn_block (--attn-block: Q/K/V, attention and the split merge of each
    layer in one launch) against the oracle as above (f16 cache, the oracle given the GPU's cache rows): ids
    identical, logits within 1e-3 relative at every step."""
    path = synth.ensure_model(name, models_dir)
    vocab = oracle.GGUF(path).tensors["token_embd.weight"]["dims"][1]
    prompt = synth.random_prompt(vocab, 40, 1)
    n = 24
    kvf = os.path.join(str(tmp_path), "kv.bin")
    r, lg = generate(path, prompt, n, "fast", "f16", str(tmp_path), extra=("--attn-block",), kv_out=kvf)
    lg = lg.reshape(-1, vocab)
    c = synth.CONFIGS[name]
    ref = read_kv_f16(kvf, c.n_layers, 256, c.nkv * c.hd, len(prompt) + n - 1)
    want_ids, want_lg = oracle_run(oracle, path, prompt, n, True, ref)
    errs = [rel(a, b) for a, b in zip(lg, want_lg)]
    assert r["ids"] == want_ids, (r["ids"], want_ids, errs)
    assert max(errs) < 1e-3, errs


def test_f16_cache_rows_are_the_rounded_values(oracle, models_dir, tmp_path):
    """The GPU's f16 cache rows of layer 0 (computed from the embeddings only, before any f16 cache value is
    used) are the f16 roundings of the oracle's float32 K and V of that layer: every element within one f16 step
    (the two sides' float32 values differ only in their last bits), nearly all equal.  (Deeper layers see the
    rounded cache of the layers before them, so their rows are not comparable element by element.)"""
    name = "mini_llama_q4km_c"
    path = synth.ensure_model(name, models_dir)
    vocab = oracle.GGUF(path).tensors["token_embd.weight"]["dims"][1]
    prompt = synth.random_prompt(vocab, 40, 1)
    kvf = os.path.join(str(tmp_path), "kv.bin")
    for mode in ("ref", "fast"):
        generate(path, prompt, 4, mode, "f16", str(tmp_path), kv_out=kvf)
        c = synth.CONFIGS[name]
        npos, kvd = len(prompt) + 3, c.nkv * c.hd
        k16, v16 = read_kv_f16(kvf, c.n_layers, 256, kvd, npos)
        m = oracle.Model(path, ctx=256, kv_f16=False)
        m.generate(prompt, 4)
        mm = oracle._Model.from_address(m.ptr)
        for name_, gpu, ptr in (("K", k16, mm.kc), ("V", v16, mm.vc)):
            ours = np.ctypeslib.as_array((ctypes.c_float * (c.n_layers * 256 * kvd)).from_address(ptr)).reshape(
                c.n_layers, 256, kvd)[0, :npos].astype(np.float16)
            g = gpu[0].view(np.float16)
            step = np.spacing(np.maximum(np.abs(ours), np.abs(g))).astype(np.float32)
            d = np.abs(ours.astype(np.float32) - g.astype(np.float32))
            assert np.all(d <= step), (mode, name_, float(np.max(d / step)))
            assert np.mean(d == 0) > 0.99, (mode, name_, float(np.mean(d == 0)))
        m.close()


def test_tiny_q8_config(oracle, models_dir, tmp_path):
    """The reference's CPU-runnable case: 8 layers, hidden 1024, 16 x 64 MHA, FFN 2816, vocab 32000, Q8_0; a
    32-token random prompt, then 128 greedy tokens, batch 1."""
    path = synth.ensure_model("tiny_q8", models_dir)
    prompt = synth.random_prompt(32000, 32, 2)
    want_ids, want_lg = oracle_run(oracle, path, prompt, 128, False)
    r, lg = generate(path, prompt, 128, "fast", "f32", str(tmp_path))
    lg = lg.reshape(-1, 32000)
    errs = [rel(a, b) for a, b in zip(lg, want_lg)]
    assert r["ids"] == want_ids
    assert max(errs) < 1e-3, max(errs)


def test_engine_loop_greedy_and_penalties(oracle, models_dir, tmp_path):
    """engine.generar: greedy on the device loop and on the host loop give the oracle's ids; with a repetition
    penalty the host sampler (penalties over the last 64 tokens of prompt + output) is followed."""
    path = synth.ensure_model("mini_llama_q4km_c", models_dir)
    vocab = oracle.GGUF(path).tensors["token_embd.weight"]["dims"][1]
    prompt = synth.random_prompt(vocab, 20, 5)
    n = 16
    want_ids, _ = oracle_run(oracle, path, prompt, n, False)
    for extra in ((), ("--host-loop",)):
        r, _ = generate(path, prompt, n, "engine", "f32", str(tmp_path), extra)
        assert r["ids"] == want_ids, extra
    # penalties: restated on the oracle's logits (sampling.js:25-42 of the reference)
    rp, fp, pp = 1.3, 0.2, 0.1
    m = oracle.Model(path, ctx=256)
    hist = list(prompt)
    lg = None
    for i in range(0, len(prompt), 32):
        lg = m.forward(prompt[i:i + 32], i + 32 >= len(prompt))
    out = []
    while len(out) < n:
        lg = lg.copy()
        counts = {}
        for t in hist[-64:]:
            counts[t] = counts.get(t, 0) + 1
        for t, c in counts.items():
            v = lg[t]
            v = v / rp if v > 0 else v * rp
            lg[t] = v - (c * fp + pp)
        t = oracle.argmax(lg)
        out.append(t)
        hist.append(t)
        if len(out) < n:
            lg = m.forward([t], True)
    m.close()
    r, _ = generate(path, prompt, n, "engine", "f32", str(tmp_path),
                    ("--repeat-penalty", str(rp), "--frequency-penalty", str(fp), "--presence-penalty", str(pp)))
    assert r["ids"] == out


def test_engine_rejects_bad_input(models_dir, tmp_path):
    path = synth.ensure_model("mini_llama_q8", models_dir)
    pf = os.path.join(str(tmp_path), "bad.json")
    for ids in ([800], [], [5] * 300):  # id outside the vocabulary (800), empty prompt, beyond the context (256)
        with open(pf, "w") as f:
            json.dump(ids, f)
        rc, out, err = run(["timeout", "-k", "5", "110", "node", CLI, "generate", "--model", path, "--prompt-file",
                            pf, "--n", "4", "--mode", "engine", "--ctx", "256"], timeout=120)
        assert rc == 1 and "error" in err, (ids, rc, err[-500:])


SAMPLER_PARAMS = [
    ["--temperature", "0.8", "--seed", "3"],                                    # the reference's defaults otherwise
    ["--temperature", "1.5", "--top-k", "128", "--top-p", "1", "--min-p", "0", "--seed", "4"],
    ["--temperature", "0.9", "--top-k", "20", "--repeat-penalty", "1.3", "--frequency-penalty", "0.2",
     "--presence-penalty", "0.1", "--seed", "5"],
    ["--temperature", "1.0", "--top-k", "0", "--seed", "6"],                   # all tokens: the host's path
    ["--temperature", "0", "--repeat-penalty", "1.5", "--seed", "7"],          # greedy with penalties: host path
]


@pytest.mark.parametrize("name", ["mini_llama_q4km_c", "mini_qwen3moe_q4k_c", "tiny_q8"])
@pytest.mark.parametrize("pi", range(len(SAMPLER_PARAMS)))
def test_sampled_decode_matches_host_sampler(models_dir, tmp_path, name, pi):
    """Stochastic decode on the fused one-token plan: penalties and top-k candidates on the device, the draw on the
    host.  Every token is also chosen on the host from the same logits by a second sampler with the same seed
    (the reference's procedure over the whole array): the penalized logits agree bit for bit and the chosen
    tokens are identical; the device candidates serve every step where the sampler allows them."""
    params = SAMPLER_PARAMS[pi]
    path = synth.ensure_model(name, models_dir)
    vocab = synth.CONFIGS[name].vocab
    prompt = synth.random_prompt(vocab, 12, 5 + pi)
    n = 40
    r, _ = generate(path, prompt, n, "sample", "f16", str(tmp_path), params)
    c = r["control"]
    assert len(r["ids"]) == n and all(0 <= t < vocab for t in r["ids"])
    assert c["distintos"] == 0 and c["penalizacion"] == 0, c
    device = "--top-k" not in params or params[params.index("--top-k") + 1] != "0"
    device = device and params[1] != "0"
    if device:
        assert c["candidatos"] >= n - 3, c     # a rare tie falls back to the host's heap
    else:
        assert c["candidatos"] == 0, c


def test_engine_sampling_is_seeded(models_dir, tmp_path):
    """engine.generar with a temperature runs the sampled device loop; the same seed gives the same tokens as the
    checked loop, another seed other tokens (temperature 100: the random-weight models' logits are too peaked
    for the draw to matter at ordinary temperatures)."""
    path = synth.ensure_model("mini_llama_q4km_c", models_dir)
    prompt = synth.random_prompt(1000, 12, 9)
    p = ["--temperature", "100", "--top-k", "64", "--top-p", "1", "--min-p", "0"]
    a, _ = generate(path, prompt, 30, "engine", "f16", str(tmp_path), p + ["--seed", "11"])
    b, _ = generate(path, prompt, 30, "sample", "f16", str(tmp_path), p + ["--seed", "11"])
    c, _ = generate(path, prompt, 30, "engine", "f16", str(tmp_path), p + ["--seed", "12"])
    assert a["ids"] == b["ids"]
    assert a["ids"] != c["ids"]


PROMPT_CACHE = r"""
const engine = require(%s);
(async () => {
  const p1 = %s, extra = %s, kv = %s;
  const m = await engine.cargarModelo(%s, {ctx: 256, options: {kv_f16: kv === 'f16'}});
  const a = await engine.generar(m, p1, {temperature: 0, max_tokens: 10});
  const p2 = p1.concat(a.ids, extra);
  const b = await engine.generar(m, p2, {temperature: 0, max_tokens: 10});
  const c = await engine.generar(m, p2, {temperature: 0, max_tokens: 10});
  const d = await engine.generar(m, p1.slice(0, 5).concat(extra), {temperature: 0, max_tokens: 10});
  m.free();
  const f = await engine.cargarModelo(%s, {ctx: 256, options: {kv_f16: kv === 'f16', prompt_cache: false}});
  const b2 = await engine.generar(f, p2, {temperature: 0, max_tokens: 10});
  const d2 = await engine.generar(f, p1.slice(0, 5).concat(extra), {temperature: 0, max_tokens: 10});
  f.free();
  console.log(JSON.stringify({a: a.ids, b: b.ids, c: c.ids, d: d.ids, b2: b2.ids, d2: d2.ids, p2: p2.length,
    rb: b.reutilizados, rc: c.reutilizados, rd: d.reutilizados, rb2: b2.reutilizados}));
})().catch((e) => { console.error(e.stack); process.exit(1); });
"""


def test_gemma3_windows_on_rings_match_oracle(oracle, models_dir, tmp_path):
    """Gemma 3 text (windows of 24 keys on the even layers, rings of 24 + 32 slots at batch 32): 40 prompt ids and
    24 greedy tokens, so the rings wrap; the reference loop and the engine loop against the oracle (f32 KV, as
    the reference keeps it), ids identical and logits within 1e-3 relative."""
    name = "mini_gemma3_q4km_c"
    path = synth.ensure_model(name, models_dir)
    vocab = synth.CONFIGS[name].vocab
    prompt = synth.random_prompt(vocab, 40, 4)
    n = 24
    want_ids, want_lg = oracle_run(oracle, path, prompt, n, False)
    r, lg = generate(path, prompt, n, "ref", "f32", str(tmp_path), ["--batch", "32"])
    lg = lg.reshape(-1, vocab)
    errs = [rel(a, b) for a, b in zip(lg, want_lg)]
    assert r["ids"] == want_ids, (r["ids"], want_ids, errs)
    assert max(errs) < 1e-3, errs
    r2, _ = generate(path, prompt, n, "engine", "f32", str(tmp_path), ["--batch", "32"])
    assert r2["ids"] == want_ids


@pytest.mark.parametrize("name,kv", [("mini_llama_q4km_c", "f16"), ("mini_qwen3moe_q4k_c", "f32")])
def test_prompt_cache_reuses_the_common_prefix(models_dir, name, kv):
    """A second request whose prompt extends the first request's prompt and answer computes only the new ids
    (the answer's last id was never processed, so it is recomputed); the same prompt again recomputes only its
    last id; a prompt sharing 5 ids reuses 5.  Greedy ids equal those of a model with the cache off."""
    path = synth.ensure_model(name, models_dir)
    p1 = synth.random_prompt(1000, 20, 21)
    extra = synth.random_prompt(1000, 7, 22)
    eng = os.path.join(ROOT, "quipullm_amd", "js", "engine.js")
    script = PROMPT_CACHE % (json.dumps(eng), json.dumps(p1), json.dumps(extra), json.dumps(kv), json.dumps(path),
                             json.dumps(path))
    print("node prompt cache", name, kv, flush=True)
    rc, out, err = run(["timeout", "-k", "5", "110", "node", "-e", script], timeout=120)
    assert rc == 0, err[-3000:]
    r = json.loads(out.strip().splitlines()[-1])
    assert r["rb"] == len(p1) + len(r["a"]) - 1
    assert r["rc"] == r["p2"] - 1
    assert r["rd"] == 5 and r["rb2"] == 0
    assert r["b"] == r["b2"] and r["c"] == r["b2"] and r["d"] == r["d2"]


@pytest.mark.parametrize("plen,rd", [(20, 5), (60, 0)])
def test_prompt_cache_on_rings(models_dir, plen, rd):
    """The prompt cache of a model with ring caches (gemma3: windows of 24, rings of 56 slots): a prefix is reused
    only while the ring still holds the window keys of the positions after it.  With a 20-id prompt every reuse
    stands (the history stays under 56 positions); with 60 ids, the 5-id prefix of the last request is refused
    (86 positions written since) and everything is recomputed.  Greedy ids equal those of the cache-off model."""
    path = synth.ensure_model("mini_gemma3_q4km_c", models_dir)
    p1 = synth.random_prompt(1000, plen, 21)
    extra = synth.random_prompt(1000, 7, 22)
    eng = os.path.join(ROOT, "quipullm_amd", "js", "engine.js")
    script = PROMPT_CACHE % (json.dumps(eng), json.dumps(p1), json.dumps(extra), json.dumps("f32"), json.dumps(path),
                             json.dumps(path))
    print("node prompt cache (rings)", plen, flush=True)
    rc, out, err = run(["timeout", "-k", "5", "110", "node", "-e", script], timeout=120)
    assert rc == 0, err[-3000:]
    r = json.loads(out.strip().splitlines()[-1])
    assert r["rb"] == len(p1) + len(r["a"]) - 1 and r["rc"] == r["p2"] - 1
    assert r["rd"] == rd and r["rb2"] == 0
    assert r["b"] == r["b2"] and r["c"] == r["b2"] and r["d"] == r["d2"]
