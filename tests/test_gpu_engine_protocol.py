"""The Node.js engine on quipullm's engine protocol with a real model on the GPU: `cli.js motor` against the stub
server (engine_stub.py), which serves a centered mini model's meta object and file (the engine loads the weights
by Range requests).  A greedy generation job's token events carry the oracle's greedy ids; a second job whose
prompt continues the first (prompt + 10 generated ids) reuses the cached prefix and continues the same sequence.
"""
import json
import os

import pytest

from conftest import ROOT, run
from engine_stub import StubServer
from quipullm_amd import build, synth

pytestmark = pytest.mark.gpu

CLI = os.path.join(ROOT, "quipullm_amd", "js", "cli.js")


def test_engine_protocol_generates_the_oracle_ids(oracle, models_dir):
    if not build.built() or not os.path.exists(build.NAPI):
        pytest.fail("native parts not built: run __graft_entry__.build() first")
    name = "mini_llama_q4km_c"
    path = synth.ensure_model(name, models_dir)
    vocab = synth.CONFIGS[name].vocab
    prompt = [int(t) for t in synth.random_prompt(vocab, 40, 1)]
    n = 24
    m = oracle.Model(path, ctx=256)
    want, _ = m.generate(prompt, n)
    m.close()
    stub = StubServer({"mini": (path, 256)}, poll_s=0.5)
    try:
        j1 = stub.submit("generar", "mini", " ".join(str(t) for t in prompt), {"temperature": 0, "max_tokens": n + 1})
        j2 = stub.submit("generar", "mini", "", {"temperature": 0, "max_tokens": 9, "prompt_ids": prompt + want[:10]})
        print("engine protocol: node cli.js motor", name, flush=True)
        rc, out, err = run(["timeout", "-k", "5", "150", "node", CLI, "motor", "--servidor", stub.url, "--kv", "f32",
                            "--batch", "32"], timeout=180)
    finally:
        stub.stop()
    assert rc == 0, err[-3000:]
    assert json.loads(out.strip().splitlines()[-1]) == {"fin": "cerrado"}
    assert "AMD" in stub.hellos[0]["gpu"]["summary"]
    e1 = stub.events[j1]
    got = [int(e["texto"]) for e in e1 if e["tipo"] == "token"]
    ini = [e for e in e1 if e["tipo"] == "inicio"]
    assert len(ini) == 1 and ini[0]["prompt_tokens"] == len(prompt)
    assert all(e["tipo"] == "progreso" for e in e1[:e1.index(ini[0])])  # model loading progress
    # the synthetic files declare the last id as the end token (tokenizer.ggml.eos_token_id): generation stops there
    eos = vocab - 1
    cut = want.index(eos) if eos in want else None
    want1 = want[:cut] if cut is not None else want
    assert got == want1, (got, want, [e["tipo"] for e in e1], e1[-1])
    f = e1[-1]
    assert f["tipo"] == "fin" and f["tps"] > 0
    if cut is None:
        assert f["razon"] == "length" and f["completion_tokens"] == n + 1
    else:
        assert f["razon"] == "stop" and f["completion_tokens"] == cut
    e2 = stub.events[j2]
    got2 = [int(e["texto"]) for e in e2 if e["tipo"] == "token"]
    want2 = want[10:18] if cut is None or cut >= 18 else want[10:cut]
    assert got2 == want2, (got2, want2, e2[-1])
    assert e2[-1]["diag"]["reutilizados"] >= len(prompt), e2[-1]["diag"]
