"""The Node.js engine (quipullm_amd/js/motor.js) on quipullm's engine protocol, against the stub server of
engine_stub.py: hello, the long poll, generation / load / unload jobs and their events, cancellation from a token
event's reply, error events, and the stop on "cerrar".

On the CPU the model behind the plugin interface is a stand-in class (load reads one tensor from the file route
by a Range request; forward answers logits whose maximum is at (7 * last id + 3) mod vocab), so this checks the
protocol and the generation loop, not the arithmetic; test_gpu_engine_protocol.py runs a real model.
"""
import json
import os

import pytest

from conftest import ROOT, run
from engine_stub import StubServer
from quipullm_amd import synth

JS = os.path.join(ROOT, "quipullm_amd", "js")

FAKE_ENGINE = r"""
const { Motor } = require(%(motor)r);
const { rango } = require(%(http)r);
class Falso {
  constructor(meta) {
    this.meta = meta; this.ctx = meta.ctx; this.batch = 4; this.pos = 0;
    this.vocab = meta.tensors.find(function (t) { return t.nombre === 'token_embd.weight'; }).dims[1];
  }
  async load(fuente) {
    const t = this.meta.tensors.find(function (t) { return t.nombre === 'output_norm.weight'; });
    const b = await rango(fuente.url, t.abs, t.bytes);
    if (b.length !== t.bytes) throw new Error('short range');
    this.norm0 = b.readFloatLE(0);
  }
  reset() { this.pos = 0; }
  async forward(ids, want) {
    if (this.pos + ids.length > this.ctx) throw new Error('context exceeded');
    this.pos += ids.length;
    if (!want) return null;
    const lg = new Float32Array(this.vocab);
    lg[(ids[ids.length - 1] * 7 + 3) %% this.vocab] = 1;
    return lg;
  }
  free() {}
}
const cargas = [];
const m = new Motor({ servidor: %(url)r, info: { summary: 'cpu stand-in' }, espera: 50,
  cargar: async function (meta, fuente) { const f = new Falso(meta); await f.load(fuente); cargas.push([meta.id, f.norm0]); return f; } });
m.correr().then(function (r) { console.log(JSON.stringify({ r: r, cargas: cargas })); },
  function (e) { console.error(e.stack); process.exit(1); });
"""


def kinds(evs):
    return [e["tipo"] for e in evs]


def test_engine_protocol_against_stub(models_dir):
    path = synth.ensure_model("mini_llama_q8", models_dir)
    V = synth.CONFIGS["mini_llama_q8"].vocab
    stub = StubServer({"mini": (path, 64), "mini-b": (path, 64)}, poll_s=0.2)
    try:
        j1 = stub.submit("generar", "mini", "5 6 7", {"temperature": 0, "max_tokens": 6})
        j2 = stub.submit("generar", "mini", "", {"temperature": 0, "max_tokens": 10, "prompt_ids": list(range(1, 11))},
                         cancel_after=2)
        j3 = stub.submit("generar", "mini", "hello world", {"max_tokens": 3})
        j4 = stub.submit("generar", "mini", " ".join(["1"] * 70), {})
        j5 = stub.submit("cargar", "mini-b")
        j6 = stub.submit("descargar", None)
        script = FAKE_ENGINE % {"motor": os.path.join(JS, "motor.js"), "http": os.path.join(JS, "http.js"),
                                "url": stub.url}
        rc, out, err = run(["node", "-e", script], timeout=120)
    finally:
        stub.stop()
    assert rc == 0, err[-2000:]
    r = json.loads(out.strip().splitlines()[-1])
    assert r["r"] == "cerrado"
    # hello, then state reports
    h = stub.hellos[0]
    assert h["gpu"] == {"summary": "cpu stand-in"} and h["recarga"] is True and h["version"] and h["motor"]
    assert any(s.get("modelo_cargado") == "mini" and s.get("estado") == "listo" for s in stub.state)
    # the models: loaded for j1 (mini), again for j5 (mini-b), each reading its file by a range request
    assert [c[0] for c in r["cargas"]] == ["mini", "mini-b"]
    assert all(abs(c[1] - 1.0) < 0.2 for c in r["cargas"])  # output_norm is N(1, 0.02)
    # j1: inicio, 5 token events (the 6th token ends the generation by length: counted, its text not sent), fin
    want, t = [], 7
    for _ in range(6):
        t = (t * 7 + 3) % V
        want.append(t)
    e1 = stub.events[j1]
    assert kinds(e1) == ["inicio"] + ["token"] * 5 + ["fin"], kinds(e1)
    assert e1[0]["prompt_tokens"] == 3
    assert [int(e["texto"]) for e in e1[1:6]] == want[:5] and all(e["n"] == 1 for e in e1[1:6])
    f = e1[-1]
    assert f["razon"] == "length" and f["completion_tokens"] == 6 and f["prompt_tokens"] == 3
    assert f["ttft"] >= 0 and f["tps_prompt"] > 0 and set(f["diag"]) >= {"modelo_ms", "tok_ms", "lotes_ms"}
    # j2: 10 prompt ids in chunks of 4 with progress events; cancelled by the reply to its second token event
    e2 = stub.events[j2]
    prog = [e["fase"] for e in e2 if e["tipo"] == "progreso"]
    assert prog == ["procesando prompt 4/10", "procesando prompt 8/10", "procesando prompt 10/10"], prog
    assert sum(1 for e in e2 if e["tipo"] == "token") == 2
    assert e2[-1]["tipo"] == "fin" and e2[-1]["razon"] == "stop" and e2[-1]["completion_tokens"] == 2
    assert len(e2[-1]["diag"]["lotes_ms"]) == 3
    # j3: a text prompt the built-in tokenizer cannot read -> error 400; j4: prompt longer than the context
    assert kinds(stub.events[j3]) == ["error"] and stub.events[j3][0]["codigo"] == 400
    e4 = stub.events[j4]
    assert kinds(e4) == ["inicio", "error"] and e4[1]["codigo"] == 400 and "context" in e4[1]["mensaje"]
    # j5 / j6: load, unload
    assert kinds(stub.events[j5]) == ["fin"] and kinds(stub.events[j6]) == ["fin"]
    assert stub.state[-1].get("modelo_cargado") is None


def test_engine_retries_until_the_server_answers(tmp_path):
    """With no server listening the engine keeps retrying (the reference engine's loop); it is stopped from
    outside by its parar() callback."""
    script = r"""
const { Motor } = require(%r);
const t0 = Date.now();
let n = 0;
const m = new Motor({ servidor: 'http://127.0.0.1:9', info: { summary: 'x' }, espera: 20, log: function () { n++; } });
m.correr({ parar: function () { return Date.now() - t0 > 500; } }).then(function (r) { console.log(JSON.stringify({ r: r, logs: n })); });
""" % os.path.join(JS, "motor.js")
    rc, out, err = run(["node", "-e", script], timeout=60)
    assert rc == 0, err
    r = json.loads(out.strip().splitlines()[-1])
    assert r["r"] == "parado" and r["logs"] == 1  # one message for a run of failures


def test_range_read_stops_a_whole_file_answer(tmp_path):
    """rango() against a server that ignores Range and answers 200 with the whole file: the wanted bytes come back
    exact, and the transfer is stopped once they are in (the server gets to write only a small part of the 256 MB
    body instead of streaming it to the end)."""
    import http.server
    import threading
    size, chunk = 256 << 20, 1 << 16
    pat = bytes(range(256)) * (chunk // 256)
    sent = []

    class H(http.server.BaseHTTPRequestHandler):
        def log_message(self, *a):
            pass

        def do_GET(self):
            self.send_response(200)
            self.send_header("Content-Type", "application/octet-stream")
            self.send_header("Content-Length", str(size))
            self.end_headers()
            n = 0
            try:
                while n < size:
                    self.wfile.write(pat)
                    n += chunk
            except OSError:
                pass
            sent.append(n)

    srv = http.server.ThreadingHTTPServer(("127.0.0.1", 0), H)
    th = threading.Thread(target=srv.serve_forever, daemon=True)
    th.start()
    try:
        url = "http://127.0.0.1:%d/file" % srv.server_address[1]
        script = ("const { rango } = require(%r);\n"
                  "rango(%r, 1000, 5000).then(function (b) { console.log(JSON.stringify(Array.from(b))); },\n"
                  "  function (e) { console.error(e.stack); process.exit(1); });\n") % (os.path.join(JS, "http.js"), url)
        rc, out, err = run(["node", "-e", script], timeout=60)
        assert rc == 0, err[-2000:]
        got = json.loads(out.strip().splitlines()[-1])
        assert got == [(1000 + i) % 256 for i in range(5000)]
        for _ in range(100):
            if sent:
                break
            threading.Event().wait(0.05)
        assert sent and sent[0] < size // 4, sent
    finally:
        srv.shutdown()
