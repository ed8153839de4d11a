"""A stand-in for quipullm's server on the engine side of its protocol, for testing the Node.js engine (motor.js).

Written from the protocol, not from the server's code: an engine says hello (POST /engine/api/hello), long-polls
GET /engine/api/next?motor=ID for jobs ({"accion": "nada"} when there is none, {"accion": "cerrar"} to make it stop),
posts events (POST /engine/api/event; a token event's reply may say {"cancelar": true}), and reads a job's model
from GET /engine/api/meta/<id> (the server's meta object: kv, tensors, data_start, ctx, overrides, arch_options,
options) and GET /engine/file/<id> (the GGUF file, with Range requests).  Jobs: {id, accion, params, prompt,
modelo: {id, arch, meta_url, archivo_url, ctx, bytes}}.
"""
from __future__ import annotations

import json
import os
import re
import sys
import threading
import urllib.parse
from collections import deque
from http.server import BaseHTTPRequestHandler, ThreadingHTTPServer

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def meta_object(model_id, path, ctx):
    """The server's meta object for the engine (its GGUF header in the engine's field names)."""
    from oracle.oracle import GGUF  # header reader
    g = GGUF(path)
    kv = {k: (v if not isinstance(v, (bytes, bytearray)) else v.decode("utf-8", "replace")) for k, v in g.kv.items()}
    tensors = [{"nombre": n, "dims": [int(d) for d in t["dims"]], "tipo": t["tipo"], "offset": int(t["offset"]),
                "bytes": t["bytes"], "tipo_nombre": t["tipo_nombre"], "abs": int(t["abs"])}
               for n, t in ((n, g.tensors[n]) for n in g.order)]
    return {"id": model_id, "kv": kv, "tensors": tensors, "data_start": int(g.data_start), "ctx": ctx, "overrides": {},
            "arch_options": {}, "options": {"tiled_prefill": True, "prompt_cache": True}}


class StubServer:
    """Threaded HTTP server on 127.0.0.1 (an ephemeral port).  models: id -> (GGUF path, ctx)."""

    def __init__(self, models, poll_s=1.0, close_when_idle=True):
        self.models = models
        self.poll_s = poll_s
        self.close_when_idle = close_when_idle
        self.cv = threading.Condition()
        self.pending = deque()
        self.jobs = {}           # id -> job dict
        self.events = {}         # job id -> [event]
        self.cancel_after = {}   # job id -> cancel when this many token events arrived
        self.state = []          # estado events
        self.hellos = []
        self.polls = 0
        self._meta = {}
        self._n = 0
        stub = self

        class H(BaseHTTPRequestHandler):
            def log_message(self, *a):
                pass

            def _json(self, code, obj):
                body = json.dumps(obj).encode()
                self.send_response(code)
                self.send_header("Content-Type", "application/json")
                self.send_header("Content-Length", str(len(body)))
                self.end_headers()
                self.wfile.write(body)

            def _body(self):
                n = int(self.headers.get("Content-Length") or 0)
                return json.loads(self.rfile.read(n) or b"{}")

            def do_GET(self):
                u = urllib.parse.urlparse(self.path)
                if u.path == "/engine/api/next":
                    return self._json(200, stub.next_job())
                if u.path.startswith("/engine/api/meta/"):
                    mid = urllib.parse.unquote(u.path[len("/engine/api/meta/"):])
                    if mid not in stub.models:
                        return self._json(404, {"error": "model not found"})
                    return self._json(200, stub.meta(mid))
                if u.path.startswith("/engine/file/"):
                    mid = urllib.parse.unquote(u.path[len("/engine/file/"):])
                    if mid not in stub.models:
                        return self._json(404, {"error": "model not found"})
                    return self._file(stub.models[mid][0])
                return self._json(404, {"error": "route not found"})

            def _file(self, path):
                size = os.path.getsize(path)
                ini, fin = 0, size - 1
                rng = self.headers.get("Range")
                if rng:
                    m = re.match(r"bytes=(\d+)-(\d+)$", rng)
                    if not m:
                        return self._json(416, {"error": "bad range"})
                    ini, fin = int(m.group(1)), min(int(m.group(2)), size - 1)
                n = fin - ini + 1
                self.send_response(206 if rng else 200)
                self.send_header("Content-Type", "application/octet-stream")
                self.send_header("Content-Length", str(n))
                self.end_headers()
                with open(path, "rb") as f:
                    f.seek(ini)
                    while n > 0:
                        chunk = f.read(min(n, 4 << 20))
                        self.wfile.write(chunk)
                        n -= len(chunk)

            def do_POST(self):
                u = urllib.parse.urlparse(self.path)
                d = self._body()
                if u.path == "/engine/api/hello":
                    stub.hellos.append(d)
                    return self._json(200, {"ok": True, "version": "stub"})
                if u.path == "/engine/api/event":
                    return self._json(200, stub.event(d))
                return self._json(404, {"error": "route not found"})

        self.httpd = ThreadingHTTPServer(("127.0.0.1", 0), H)
        self.url = "http://127.0.0.1:%d" % self.httpd.server_address[1]
        self.thread = threading.Thread(target=self.httpd.serve_forever, daemon=True)
        self.thread.start()

    def meta(self, mid):
        if mid not in self._meta:
            path, ctx = self.models[mid]
            self._meta[mid] = meta_object(mid, path, ctx)
        return self._meta[mid]

    def submit(self, accion, model_id, prompt="", params=None, cancel_after=None):
        with self.cv:
            self._n += 1
            jid = "t%03d" % self._n
            job = {"id": jid, "accion": accion, "params": params or {}, "prompt": prompt}
            if model_id:
                path, ctx = self.models[model_id]
                q = urllib.parse.quote(model_id)
                job["modelo"] = {"id": model_id, "arch": self.meta(model_id)["kv"]["general.architecture"],
                                 "meta_url": "/engine/api/meta/" + q, "archivo_url": "/engine/file/" + q, "ctx": ctx,
                                 "bytes": os.path.getsize(path)}
            self.jobs[jid] = job
            self.events[jid] = []
            if cancel_after:
                self.cancel_after[jid] = cancel_after
            self.pending.append(job)
            self.cv.notify_all()
        return jid

    def _done(self, jid):
        return any(e.get("tipo") in ("fin", "error") for e in self.events[jid])

    def next_job(self):
        with self.cv:
            self.polls += 1
            if not self.pending:
                self.cv.wait(self.poll_s)
            if self.pending:
                return self.pending.popleft()
            if self.close_when_idle and all(self._done(j) for j in self.jobs):
                return {"accion": "cerrar"}
            return {"accion": "nada"}

    def event(self, d):
        with self.cv:
            if d.get("tipo") == "estado":
                self.state.append(d)
                return {"ok": True}
            jid = d.get("id")
            if jid not in self.events:
                return {"cancelar": True}
            self.events[jid].append(d)
            self.cv.notify_all()
            if d.get("tipo") == "token" and jid in self.cancel_after:
                ntok = sum(1 for e in self.events[jid] if e.get("tipo") == "token")
                return {"cancelar": ntok >= self.cancel_after[jid]}
            return {"cancelar": False}

    def stop(self):
        self.httpd.shutdown()
        self.httpd.server_close()
