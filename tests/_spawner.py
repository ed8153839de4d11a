"""Runs commands on behalf of the test process.

The pytest process opens the GPU (through ctypes) for the op-level tests.  Programs such as the Node.js engine
are therefore not started from it: this helper is started before any GPU use and starts them instead, reading one
JSON request per line on stdin ({"cmd": [...], "timeout": s, "env": {...}}) and answering one JSON line
({"rc", "stdout", "stderr"}) on stdout.
"""
import json
import os
import subprocess
import sys


def main():
    for line in sys.stdin:
        req = json.loads(line)
        env = dict(os.environ)
        env.update(req.get("env") or {})
        try:
            r = subprocess.run(req["cmd"], capture_output=True, text=True, timeout=req.get("timeout", 300), env=env,
                               cwd=req.get("cwd"))
            out = {"rc": r.returncode, "stdout": r.stdout, "stderr": r.stderr}
        except subprocess.TimeoutExpired as e:
            out = {"rc": -9, "stdout": e.stdout or "", "stderr": (e.stderr or "") + "\ntimeout"}
        sys.stdout.write(json.dumps(out) + "\n")
        sys.stdout.flush()


if __name__ == "__main__":
    main()
