import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

_spawner = None


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_sessionstart(session):
    # started before any test can open the GPU; see _spawner.py
    global _spawner
    _spawner = subprocess.Popen([sys.executable, os.path.join(ROOT, "tests", "_spawner.py")], stdin=subprocess.PIPE,
                                stdout=subprocess.PIPE, text=True)


# One line per end-to-end parity case (steps compared, distinct ids, ties, errors), printed at the end of the run
# so that the short summary of a quiet run shows how much each case checked.
E2E_SUMMARY = []


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    if E2E_SUMMARY:
        terminalreporter.section("end-to-end parity")
        for line in E2E_SUMMARY:
            terminalreporter.write_line(line)


def pytest_sessionfinish(session, exitstatus):
    if _spawner is not None:
        _spawner.stdin.close()
        _spawner.wait(timeout=30)


def run(cmd, timeout=300, env=None):
    """Runs cmd through the spawner; returns (rc, stdout, stderr)."""
    _spawner.stdin.write(json.dumps({"cmd": cmd, "timeout": timeout, "env": env or {}}) + "\n")
    _spawner.stdin.flush()
    r = json.loads(_spawner.stdout.readline())
    return r["rc"], r["stdout"], r["stderr"]


@pytest.fixture(scope="session")
def models_dir():
    """The synthetic models' directory: bench.py's by default (QP_MODEL_DIR, else $TMPDIR/quipu_models), so that a
    test run and a benchmark on one machine write the models they share (the 8B and MoE shapes, ~22 GB) once."""
    d = (os.environ.get("QP_TEST_MODEL_DIR") or os.environ.get("QP_MODEL_DIR")
         or os.path.join(os.environ.get("TMPDIR") or "/tmp", "quipu_models"))
    os.makedirs(d, exist_ok=True)
    return d


@pytest.fixture(scope="session")
def quipu():
    from quipullm_amd import build, capi
    if not build.built():
        build.build_all()
    return capi.Quipu(0)


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.lib()
    return O
