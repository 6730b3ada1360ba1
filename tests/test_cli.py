"""g4run's command line (host/cli.c), without a GPU: usage and option
errors exit with status 1 before any model is opened, as main() of
gemma4-4b/cpu-blas/main.c does."""
import os
import subprocess

import pytest

G4RUN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "gemma4.c_amd", "g4run")


def _run(*args):
    if not os.path.exists(G4RUN):
        pytest.skip("g4run is not built")
    return subprocess.run([G4RUN, *args], capture_output=True, text=True, timeout=60)


def test_usage():
    r = _run()
    assert r.returncode == 1 and "Usage:" in r.stderr and "--thinking-budget" in r.stderr


def test_option_errors():
    r = _run("m.gguf", "--bogus", "1")
    assert r.returncode == 1 and "unknown option --bogus" in r.stderr
    r = _run("m.gguf", "-p")
    assert r.returncode == 1 and "requires a value" in r.stderr
    r = _run("m.gguf", "--thinking-budget")
    assert r.returncode == 1 and "requires a value" in r.stderr


def test_missing_model():
    r = _run("/nonexistent/model.gguf", "-n", "1")
    assert r.returncode == 1 and "Error" in r.stderr
