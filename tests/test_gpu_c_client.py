"""The C ABI driven from a plain C99 program (tests/c/srbcrs_c_client.c):
host and device CSR plans, run, tune, an error path, each checked against a
double-precision loop in the client itself."""
from __future__ import annotations

import subprocess

import pytest

pytestmark = pytest.mark.gpu


def test_c_client_runs(gpu, tmp_path):
    from tests.c_client import compile_client
    exe = compile_client(tmp_path / "client")
    print("[case] c client", exe, flush=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr + res.stdout
    assert "C-ABI OK" in res.stdout
