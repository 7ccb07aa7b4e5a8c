"""The C ABI without torch on the GPU: ``tests/abi_smoke.cpp`` (built by
``flashslice_amd.build`` into ``tests/_bin/fs_abi_smoke``) is what a C or
C++ caller writes -- hipMalloc'd buffers, workspaces sized by
``fs_workspace_bytes``, its own stream -- running the slice and deslice
forward and the slice backward and checking every output against its own
double-precision loops (1e-5 relative). Run here as a child process."""

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_bin", "fs_abi_smoke")


def test_c_abi_without_torch():
    if not os.path.exists(BIN):
        pytest.fail("%s is not built: run `python -m flashslice_amd.build`" % BIN)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("OK")
