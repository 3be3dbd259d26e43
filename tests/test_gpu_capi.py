"""The C ABI from a non-Python host: locks-kv_amd/examples/capi_decode.cpp
(built next to the library) runs one decode step -- summary build, page
parameters, scores, top-b, fused split-K decode -- through include/locks_hip.h
only, and checks the output against a host fp32 attention over the pages the
selector returned."""
from __future__ import annotations

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                   "locks-kv_amd", "locks", "_lib", "capi_decode")


def test_c_abi_decode_step_from_cpp():
    assert os.path.isfile(EXE), f"{EXE} missing: run __graft_entry__.build()"
    print("[case] capi_decode", flush=True)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "capi ok" in r.stdout
