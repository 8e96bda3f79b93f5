"""Runs the compiled C++ caller of the C ABI (tests/abi_caller.cpp, built by
gfx906-qwen3.8fn_amd/Makefile into build/abi_caller): moe_ffn_create_tensors,
moe_router_select and moe_ffn_forward on a hipStream_t, outputs compared bit
for bit with the oracle's (tests/golden/abi_caller_case.bin, written by
tests/golden/make_abi_case.py).  The program prints one line per batch and
exits 0 only when the error word is 0 and ids, weights and y all match."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CALLER = os.path.join(ROOT, "gfx906-qwen3.8fn_amd", "build", "abi_caller")
CASE = os.path.join(ROOT, "tests", "golden", "abi_caller_case.bin")


def test_cpp_caller_router_and_forward_match_oracle():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert os.path.exists(CALLER), f"{CALLER} missing: run __graft_entry__.build()"
    print(f"\n[abi_caller] {CALLER} {CASE}", flush=True)
    r = subprocess.run([CALLER, CASE], capture_output=True, text=True, timeout=90)
    print(r.stdout + r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("PASS")
