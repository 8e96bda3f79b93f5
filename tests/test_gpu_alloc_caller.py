"""Runs the compiled host-allocation check of the C ABI (tests/alloc_caller.cpp,
built by gfx906-qwen3.8fn_amd/Makefile into build/alloc_caller).  The program
replaces operator new and malloc for the whole process, attributes every
allocation to its call site, and after a warm-up repeats quantize, router,
forward (decode, grouped streaming and grouped MFMA batches), forward_q8,
combine and the quantized linear (with and without its workspace): none of
those calls may allocate from inside libmoe_ffn.so.  The reference counts
operator new the same way while its CPU jobs run (tests/cpu_expert_test.cpp:20-55)."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CALLER = os.path.join(ROOT, "gfx906-qwen3.8fn_amd", "build", "alloc_caller")


def test_abi_launch_paths_allocate_nothing_on_the_host():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert os.path.exists(CALLER), f"{CALLER} missing: run __graft_entry__.build()"
    print(f"\n[alloc_caller] {CALLER}", flush=True)
    r = subprocess.run([CALLER], capture_output=True, text=True, timeout=120)
    print(r.stdout + r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("PASS")
