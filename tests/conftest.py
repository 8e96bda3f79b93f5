"""Test configuration: the `gpu` marker and import paths.

The package directory (gfx906-qwen3.8fn_amd/) is not an importable Python
package name, so its modules (moe_ffn, workloads) and the oracle binding are
put on sys.path here.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gfx906-qwen3.8fn_amd")
for p in (PKG, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests"), os.path.join(ROOT, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
