"""pytest setup: the `gpu` marker and import paths.

GPU tests (marked `gpu`) run only on an MI355X box; everything else runs
on the CPU.  The product binding lives in nelisp-gpu_amd/nlgpu.py and the
CPU restatement (test infrastructure) in oracle/nlg_oracle.py.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("nelisp-gpu_amd", "oracle", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu on the GPU box)")
