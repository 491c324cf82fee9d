"""The C-ABI library loads and exports what include/nlgpu.h declares; its
kernel table agrees with the reference ABI the oracle restates; the CLI
hosts are built.  No GPU is used (nothing here initialises a device)."""
import ctypes
import os
import re

import nlg_oracle as orc
import nlgpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    txt = open(os.path.join(ROOT, "include", "nlgpu.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(nlg_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(nlgpu.LIB_PATH)
    names = declared_functions()
    assert len(names) > 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    nlgpu.lib()  # sets restype/argtypes for each; raises if a symbol is absent
    src = open(os.path.join(ROOT, "nelisp-gpu_amd", "nlgpu.py")).read()
    for n in declared_functions():
        assert f'"{n}"' in src, n


def test_kernel_table_matches_reference_abi():
    gpu = set(nlgpu.kernel_names())
    ref = set(orc.kernel_names())
    assert ref <= gpu and gpu - ref == {"ternary-i8"}
    for n in ref:
        assert nlgpu.kernel_abi(n) == orc.kernel_abi(n), n


def test_reference_kernel_abi_counts():
    # :buffers / :push lengths from lisp/nelisp-gpu-kernels.el
    expect = {"pack-act-rows": (3, 3), "ternary-rows": (5, 5), "bitlinear-dp4a-1f": (6, 3),
              "softmax": (2, 2), "silu-mul": (3, 1), "decode-attn-b": (5, 5), "rope-half": (2, 5),
              "attn-causal-gqa": (4, 4), "bitlinear-packed-v": (5, 5), "embed-gather": (3, 2)}
    for k, v in expect.items():
        assert nlgpu.kernel_abi(k) == v, k


def test_unknown_kernel_is_an_error_without_a_device():
    try:
        nlgpu.kernel_abi("no-such-kernel")
    except nlgpu.NlgError as e:
        assert "no-such-kernel" in str(e)
    else:
        raise AssertionError("expected NlgError")


def test_cli_hosts_are_built():
    for h in ("vkserver", "vkrun", "vkmatmul", "vksoftmax", "vkcompute"):
        p = os.path.join(nlgpu.BIN_DIR, h)
        assert os.path.isfile(p) and os.access(p, os.X_OK), p
