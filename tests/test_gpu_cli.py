"""The CLI hosts that replace host/vkcompute.c, vkmatmul.c, vksoftmax.c and
vkrun.c: same arguments, output lines and exit codes, checked on the GPU."""
import os
import subprocess

import numpy as np
import pytest

import nlgpu

pytestmark = pytest.mark.gpu
BIN = nlgpu.BIN_DIR


def run(args, **kw):
    return subprocess.run([os.path.join(BIN, args[0])] + list(args[1:]), capture_output=True, text=True,
                          timeout=120, **kw)


def test_vkcompute():
    p = run(["vkcompute", "kernels/vadd.spv", "100000"])
    assert p.returncode == 0, p.stderr
    assert "PASS" in p.stdout and "c[last]=299997" in p.stdout


@pytest.mark.parametrize("variant", [[], ["naive"], ["tiled"], ["reg"]])
def test_vkmatmul(variant):
    p = run(["vkmatmul", "kernels/matmul.spv", "256", "256", "256"] + variant)
    assert p.returncode == 0, p.stderr
    assert "matmul 256x256 x 256x256" in p.stdout and "PASS" in p.stdout


def test_vksoftmax():
    p = run(["vksoftmax", "kernels/softmax.spv"])
    assert p.returncode == 0, p.stderr
    assert "softmax 64x256" in p.stdout and "PASS" in p.stdout and "row0_sum=1.00000" in p.stdout


def test_vkrun_round_trip(tmp_path):
    n = 1000
    a = np.arange(n, dtype=np.float32)
    b = 2 * a
    inp, out = tmp_path / "in.bin", tmp_path / "out.bin"
    (np.concatenate([a, b])).tofile(inp)  # C omitted: short file is zero-padded
    p = run(["vkrun", "name:vadd", str(inp), str(out), "64", str((n + 63) // 64), str(n), f"{n},{n},{n}"])
    assert p.returncode == 0, p.stderr
    o = np.fromfile(out, dtype=np.float32)
    assert o.size == 3 * n and np.array_equal(o[2 * n:], 3 * a) and np.array_equal(o[:n], a)
    # basename rule and NLG_KERNEL for a random temporary path
    p = run(["vkrun", "/tmp/kernels/vadd.spv", str(inp), str(out), "64", "16", str(n), f"{n},{n},{n}"])
    assert p.returncode == 0
    env = dict(os.environ, NLG_KERNEL="vadd")
    p = run(["vkrun", "/tmp/nlgpuXYZ.spv", str(inp), str(out), "64", "16", str(n), f"{n},{n},{n}"], env=env)
    assert p.returncode == 0
    p = run(["vkrun", "/tmp/nlgpuXYZ.spv", str(inp), str(out), "64", "16", str(n), f"{n},{n},{n}"])
    assert p.returncode == 2
    p = run(["vkrun", "x"])
    assert p.returncode == 1
