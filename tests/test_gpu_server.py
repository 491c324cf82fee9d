"""vkserver on the MI355X, driven byte for byte as lisp/nelisp-gpu-server.el
drives the reference server: the reference's own ternary-kernel and
upload-file test flows (test/ternary-kernel-test.el, test/upload-file-test.el)
with their controls, the legacy inout run path, compiled batches with
write-resident, and every failure status the protocol defines."""
import os
import struct
import subprocess
import tempfile

import numpy as np
import pytest

import nlgpu
from nlg_client import OP_COMPILE, OP_RUN, Server, f32, u32

pytestmark = pytest.mark.gpu
SERVER = os.path.join(nlgpu.BIN_DIR, "vkserver")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ternary_rows_lcg.npz")


@pytest.fixture()
def srv():
    s = Server(SERVER)
    yield s
    s.close()


def test_ready_and_device_lines(srv):
    assert any("device =" in l for l in srv.stderr_lines)
    assert srv.stderr_lines[-1].endswith("ready")


def ternary_forward(srv, h, d, beta, bias=None):
    seq, out, cols, nblk, wng = (int(d[k]) for k in ("seq", "out", "cols", "nblk", "wng"))
    return srv.batch([("in", d["x"]), ("res", h, out * wng), ("in", d["bias"] if bias is None else bias),
                      ("in", beta), ("out", seq * out)],
                     [("ternary-rows", [0, 1, 2, 3, 4], [seq, out, cols, nblk, wng], (seq * out + 63) // 64)])[0]


def test_reference_ternary_kernel_flow(srv):
    d = np.load(GOLDEN)
    h = srv.upload_bytes(d["wp"].astype("<u4").tobytes())  # upload-bytes of tk-pack output
    y = ternary_forward(srv, h, d, d["beta"])
    want = d["y"]
    assert np.max(np.abs(y - want)) / np.max(np.abs(want)) < 1e-5
    assert np.any(y != 0)
    b2 = d["beta"].copy()
    b2[1] *= 3.0
    y1 = ternary_forward(srv, h, d, b2).reshape(3, 6)
    y0 = y.reshape(3, 6)
    assert np.all(y0[:, 0] != y1[:, 0]) and np.array_equal(y0[:, 1:], y1[:, 1:])
    assert srv.free(h) == 0


def readback(srv, h, n):
    # uft-readback: add2 against a zero vector (upload-file-test.el:21-27)
    return srv.batch([("res", h, n), ("in", np.zeros(n, np.float32)), ("out", n)],
                     [("add2", [0, 1, 2], [n], (n + 63) // 64)])[0]


def test_reference_upload_file_flow(srv, tmp_path):
    n, pad = 4096, 12
    vec = (3.0 * np.arange(n) - 5000.0).astype(np.float32)
    path = tmp_path / "uft.bin"
    path.write_bytes(b"\0" * (pad * 4) + vec.tobytes())
    h = srv.upload_file(str(path), pad * 4, n * 4)
    got = readback(srv, h, n)
    assert np.array_equal(got, vec) and np.any(got != 0)
    h2 = srv.upload_file(str(path), (pad + 1) * 4, (n - 1) * 4)
    g2 = readback(srv, h2, n - 1)
    assert not np.array_equal(g2, vec[:n - 1]) and np.array_equal(g2, vec[1:])
    srv.free(h2)
    h3 = srv.upload_bytes(path.read_bytes()[pad * 4:])
    assert np.array_equal(readback(srv, h3, n), got)
    srv.free(h3)
    half = n // 2
    h4 = srv.upload_file(str(path), (pad + half) * 4, half * 4)
    assert np.array_equal(readback(srv, h4, half), vec[half:])
    srv.free(h4)
    srv.free(h)


def test_upload_file_failures_keep_the_stream(srv, tmp_path):
    st, h = srv.upload_file_raw(str(tmp_path / "missing.bin"), 0, 16)
    assert (st, h) == (1, 0)
    p = tmp_path / "short.bin"
    p.write_bytes(b"\1" * 40)
    assert srv.upload_file_raw(str(p), 0, 400) == (1, 0)   # short read frees the slot
    assert srv.upload_file_raw(str(p), 8, 32) [0] == 0     # and the server goes on


def test_legacy_inout_run_and_resident_readback(srv):
    # nelisp-gpu-run through the server: every buffer inout, all returned
    a = np.linspace(-2, 2, 64 * 10).astype(np.float32)
    st, outs = srv.run2_raw("softmax", [("inout", a), ("inout", np.zeros_like(a))], [10, 64], 1)
    assert st == 0 and len(outs) == 2
    assert np.array_equal(outs[0], a)
    assert np.allclose(outs[1].reshape(10, 64).sum(1), 1.0, atol=1e-5)
    # nelisp-gpu-server-read-resident: scale-by-1 of a resident
    v = np.arange(100, dtype=np.float32) * 0.25
    h = srv.upload(v)
    got = srv.run2("scale", [("res", h, 100), ("in", np.array([1.0], np.float32)), ("out", 100)], [100], 2)[0]
    assert np.array_equal(got, v)


def test_raw_bits_survive_the_wire(srv):
    # NaN payloads and subnormals are copied, never canonicalised
    bits = np.array([0x7FC00001, 0xFFA00000, 0x00000001, 0x80000003, 0x7F7FFFFF, 0x3F800000], np.uint32)
    h = srv.upload(bits.view(np.float32))
    got = srv.run2("cache-append", [("res", h, 6), ("in", np.array([0.0], np.float32)), ("out", 6)], [6], 1)[0]
    assert np.array_equal(got.view(np.uint32), bits)


def test_compiled_batch_rezeros_and_sees_resident_writes(srv):
    n = 256
    x = srv.upload(np.ones(n, np.float32))
    # out <- out + x : with out re-zeroed on every run the result never accumulates
    st, h, outsizes = srv.compile_raw([("res", x, n), ("out", n), ("tmp", n)],
                                      [("add2", [0, 1, 1], [n], 4), ("add2", [1, 2, 2], [n], 4)])
    assert st == 0
    for _ in range(3):
        assert np.all(srv.run_compiled(h, outsizes)[0] == 1.0)
    assert srv.write_resident(x, np.full(n, 2.5, np.float32)) == 0
    assert np.all(srv.run_compiled(h, outsizes)[0] == 2.5)
    assert srv.write_resident(x, np.zeros(n + 1, np.float32)) == 1  # past the end
    assert srv.free_compiled(h) == 0
    assert srv.free_compiled(h) == 0  # already free: still 0


def test_failed_requests_reply_status_1_and_stay_in_sync(srv):
    # unknown kernel: status 1 plus the zeros the client waits for
    st, outs = srv.run2_raw("no-such-kernel", [("in", np.ones(8, np.float32)), ("out", 8)], [8], 1)
    assert st == 1 and np.all(outs[0] == 0)
    # short buffer for the push constants: rejected before launch
    st, outs = srv.batch_raw([("in", np.ones(10, np.float32)), ("out", 5)], [("softmax", [0, 1], [1, 10], 1)])
    assert st == 1 and np.all(outs[0] == 0)
    # bad resident handle
    st, outs = srv.run2_raw("scale", [("res", 999, 4), ("in", np.ones(1, np.float32)), ("out", 4)], [4], 1)
    assert st == 1
    # bad compiled handle: status alone, as the reference
    buf = srv.xfer(u32(5) + u32(15), 4)
    assert srv.status(buf) == 1
    # freeing nothing is fine
    assert srv.free(4000) == 0
    # and the server still works
    v = srv.run2("vadd", [("in", np.ones(4, np.float32)), ("in", np.ones(4, np.float32)), ("out", 4)], [4], 1)[0]
    assert np.all(v == 2)


def test_compiled_table_full_consumes_inline_data(srv):
    hs = []
    for _ in range(16):
        st, h, _ = srv.compile_raw([("in", np.ones(4, np.float32)), ("out", 4)], [("scale", [0, 0, 1], [4], 1)])
        assert st == 0
        hs.append(h)
    st, h, _ = srv.compile_raw([("in", np.ones(4, np.float32)), ("out", 4)], [("scale", [0, 0, 1], [4], 1)])
    assert (st, h) == (1, 0)
    for h in hs:
        srv.free_compiled(h)
    v = srv.run2("vadd", [("in", np.ones(4, np.float32)), ("in", np.ones(4, np.float32)), ("out", 4)], [4], 1)[0]
    assert np.all(v == 2)


def test_free_of_a_bound_resident_is_deferred(srv):
    n = 64
    x = srv.upload(np.full(n, 3.0, np.float32))
    st, h, outsizes = srv.compile_raw([("res", x, n), ("out", n)], [("add2", [0, 0, 1], [n], 1)])
    assert st == 0
    assert srv.free(x) == 0
    assert np.all(srv.run_compiled(h, outsizes)[0] == 6.0)  # still reads the old, live memory
    srv.free_compiled(h)


def _exit_code(payload: bytes) -> int:
    p = subprocess.run([SERVER, tempfile.gettempdir()], input=payload, capture_output=True, timeout=120)
    return p.returncode


def test_bad_opcode_exits_2_and_eof_exits_0():
    assert _exit_code(u32(9)) == 2
    assert _exit_code(b"") == 0
    assert _exit_code(u32(OP_RUN) + u32(4)) == 0      # EOF mid-request
    assert _exit_code(u32(OP_RUN) + u32(64)) == 2     # name too long
    assert _exit_code(u32(8) + u32(0)) == 0           # bad path length exits 0 (vkserver.c:374)


def test_many_residents_reuse_freed_slots(srv):
    hs = [srv.upload(np.ones(4, np.float32)) for _ in range(10)]
    assert hs == list(range(10))
    srv.free(3)
    assert srv.upload(np.ones(4, np.float32)) == 3  # first free slot
