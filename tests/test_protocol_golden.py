"""The vkserver protocol against hand-written request/response bytes
(tests/golden/protocol/session.txt, laid out from host/vkserver.c:11-38,
:274-615 and lisp/nelisp-gpu-server.el:240-389).

* CPU: the session file is self-consistent (every name or path length word
  equals the bytes that follow it) and the test client (tests/nlg_client.py)
  encodes the same requests to the same bytes, so the client is pinned by
  bytes written independently of it.
* GPU: the built server replays the whole session byte for byte -- every
  opcode, resident-slot reuse, compiled-graph re-runs after a resident is
  rewritten, file uploads (offset, missing file, short read), the
  failure statuses -- and exits with status 2 on an undefined opcode.
"""
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests", "golden", "protocol"))
import session  # noqa: E402

import nlg_client  # noqa: E402

SESSION = session.load()


def test_session_covers_every_opcode():
    ops = {struct.unpack_from("<I", e["req"])[0] for e in SESSION}
    assert set(range(9)) <= ops and 99 in ops
    assert SESSION[-1]["exit"] == 2 and all(e["exit"] is None for e in SESSION[:-1])


def test_length_words_match_the_bytes_that_follow():
    for e in SESSION:
        r = e["req"]
        op = struct.unpack_from("<I", r)[0]
        if op in (0, 8):  # RUN name / UPLOAD_FILE path: length word, then the text
            n = struct.unpack_from("<I", r, 4)[0]
            text = r[8:8 + n]
            assert text.replace(b"/", b"").replace(b"-", b"").replace(b".", b"").isalnum(), e["title"]
            assert len(r) >= 8 + n
        if op == 1:  # UPLOAD: nfloats words of data
            assert len(r) == 8 + 4 * struct.unpack_from("<I", r, 4)[0], e["title"]


class _Capture(nlg_client.Server):
    """The client's encoders without a process: requests are captured and
    answered with the golden responses."""

    def __init__(self):
        self.sent = []
        self.answers = []

    def xfer(self, req, expected):
        self.sent.append(req)
        ans = self.answers.pop(0)
        assert len(ans) == expected
        return ans


def test_client_encodes_the_golden_requests():
    c = _Capture()
    pick = {e["title"]: e for e in SESSION}

    def expect(title):
        e = pick[title]
        c.answers.append(e["resp"])
        return e

    e = expect("UPLOAD R0 = [1 2 3 4]")
    assert c.upload([1, 2, 3, 4]) == 0 and c.sent[-1] == e["req"]
    e = expect("RUN vadd: A resident R0, B inline, C out   (per buffer: size, kind[, handle])")
    out = c.run2("vadd", [("res", 0, 4), ("in", [10, 20, 30, 40]), ("out", 4)], [4], 1)
    assert c.sent[-1] == e["req"] and np.array_equal(out[0], [11, 22, 33, 44])
    e = expect("RUN mul: A inline, B resident R1, C inout (kind 3: read in, returned)")
    c.run2("mul", [("in", [2, 3, 4, 5]), ("res", 1, 4), ("inout", [9, 9, 9, 9])], [4], 1)
    assert c.sent[-1] == e["req"]
    e = expect("WRITE_RESIDENT R1 := [1 1 1 1]")
    assert c.write_resident(1, [1, 1, 1, 1]) == 0 and c.sent[-1] == e["req"]
    e = expect("FREE R0")
    assert c.free(0) == 0 and c.sent[-1] == e["req"]
    slots = [("in", [1, 2, 3, 4]), ("res", 1, 4), ("tmp", 4), ("out", 4)]
    disps = [("vadd", [0, 1, 2], [4], 1), ("mul", [2, 0, 3], [4], 1)]
    e = expect("BATCH: slots (kind, size[, handle]), vadd into a transient, then mul into an output")
    out = c.batch(slots, disps)
    assert c.sent[-1] == e["req"] and np.array_equal(out[0], [2, 6, 12, 20])
    e = expect("COMPILE the same graph with slot 0 = [2 2 2 2]")
    st, h, outsizes = c.compile_raw([("in", [2, 2, 2, 2])] + slots[1:], disps)
    assert (st, h) == (0, 0) and c.sent[-1] == e["req"]
    e = expect("RUN_COMPILED 0")
    assert np.array_equal(c.run_compiled(0, outsizes)[0], [6, 6, 6, 6]) and c.sent[-1] == e["req"]
    e = expect("FREE_COMPILED 0")
    assert c.free_compiled(0) == 0 and c.sent[-1] == e["req"]


@pytest.mark.gpu
def test_server_replays_the_golden_session():
    binary = os.path.join(ROOT, "nelisp-gpu_amd", "bin", "vkserver")
    p = subprocess.Popen([binary, "/nonexistent-kernel-dir"], stdin=subprocess.PIPE, stdout=subprocess.PIPE,
                         stderr=subprocess.PIPE, cwd=ROOT)
    try:
        while b"ready" not in (line := p.stderr.readline()):
            assert line, f"server exited before ready: {p.wait()}"
        for e in SESSION:
            print(f"[gpu] vkserver golden: {e['title']}", flush=True)
            p.stdin.write(e["req"])
            p.stdin.flush()
            if e["exit"] is not None:
                p.stdin.close()
                assert p.stdout.read() == b"", e["title"]
                assert p.wait(timeout=60) == e["exit"], e["title"]
                continue
            got = b""
            while len(got) < len(e["resp"]):
                chunk = p.stdout.read1(len(e["resp"]) - len(got))
                assert chunk, f"server closed during: {e['title']}"
                got += chunk
            assert got == e["resp"], f"{e['title']} (session line {e['line']}): {got.hex()} != {e['resp'].hex()}"
    finally:
        if p.poll() is None:
            p.kill()
            p.wait()
