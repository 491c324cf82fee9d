"""A protocol client for vkserver that encodes requests byte for byte as
lisp/nelisp-gpu-server.el does (opcodes :19-27, run2 :240-291, batch body
:300-331, upload paths :121-189, compile/run-compiled :358-389), so the
server is exercised exactly as the unchanged Emacs client would drive it.
Floats go over the wire as raw little-endian f32 (the Elisp encoder's output
for representable values).
"""
from __future__ import annotations

import os
import struct
import subprocess
import tempfile

import numpy as np

OP_RUN, OP_UPLOAD, OP_FREE, OP_BATCH, OP_COMPILE = 0, 1, 2, 3, 4
OP_RUN_COMPILED, OP_FREE_COMPILED, OP_WRITE_RESIDENT, OP_UPLOAD_FILE = 5, 6, 7, 8


def u32(n: int) -> bytes:
    return struct.pack("<I", int(n) & 0xFFFFFFFF)


def f32(vec) -> bytes:
    return np.ascontiguousarray(vec, dtype=np.float32).tobytes()


class ServerError(RuntimeError):
    pass


class Server:
    def __init__(self, binary: str, kdir: str | None = None, env=None):
        self.kdir = kdir or tempfile.mkdtemp(prefix="nlgpu-k")
        self.proc = subprocess.Popen([binary, self.kdir], stdin=subprocess.PIPE, stdout=subprocess.PIPE,
                                     stderr=subprocess.PIPE, env=env)
        self.stderr_lines = []
        # wait for "vkserver: ready" on stderr
        while True:
            line = self.proc.stderr.readline()
            if not line:
                raise ServerError(f"server exited: rc={self.proc.wait()}")
            self.stderr_lines.append(line.decode(errors="replace").rstrip())
            if b"ready" in line:
                break

    # -- transport (nelisp-gpu--server-xfer, server.el:112-119)
    def xfer(self, req: bytes, expected: int) -> bytes:
        self.proc.stdin.write(req)
        self.proc.stdin.flush()
        buf = b""
        while len(buf) < expected:
            chunk = self.proc.stdout.read(expected - len(buf))
            if not chunk:
                raise ServerError("vkserver died")
            buf += chunk
        return buf

    @staticmethod
    def status(buf: bytes) -> int:
        return struct.unpack_from("<I", buf, 0)[0]

    def close(self) -> int:
        try:
            self.proc.stdin.close()
        except Exception:
            pass
        rc = self.proc.wait(timeout=60)
        return rc

    # -- resident buffers
    def upload(self, vec) -> int:
        v = np.asarray(vec, np.float32)
        buf = self.xfer(u32(OP_UPLOAD) + u32(v.size) + f32(v), 8)
        if self.status(buf):
            raise ServerError("upload error")
        return struct.unpack_from("<I", buf, 4)[0]

    def upload_bytes(self, data: bytes) -> int:
        assert len(data) % 4 == 0
        buf = self.xfer(u32(OP_UPLOAD) + u32(len(data) // 4) + data, 8)
        if self.status(buf):
            raise ServerError("upload-bytes error")
        return struct.unpack_from("<I", buf, 4)[0]

    def upload_file_raw(self, path: str, offset: int, nbytes: int) -> tuple[int, int]:
        full = os.path.abspath(path).encode()
        req = (u32(OP_UPLOAD_FILE) + u32(len(full)) + full + u32(offset & 0xFFFFFFFF) + u32(offset >> 32)
               + u32(nbytes // 4))
        buf = self.xfer(req, 8)
        return struct.unpack("<II", buf)

    def upload_file(self, path: str, offset: int, nbytes: int) -> int:
        st, h = self.upload_file_raw(path, offset, nbytes)
        if st:
            raise ServerError(f"upload-file error ({path} +{offset}, {nbytes} bytes)")
        return h

    def free(self, h: int) -> int:
        return self.status(self.xfer(u32(OP_FREE) + u32(h), 4))

    def write_resident(self, h: int, vec) -> int:
        v = np.asarray(vec, np.float32)
        return self.status(self.xfer(u32(OP_WRITE_RESIDENT) + u32(h) + u32(v.size) + f32(v), 4))

    # -- single dispatch (run2, server.el:240-291)
    def run2_raw(self, name: str, descs, push, groups) -> tuple[int, list]:
        nm = name.encode()
        parts = [u32(OP_RUN), u32(len(nm)), nm, u32(len(descs))]
        inline, outsizes = [], []
        for d in descs:
            kind = d[0]
            if kind == "in":
                v = np.asarray(d[1], np.float32)
                parts += [u32(v.size), u32(0)]
                inline.append(v)
            elif kind == "res":
                parts += [u32(d[2]), u32(1), u32(d[1])]
            elif kind == "out":
                parts += [u32(d[1]), u32(2)]
                outsizes.append(d[1])
            elif kind == "inout":
                v = np.asarray(d[1], np.float32)
                parts += [u32(v.size), u32(3)]
                inline.append(v)
                outsizes.append(v.size)
        parts += [u32(len(push))] + [u32(p) for p in push] + [u32(groups)]
        parts += [f32(v) for v in inline]
        buf = self.xfer(b"".join(parts), 4 + 4 * sum(outsizes))
        return self.status(buf), self._decode(buf, outsizes)

    def run2(self, name, descs, push, groups):
        st, outs = self.run2_raw(name, descs, push, groups)
        if st:
            raise ServerError("vkserver run error")
        return outs

    # -- fused batch (batch-body, server.el:300-331)
    @staticmethod
    def batch_body(slots, disps) -> tuple[bytes, list]:
        parts, inline, outsizes = [u32(len(slots))], [], []
        for s in slots:
            kind = s[0]
            if kind == "in":
                v = np.asarray(s[1], np.float32)
                parts += [u32(0), u32(v.size)]
                inline.append(v)
            elif kind == "res":
                parts += [u32(1), u32(s[2]), u32(s[1])]
            elif kind == "tmp":
                parts += [u32(2), u32(s[1])]
            elif kind == "out":
                parts += [u32(3), u32(s[1])]
                outsizes.append(s[1])
        parts.append(u32(len(disps)))
        for name, slotidx, pushv, grp in disps:
            nm = name.encode()
            parts += [u32(len(nm)), nm, u32(len(slotidx))] + [u32(i) for i in slotidx]
            parts += [u32(len(pushv))] + [u32(p) for p in pushv] + [u32(grp)]
        parts += [f32(v) for v in inline]
        return b"".join(parts), outsizes

    def batch_raw(self, slots, disps) -> tuple[int, list]:
        body, outsizes = self.batch_body(slots, disps)
        buf = self.xfer(u32(OP_BATCH) + body, 4 + 4 * sum(outsizes))
        return self.status(buf), self._decode(buf, outsizes)

    def batch(self, slots, disps):
        st, outs = self.batch_raw(slots, disps)
        if st:
            raise ServerError("vkserver batch error")
        return outs

    def compile_raw(self, slots, disps) -> tuple[int, int, list]:
        body, outsizes = self.batch_body(slots, disps)
        buf = self.xfer(u32(OP_COMPILE) + body, 8)
        st, h = struct.unpack("<II", buf)
        return st, h, outsizes

    def run_compiled(self, h: int, outsizes) -> list:
        buf = self.xfer(u32(OP_RUN_COMPILED) + u32(h), 4 + 4 * sum(outsizes))
        if self.status(buf):
            raise ServerError("vkserver run-compiled error")
        return self._decode(buf, outsizes)

    def free_compiled(self, h: int) -> int:
        return self.status(self.xfer(u32(OP_FREE_COMPILED) + u32(h), 4))

    @staticmethod
    def _decode(buf: bytes, outsizes) -> list:
        res, off = [], 4
        for s in outsizes:
            res.append(np.frombuffer(buf, dtype="<f4", count=s, offset=off).copy())
            off += 4 * s
        return res
