"""Reader for the hand-written vkserver session files in this directory.

A session is a list of exchanges (title, request bytes, expected response
bytes, expected exit status or None); the file format is described at the
top of session.txt.  This turns the written-out words into bytes and
nothing more: it knows no opcode layout, so a layout misread in the
product's server or in the test client cannot leak into the expectations.
"""
from __future__ import annotations

import os
import shlex
import struct

HERE = os.path.dirname(os.path.abspath(__file__))


def _words(kind: str, args: list[str]) -> bytes:
    if kind == "u32":
        return b"".join(struct.pack("<I", int(a, 0)) for a in args)
    if kind == "f32":
        return b"".join(struct.pack("<f", float(a)) for a in args)
    if kind == "ascii":
        return " ".join(args).encode("ascii")
    raise ValueError(f"unknown line kind {kind!r}")


def load(name: str = "session.txt"):
    out = []
    cur = None
    for n, raw in enumerate(open(os.path.join(HERE, name)), 1):
        line = raw.split(";", 1)[0].rstrip()
        if not line.strip() or line.lstrip().startswith("#"):
            continue
        if line.startswith(">"):
            cur = {"title": line[1:].strip(), "req": b"", "resp": b"", "exit": None, "line": n}
            out.append(cur)
            section = "req"
        elif line.startswith("<"):
            section = "resp"
        elif line.startswith("!"):
            parts = line[1:].split()
            assert parts[0] == "exit", f"line {n}: {line}"
            cur["exit"] = int(parts[1])
        else:
            parts = shlex.split(line) if line.split()[0] == "ascii" else line.split()
            cur[section] += _words(parts[0], parts[1:])
    return out
