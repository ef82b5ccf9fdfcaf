"""Minimal GGUF v3 reader for the oracle (test infrastructure only; the product has its own C++ reader).

Follows the GGUF layout the reference's own golden fixture records
(engine/sllm-core/tests/fixtures/gguf_py_qwen3-0.6b-Q4_0.json: kv table, tensor table with ne = [K, N, ...], offsets
from an aligned data section). Tensors come back as numpy views of a memory map: F32 as float32 [..., ne1, ne0],
Q4_0 / Q8_0 / Q6_K as uint8 rows [..., ne1, row_bytes].
"""
from __future__ import annotations

import struct

import numpy as np

TYPES = {0: ("F32", 4, 1), 1: ("F16", 2, 1), 2: ("Q4_0", 18, 32), 8: ("Q8_0", 34, 32), 14: ("Q6_K", 210, 256)}
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}


class GGUF:
    def __init__(self, path: str):
        self.path = path
        self.mm = np.memmap(path, np.uint8, mode="r")
        buf = self.mm
        off = 0

        def rd(fmt):
            nonlocal off
            n = struct.calcsize(fmt)
            v = struct.unpack_from(fmt, buf, off)[0]
            off += n
            return v

        def rs():
            n = rd("<Q")
            nonlocal off
            s = bytes(buf[off:off + n]).decode()
            off += n
            return s

        assert rd("<I") == 0x46554747, "not a GGUF file"
        self.version = rd("<I")
        n_t, n_kv = rd("<Q"), rd("<Q")
        self.kv = {}
        for _ in range(n_kv):
            k = rs()
            t = rd("<I")
            if t == 8:
                self.kv[k] = rs()
            elif t == 9:
                it, n = rd("<I"), rd("<Q")
                if it == 8:
                    self.kv[k] = [rs() for _ in range(n)]
                else:
                    fmt = _SCALAR[it]
                    self.kv[k] = [rd(fmt) for _ in range(n)]
            else:
                self.kv[k] = rd(_SCALAR[t])
        self.alignment = int(self.kv.get("general.alignment", 32))
        self.tinfo = {}
        for _ in range(n_t):
            name = rs()
            nd = rd("<I")
            ne = [rd("<Q") for _ in range(nd)]
            t = rd("<I")
            o = rd("<Q")
            self.tinfo[name] = (ne, t, o)
        self.data_offset = (off + self.alignment - 1) // self.alignment * self.alignment

    def tensor(self, name: str) -> np.ndarray:
        ne, t, o = self.tinfo[name]
        tname, bsz, bk = TYPES[t]
        rows = int(np.prod(ne[1:])) if len(ne) > 1 else 1
        row_bytes = ne[0] // bk * bsz
        start = self.data_offset + o
        raw = self.mm[start:start + rows * row_bytes]
        shape = tuple(reversed(ne[1:]))
        if tname == "F32":
            return raw.view(np.float32).reshape(shape + (ne[0],))
        if tname == "F16":
            return raw.view(np.float16).reshape(shape + (ne[0],))
        return raw.reshape(shape + (row_bytes,))

    def type_name(self, name: str) -> str:
        return TYPES[self.tinfo[name][1]][0]
