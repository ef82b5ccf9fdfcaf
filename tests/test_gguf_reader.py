"""The GGUF reader's checks on the CPU (no GPU: sn_check parses the file and the model's layout only). The reader is the
engine's replacement for the reference's gguf_open (core.h:15-199); a file it cannot trust is refused with a reason,
never mapped past its end."""
import ctypes as C
import struct

import pytest

import sllm_next as S


def gguf_bytes(kv=(), tensors=(), data=b"", alignment_pad=32, n_kv=None, n_t=None):
    """a GGUF v3 file: kv = [(key, type, packed value bytes)], tensors = [(name, ne list, type, offset)]"""
    out = struct.pack("<IIQQ", 0x46554747, 3, len(tensors) if n_t is None else n_t, len(kv) if n_kv is None else n_kv)
    for k, t, v in kv:
        out += struct.pack("<Q", len(k)) + k.encode() + struct.pack("<I", t) + v
    for name, ne, t, off in tensors:
        out += struct.pack("<Q", len(name)) + name.encode() + struct.pack("<I", len(ne))
        out += b"".join(struct.pack("<Q", e) for e in ne) + struct.pack("<IQ", t, off)
    out += b"\0" * ((-len(out)) % alignment_pad)
    return out + data


def check(tmp_path, blob):
    p = tmp_path / "m.gguf"
    p.write_bytes(blob)
    buf = C.create_string_buffer(512)
    rows = C.c_int()
    rc = S.lib().sn_check(str(p).encode(), C.byref(rows), buf, 512)
    return rc, buf.value.decode()


def arch():
    s = b"qwen3"
    return ("general.architecture", 8, struct.pack("<Q", len(s)) + s)


@pytest.mark.parametrize("a", [0, 3, 48, 1 << 21])
def test_bad_alignment_is_refused(tmp_path, a):
    rc, why = check(tmp_path, gguf_bytes([arch(), ("general.alignment", 4, struct.pack("<I", a))]))
    assert rc == -1 and "alignment" in why, why


def test_array_longer_than_the_file_is_refused(tmp_path):
    arr = struct.pack("<IQ", 6, (1 << 62) + 1)  # float array whose byte count wraps around 64 bits
    rc, why = check(tmp_path, gguf_bytes([arch(), ("tokenizer.ggml.scores", 9, arr)]))
    assert rc == -1 and "malformed" in why, why


def test_string_longer_than_the_file_is_refused(tmp_path):
    bad = ("general.name", 8, struct.pack("<Q", (1 << 64) - 8) + b"x")
    rc, why = check(tmp_path, gguf_bytes([arch(), bad]))
    assert rc == -1 and "malformed" in why, why


@pytest.mark.parametrize("ne,off", [([32, 1 << 40, 1 << 40], 0),  # rows overflow 64 bits
                                    ([32, 4], 1 << 63),              # offset far past the end
                                    ([32, 4], 64),                   # 72 bytes from 64 in a 96-byte section
                                    ([33, 1], 0),                    # not whole Q4_0 blocks
                                    ([0, 1], 0)])                    # an empty dimension
def test_tensor_outside_the_file_is_refused(tmp_path, ne, off):
    blob = gguf_bytes([arch()], [("token_embd.weight", ne, 2, off)], data=b"\0" * 96)
    rc, why = check(tmp_path, blob)
    assert rc == -1 and ("out of the file" in why or "malformed" in why), why


def test_a_well_formed_file_reaches_the_model_checks(tmp_path):
    """a small valid file passes the reader and is refused only for what it lacks as a model"""
    blob = gguf_bytes([arch(), ("general.alignment", 4, struct.pack("<I", 64))],
                      [("token_embd.weight", [32, 4], 0, 0)], data=b"\0" * 512, alignment_pad=64)
    rc, why = check(tmp_path, blob)
    assert rc == -1 and "GGUF" not in why and "out of the file" not in why, why
