"""Device-memory helpers for the GPU tests (torch is used for allocation and streams only)."""
import ctypes as C

import numpy as np


def torch():
    import torch as T
    return T


def dev(a: np.ndarray):
    """A device copy of a numpy array (as a torch tensor of the same bytes)."""
    T = torch()
    a = np.ascontiguousarray(a)
    t = T.from_numpy(a.view(np.uint8).reshape(-1).copy()).to("cuda")
    return t


def k_pages(kpool: np.ndarray) -> np.ndarray:
    """A K pool given cell-major, [pages][KVH][cells][128] fp16 (the reference's layout, the oracle's input), in the
    library's layout: each (page, KV head) region holds its cells' dims in 16-byte chunks of 8, chunk-major
    ([16][cells][8]), so that chunk j of consecutive cells is contiguous."""
    P, KVH, pc, D = kpool.shape
    return np.ascontiguousarray(kpool.reshape(P, KVH, pc, D // 8, 8).transpose(0, 1, 3, 2, 4)).reshape(P, KVH, pc, D)


def k_cells(kdev: np.ndarray) -> np.ndarray:
    """The inverse of k_pages: a K pool read back from the library, cell-major."""
    P, KVH, pc, D = kdev.shape
    return np.ascontiguousarray(kdev.reshape(P, KVH, D // 8, pc, 8).transpose(0, 1, 3, 2, 4)).reshape(P, KVH, pc, D)


def empty(nbytes: int):
    T = torch()
    return T.zeros(max(int(nbytes), 256), dtype=T.uint8, device="cuda")


def host(t, dtype, shape=None):
    T = torch()
    T.cuda.synchronize()
    a = t.cpu().numpy().view(dtype)
    return a.reshape(shape) if shape is not None else a


def ptr(t):
    return C.c_void_p(t.data_ptr())


def stream():
    T = torch()
    return C.c_void_p(T.cuda.current_stream().cuda_stream)


def xa_decode(xa: np.ndarray, M: int, K: int):
    """The activation operand back to (q [M][K] as int, d [M][K/32] as float32): undoes the record layout (one 4864-byte
    record per 16-row tile and 4-block group: 4 fragments whose lane l = m + 16 g holds row m's elements 4g..4g+3 as q
    and 16+4g.. as q / 16, then the rows' scales and two corrections as fp32). Also checks every block's corrections
    against its integers: -(1032 * sum of q over elements 0..15 + 72 * sum over 16..31) and -1152 * sum of q."""
    nb = K // 32
    ng = (nb + 3) // 4
    mtp = (M + 31) // 32 * 2  # row tiles, rounded up to an even count
    mt = (M + 15) // 16
    rec = xa.view(np.uint8)[:mtp * ng * 4864].reshape(mtp, ng, 4864)[:mt]
    frag = rec[:, :, :4096].copy().view(np.float16).reshape(mt, ng, 4, 4, 16, 8).astype(np.float32)  # [mt][c][bb][g][m][j]
    dx = rec[:, :, 4096:4352].copy().view(np.float32).reshape(mt, ng, 4, 16)
    corr = rec[:, :, 4352:4608].copy().view(np.float32).reshape(mt, ng, 4, 16)
    corr8 = rec[:, :, 4608:4864].copy().view(np.float32).reshape(mt, ng, 4, 16)
    q = np.zeros((mt, 16, ng * 4, 32), np.float32)  # [mt][m][block][element]
    for g in range(4):
        for j in range(8):
            e = 4 * g + j if j < 4 else 16 + 4 * g + (j - 4)
            v = frag[:, :, :, g, :, j] * (1.0 if j < 4 else 16.0)  # [mt][c][bb][m]
            q[:, :, :, e] = v.transpose(0, 3, 1, 2).reshape(mt, 16, ng * 4)
    want_corr = -(1032.0 * q[..., :16].sum(-1) + 72.0 * q[..., 16:].sum(-1))  # [mt][m][block]
    got_corr = corr.transpose(0, 3, 1, 2).reshape(mt, 16, ng * 4)
    assert np.array_equal(got_corr, want_corr), "activation operand: a block's correction does not match its integers"
    got8 = corr8.transpose(0, 3, 1, 2).reshape(mt, 16, ng * 4)
    assert np.array_equal(got8, -1152.0 * q.sum(-1)), "activation operand: a block's Q8_0 correction is wrong"
    d = dx.transpose(0, 3, 1, 2).reshape(mt * 16, ng * 4)[:, :nb]
    return q.reshape(mt * 16, ng * 4 * 32)[:M, :K], d[:M]


def xa_values(xa: np.ndarray, M: int, K: int) -> np.ndarray:
    """The operand's values d * q as fp32 [M][K] (exact: fp16 d times an integer |q| <= 127)."""
    q, d = xa_decode(xa, M, K)
    return q * np.repeat(d, 32, axis=1)
