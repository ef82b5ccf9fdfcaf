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
    """The activation operand back to (q [M][K] as int, d [M][K/32] as float32): undoes the fragment lane layout."""
    nb = K // 32
    nbp = (nb + 3) // 4 * 4  # blocks per row tile (padded to whole 4-block groups)
    mtp = (M + 31) // 32 * 2  # row tiles, rounded up to an even count
    mt = (M + 15) // 16
    frag = xa.view(np.float16)[:mtp * nbp * 512].reshape(mtp, nbp, 4, 16, 8)[:mt, :nb]  # [mt][b][g][m][j]
    q = np.zeros((mt * 16, K), np.float32)
    for g in range(4):
        for j in range(8):
            e = 4 * g + j if j < 4 else 16 + 4 * g + (j - 4)
            q[:, e::32] = frag[:, :, g, :, j].astype(np.float32).transpose(0, 2, 1).reshape(mt * 16, nb)
    sc = xa.view(np.uint8)[mtp * nbp * 1024:mtp * nbp * 1056].view(np.float16).reshape(mtp, nbp, 16)[:mt, :nb]
    d = sc.astype(np.float32).transpose(0, 2, 1).reshape(mt * 16, nb)
    return q[:M], d[:M]


def xa_values(xa: np.ndarray, M: int, K: int) -> np.ndarray:
    """The operand's values d * q as fp32 [M][K] (exact: fp16 d times an integer |q| <= 127)."""
    q, d = xa_decode(xa, M, K)
    return q * np.repeat(d, 32, axis=1)
