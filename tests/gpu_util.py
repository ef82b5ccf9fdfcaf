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


def xa_decode(xa: np.ndarray, M: int, K: int) -> np.ndarray:
    """The activation operand (hi + lo fp16 fragments) back to fp32 rows [M][K], undoing the lane layout."""
    nb = K // 32
    nbp = (nb + 3) // 4 * 4  # blocks per row tile (padded to whole 4-block groups)
    mt = (M + 15) // 16
    a = xa.view(np.float16)[:mt * nbp * 1024].reshape(mt, nbp, 2, 4, 16, 8)[:, :nb].astype(np.float32)
    v = a[:, :, 0] + a[:, :, 1]  # [mt][b][g][m][j]
    out = np.zeros((mt * 16, K), np.float32)
    for g in range(4):
        for j in range(8):
            e = 4 * g + j if j < 4 else 16 + 4 * g + (j - 4)
            # rows mt*16 + m, columns 32 b + e
            blockvals = v[:, :, g, :, j]  # [mt][b][m]
            out[:, e::32] = blockvals.transpose(0, 2, 1).reshape(mt * 16, nb)
    return out[:M]
