"""tinygiant_amd -- MI355X-native fused quantized MoE expert path.

The product is libtinygiant_hip.so (csrc/, include/tinygiant_hip.h): a C-ABI
drop-in for the reference's libtinygiant that runs the q8 quantizer, the
q4_K / q6_K / mxfp4 / q8_0 x q8 GEMVs and the top-k SwiGLU expert FFN with
its router-weighted combine as HIP kernels on gfx950.  This module loads it
and offers numpy-level wrappers with the reference's argument meaning
(tinygiant/engine.py:323-340 marshals the same way).
"""

import ctypes

import numpy as np

from ._lib import find_library, load_tinygiant_lib  # noqa: F401

FMT_Q4K, FMT_F16, FMT_Q6K, FMT_MXFP4, FMT_Q80 = 0, 1, 2, 3, 4
FMT_NAMES = {"q4_k": 0, "float16": 1, "q6_k": 2, "mxfp4": 3, "q8_0": 4}   # tinygiant/engine.py:21
ACT_SILU, ACT_GPTOSS = 0, 1
Q8_DTYPE = np.dtype([("scale", "<f4"), ("sum", "<i4"), ("bsums", "<i4", (8,)), ("qs", "i1", (256,))])

_LIB = None


def lib():
    """The loaded library (built in-tree); raises if it is not built."""
    global _LIB
    if _LIB is None:
        _LIB = load_tinygiant_lib()
    return _LIB


def last_error():
    return (lib().tg_hip_last_error() or b"").decode()


def row_bytes(fmt, ncols):
    return lib().tg_row_bytes(fmt, ncols)


def _ptrs(arrs):
    keep = [None if a is None else np.ascontiguousarray(a) for a in arrs]
    arr = (ctypes.c_void_p * max(1, len(keep)))(*[None if a is None else a.ctypes.data for a in keep])
    return arr, keep


def moe_forward_rows_v2(gates, ups, downs, gate_fmt, down_fmts, gbias, ubias, dbias, act,
                        row_weights, inputs, output, inter_dim, hidden_out=None, hq_out=None):
    """tg_moe_forward_rows_v2 on numpy arrays; `output` [k, D] is accumulated.
    With hidden_out ([pairs, I] f32) and hq_out ([pairs, nb] Q8_DTYPE) the
    call goes through tg_hip_moe_forward_stages and also returns the stages."""
    n = len(gates)
    k, D = inputs.shape
    gp, k1 = _ptrs(gates)
    up, k2 = _ptrs(ups)
    dp, k3 = _ptrs(downs)
    bias = []
    keep = [k1, k2, k3]
    for b in (gbias, ubias, dbias):
        if b is None:
            bias.append(None)
        else:
            arr, kk = _ptrs(b)
            keep.append(kk)
            bias.append(arr)
    fm = np.ascontiguousarray(down_fmts, dtype=np.int32)
    rw = np.ascontiguousarray(row_weights, dtype=np.float32)
    x = np.ascontiguousarray(inputs, dtype=np.float32)
    assert output.dtype == np.float32 and output.flags.c_contiguous and output.shape == (k, D)
    args = [ctypes.addressof(gp), ctypes.addressof(up), ctypes.addressof(dp), gate_fmt, fm.ctypes.data,
            *[None if b is None else ctypes.addressof(b) for b in bias],
            act, n, rw.ctypes.data, x.ctypes.data, output.ctypes.data, k, D, inter_dim]
    if hidden_out is None and hq_out is None:
        lib().tg_moe_forward_rows_v2(*args)
    else:
        lib().tg_hip_moe_forward_stages(*args, None if hidden_out is None else hidden_out.ctypes.data,
                                        None if hq_out is None else hq_out.ctypes.data)
    del keep
    return output


def matmul(fmt, mat, bias, x, nrows, ncols):
    mat = np.ascontiguousarray(mat)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(nrows, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().tg_matmul(fmt, mat.ctypes.data, None if b is None else b.ctypes.data, x.ctypes.data,
                    out.ctypes.data, nrows, ncols)
    return out


def quantize_q8(x):
    """GPU q8 quantization in the reference's 296-byte block layout."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    nb = (x2.shape[1] + 255) // 256
    out = np.zeros((x2.shape[0], nb), Q8_DTYPE)
    lib().tg_hip_quantize_q8(x2.ctypes.data, x2.shape[1], x2.shape[0], out.ctypes.data)
    return out if x.ndim > 1 else out[0]


def isums(fmt, mat, nrows, ncols, x):
    """GPU per-sub-block integer sums [nrows, nsums] of mat rows against q8(x)."""
    mat = np.ascontiguousarray(mat)
    x = np.ascontiguousarray(x, dtype=np.float32)
    ns = {FMT_Q4K: ncols // 256 * 8, FMT_Q6K: ncols // 256 * 16}.get(fmt, ncols // 32)
    out = np.zeros((nrows, ns), np.int32)
    r = lib().tg_hip_isums(fmt, mat.ctypes.data, nrows, ncols, x.ctypes.data, out.ctypes.data)
    if r < 0:
        raise RuntimeError(last_error())
    return out


def synth_host(kind, seed, nbytes):
    """Seeded synthetic tensor bytes (identical to the device fill)."""
    out = np.empty(nbytes, np.uint8)
    lib().tg_hip_synth_fill_host(kind, seed, out.ctypes.data, nbytes)
    return out


class DeviceArray:
    """A plain HBM allocation owned by the library (no torch involved)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = lib().tg_hip_malloc(self.nbytes)
        if not self.ptr:
            raise MemoryError(last_error())

    def upload(self, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        lib().tg_hip_memcpy_h2d(self.ptr + offset, arr.ctypes.data, arr.nbytes)

    def download(self, dtype, count, offset=0):
        out = np.empty(count, dtype)
        assert offset + out.nbytes <= self.nbytes
        lib().tg_hip_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes)
        return out

    def free(self):
        if self.ptr:
            lib().tg_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
