"""CPU oracle for the fused quantized MoE expert path -- TEST INFRASTRUCTURE.

A ctypes/numpy front end over oracle/libtg_oracle.so, the scalar C
restatement of csrc/libtinygiant.c (see tg_oracle.c for the per-function
citations and how each function is pinned).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker / reported CPU baseline -- never as a
product path.
"""

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libtg_oracle.so"

Q8_DTYPE = np.dtype([("scale", "<f4"), ("sum", "<i4"), ("bsums", "<i4", (8,)), ("qs", "i1", (256,))])
assert Q8_DTYPE.itemsize == 296

FMT_Q4K, FMT_F16, FMT_Q6K, FMT_MXFP4, FMT_Q80 = 0, 1, 2, 3, 4
ACT_SILU, ACT_GPTOSS = 0, 1

VP, CI, CF = ctypes.c_void_p, ctypes.c_int, ctypes.c_float

_lib = None


def build():
    """Compiles libtg_oracle.so with its Makefile (gcc, no contraction)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.or_f16_to_f32.restype = CF
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_e8m0_half.restype = CF
        L.or_e8m0_half.argtypes = [ctypes.c_uint8]
        L.or_row_bytes.restype = ctypes.c_size_t
        L.or_row_bytes.argtypes = [CI, CI]
        L.or_quantize_q8.argtypes = [VP, VP, CI]
        for name in ("or_dot_q4k_q8", "or_dot_q6k_q8"):
            getattr(L, name).restype = CF
            getattr(L, name).argtypes = [VP, VP, CI]
        for name in ("or_dot_mxfp4_q8", "or_dot_q80_q8", "or_dot_f16"):
            getattr(L, name).restype = CF
            getattr(L, name).argtypes = [VP, VP, CI]
        for name in ("or_dot_q4k_q8_x4", "or_dot_q6k_q8_x4", "or_dot_mxfp4_q8_x4"):
            getattr(L, name).argtypes = [VP, VP, CI, VP]
        L.or_isums.restype = CI
        L.or_isums.argtypes = [CI, VP, VP, CI, VP]
        L.or_set_threads.argtypes = [CI]
        L.or_get_threads.restype = CI
        L.or_matmul.argtypes = [CI, VP, VP, VP, VP, CI, CI]
        L.or_matmul_q4k_scalar.argtypes = [VP, VP, VP, CI, CI]
        L.or_rms_norm.argtypes = [VP, VP, VP, CI, CF]
        L.or_moe_forward_rows_v2.argtypes = [VP, VP, VP, CI, VP, VP, VP, VP, CI, CI, VP, VP, VP, CI, CI, CI]
        L.or_moe_forward_rows_v2_ex.argtypes = [VP, VP, VP, CI, VP, VP, VP, VP, CI, CI, VP, VP, VP, CI, CI, CI,
                                                VP, VP]
        L.or_attention_v2.argtypes = [CI, CI, CI, CI, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, CI, CI,
                                      CI, VP, VP, VP, VP, CI, CI, CI, CI, CI, CF, VP]
        L.or_expert_forward.argtypes = [VP, VP, VP, CF, CI, CI]
        L.or_expert_forward_mixed.argtypes = [VP, VP, VP, CI, VP, VP, CF, CI, CI]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data if a is not None else None


def row_bytes(fmt, ncols):
    return lib().or_row_bytes(fmt, ncols)


def set_threads(n):
    lib().or_set_threads(int(n))


def f16_to_f32(h):
    return lib().or_f16_to_f32(int(h))


def e8m0_half(e):
    return lib().or_e8m0_half(int(e))


def quantize_q8(x):
    """x: float32 [ncols] or [rows, ncols] -> q8 blocks [rows, nb] (Q8_DTYPE)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    ncols = x2.shape[1]
    nb = (ncols + 255) // 256
    out = np.zeros((x2.shape[0], nb), Q8_DTYPE)
    for r in range(x2.shape[0]):
        lib().or_quantize_q8(x2[r].ctypes.data, out[r].ctypes.data, ncols)
    return out if x.ndim > 1 else out[0]


def dot(fmt, row, xq, ncols, xf=None):
    """One weight row (uint8 bytes) against one q8 row (or f32 row for F16)."""
    L = lib()
    row = np.ascontiguousarray(row, dtype=np.uint8)
    if fmt == FMT_Q4K:
        return L.or_dot_q4k_q8(row.ctypes.data, xq.ctypes.data, ncols // 256)
    if fmt == FMT_Q6K:
        return L.or_dot_q6k_q8(row.ctypes.data, xq.ctypes.data, ncols // 256)
    if fmt == FMT_MXFP4:
        return L.or_dot_mxfp4_q8(row.ctypes.data, xq.ctypes.data, ncols)
    if fmt == FMT_Q80:
        return L.or_dot_q80_q8(row.ctypes.data, xq.ctypes.data, ncols)
    xf = np.ascontiguousarray(xf, dtype=np.float32)
    return L.or_dot_f16(row.ctypes.data, xf.ctypes.data, ncols)


def dot_x4(fmt, row, xqs, ncols):
    """x4 kernels: one row against four q8 rows (list of 4 arrays)."""
    L = lib()
    row = np.ascontiguousarray(row, dtype=np.uint8)
    ptrs = (ctypes.c_void_p * 4)(*[x.ctypes.data for x in xqs])
    out = np.zeros(4, np.float32)
    if fmt == FMT_Q4K:
        L.or_dot_q4k_q8_x4(row.ctypes.data, ctypes.addressof(ptrs), ncols // 256, out.ctypes.data)
    elif fmt == FMT_Q6K:
        L.or_dot_q6k_q8_x4(row.ctypes.data, ctypes.addressof(ptrs), ncols // 256, out.ctypes.data)
    else:
        L.or_dot_mxfp4_q8_x4(row.ctypes.data, ctypes.addressof(ptrs), ncols, out.ctypes.data)
    return out


def isums_per_row(fmt, ncols):
    return {FMT_Q4K: ncols // 256 * 8, FMT_Q6K: ncols // 256 * 16}.get(fmt, ncols // 32)


def isums(fmt, mat, nrows, ncols, x):
    """Integer sub-block sums of every row of mat against q8(x): [nrows, nsums]."""
    mat = np.ascontiguousarray(mat, dtype=np.uint8).reshape(-1)
    xq = quantize_q8(np.asarray(x, np.float32))
    ns = isums_per_row(fmt, ncols)
    rb = row_bytes(fmt, ncols)
    out = np.zeros((nrows, ns), np.int32)
    for r in range(nrows):
        lib().or_isums(fmt, mat[r * rb:].ctypes.data, xq.ctypes.data, ncols, out[r].ctypes.data)
    return out


def matmul(fmt, mat, bias, x, nrows, ncols):
    mat = np.ascontiguousarray(mat, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(nrows, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().or_matmul(fmt, mat.ctypes.data, _p(b), x.ctypes.data, out.ctypes.data, nrows, ncols)
    return out


def matmul_q4k_scalar(mat, x, nrows, ncols):
    out = np.zeros(nrows, np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    mat = np.ascontiguousarray(mat, dtype=np.uint8)
    lib().or_matmul_q4k_scalar(mat.ctypes.data, x.ctypes.data, out.ctypes.data, nrows, ncols)
    return out


def attention_v2(fmts, w, b, q_norm_w, k_norm_w, sinks, kv_k, kv_v, kv_len, kv_max, window, rope_cos, rope_sin,
                 x, embed_dim, n_heads, n_kv_heads, head_dim, pos, eps):
    """tg_attention_v2 for one row (csrc/libtinygiant.c:939-983).  fmts and w
    hold (q, k, v, o); b the four biases or None; kv_k / kv_v are updated in
    place.  Returns (output [embed_dim], attention output [n_heads*head_dim])."""
    ws = [np.ascontiguousarray(m) for m in w]
    bs = [None if v is None else np.ascontiguousarray(v, np.float32) for v in (b or (None,) * 4)]
    opt = [None if v is None else np.ascontiguousarray(v, np.float32) for v in (q_norm_w, k_norm_w, sinks)]
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(embed_dim, np.float32)
    att = np.zeros(n_heads * head_dim, np.float32)
    rc = np.ascontiguousarray(rope_cos, np.float32)
    rs = np.ascontiguousarray(rope_sin, np.float32)
    assert kv_k.flags.c_contiguous and kv_v.flags.c_contiguous and kv_k.dtype == np.float32
    lib().or_attention_v2(*fmts, *[m.ctypes.data for m in ws], *[_p(v) for v in bs], *[_p(v) for v in opt],
                          kv_k.ctypes.data, kv_v.ctypes.data, kv_len, kv_max, window, rc.ctypes.data, rs.ctypes.data,
                          x.ctypes.data, out.ctypes.data, embed_dim, n_heads, n_kv_heads, head_dim, pos, eps,
                          att.ctypes.data)
    return out, att


def rms_norm(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros_like(x)
    lib().or_rms_norm(x.ctypes.data, w.ctypes.data, out.ctypes.data, x.shape[0], eps)
    return out


def _ptr_array(arrs):
    if arrs is None:
        return None, None
    keep = [None if a is None else np.ascontiguousarray(a) for a in arrs]
    arr = (ctypes.c_void_p * len(keep))(*[None if a is None else a.ctypes.data for a in keep])
    return arr, keep


def moe_v2(gates, ups, downs, gate_fmt, down_fmts, gbias, ubias, dbias, act, row_weights,
           inputs, output, inter_dim, hidden_in=None, hidden_out=None):
    """Reference tg_moe_forward_rows_v2 semantics; `output` [k, D] float32 is
    accumulated in place and returned.  hidden_out ([pairs, I] float32)
    receives phase A's hidden rows; hidden_in replaces them before phase B."""
    n = len(gates)
    k, D = inputs.shape
    gp, k1 = _ptr_array(gates)
    up, k2 = _ptr_array(ups)
    dp, k3 = _ptr_array(downs)
    gb, k4 = _ptr_array(gbias)
    ub, k5 = _ptr_array(ubias)
    db, k6 = _ptr_array(dbias)
    fm = np.ascontiguousarray(down_fmts, dtype=np.int32)
    rw = np.ascontiguousarray(row_weights, dtype=np.float32)
    x = np.ascontiguousarray(inputs, dtype=np.float32)
    assert output.dtype == np.float32 and output.flags.c_contiguous
    hin = None if hidden_in is None else np.ascontiguousarray(hidden_in, dtype=np.float32)
    if hidden_out is not None:
        assert hidden_out.dtype == np.float32 and hidden_out.flags.c_contiguous
    lib().or_moe_forward_rows_v2_ex(
        ctypes.addressof(gp), ctypes.addressof(up), ctypes.addressof(dp), gate_fmt, fm.ctypes.data,
        None if gb is None else ctypes.addressof(gb), None if ub is None else ctypes.addressof(ub),
        None if db is None else ctypes.addressof(db), act, n, rw.ctypes.data, x.ctypes.data,
        output.ctypes.data, k, D, inter_dim, _p(hin), _p(hidden_out))
    del k1, k2, k3, k4, k5, k6
    return output


def expert_forward_mixed(gate, up, down, down_format, x, output, weight, D, I):
    lib().or_expert_forward_mixed(_p(gate), _p(up), _p(down), down_format,
                                  np.ascontiguousarray(x, np.float32).ctypes.data,
                                  output.ctypes.data, weight, D, I)
    return output


def expert_forward(q4_data, x, output, weight, D, I):
    lib().or_expert_forward(_p(q4_data), np.ascontiguousarray(x, np.float32).ctypes.data,
                            output.ctypes.data, weight, D, I)
    return output


def route(router, bias, x, top_k, resident=None):
    """Restates Router.logits, _topk and _weights (tinygiant/router.py:29-42)
    for one normalized row x: float32 logits = router @ x (+ bias), the top_k
    experts by descending logit, and float32 softmax weights over the selected
    logits only.  Returns (logits, idx, weights).  With a resident mask (bool
    per expert) the selection is Router.select(restrict=True)
    (router.py:46-54): the top_k of the logits with the non-resident ones at
    -inf, weights from the unmasked logits of the selected experts; fewer than
    top_k resident experts fall back to the unrestricted top_k.

    Pinned by: a full sort of the logits on small inputs (selection and
    order), closed forms of the softmax (weights sum to 1, are decreasing
    with the logits, and equal for equal logits), and the restricted
    selection against a brute-force filter of the sorted logits, in
    tests/test_oracle_pins.py."""
    router = np.asarray(router, np.float32)
    logits = router @ np.asarray(x, np.float32)
    if bias is not None:
        logits = logits + np.asarray(bias, np.float32)
    sel_from = logits
    if resident is not None and int(np.count_nonzero(resident)) >= top_k:
        sel_from = np.where(np.asarray(resident, bool), logits, np.float32(-np.inf))
    idx = np.argpartition(sel_from, -top_k)[-top_k:]
    idx = idx[np.argsort(sel_from[idx])[::-1]]
    sel = logits[idx]
    e = np.exp(sel - sel.max())
    return logits, idx, (e / e.sum()).astype(np.float32)
