"""GPU parity of decode attention (tg_hip_attention_dev and the host-pointer
tg_attention_v2), against the oracle's restatement of tg_attention_v2
(csrc/libtinygiant.c:939-983).

Bars, stage by stage (the output projection re-quantizes the attention
output, so a last-bit difference there can flip one q8 rounding):
  K / V rows stored at kv_len     <= 2e-5 of max|row| (projection, norm, RoPE)
  attention output (pre-proj.)    <= 1e-4 of max (the scores, exponentials and
                                  sums are f32 in a chunked order)
  output from the GPU's own
  attention output                <= 1e-5 of max (q8 bit-exact, then the GEMV)
  end to end                      <= 1e-5 when no q8 rounding of the attention
                                  output flipped
  exact cases                     one position, a window of 1: the output is
                                  the new V row bit for bit
"""

import ctypes
import sys

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _rope_tables(kv_max, hd, base=10000.0):
    half = hd // 2
    ang = np.arange(kv_max)[:, None] / (base ** (np.arange(half)[None, :] * 2.0 / hd))
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def _case(seed, D, nh, nkv, hd, fmts, kv_max, kv_len, bias=False, norms=False, sinks=False, x_scale=1.0):
    """Synthetic weights, cache and input.  Without QK norm the synthetic
    projections make q and k large; x_scale keeps the scores in the range of
    a trained model (|score| of tens), where the softmax does not magnify
    last-bit differences of the projections beyond the bar."""
    import tinygiant_amd.synth as S
    rng = np.random.default_rng(seed)
    qd, kd = nh * hd, nkv * hd
    rows = (qd, kd, kd, D)
    cols = (D, D, D, qd)
    def mat(i):
        if fmts[i] == O.FMT_F16:   # finite halves (random bytes would hold Inf / NaN patterns)
            return (rng.standard_normal(rows[i] * cols[i]) * 0.05).astype(np.float16).view(np.uint8)
        return S.matrix_host(fmts[i], S.tensor_seed(seed, 1, i, 0), rows[i], cols[i])

    w = [mat(i) for i in range(4)]
    b = [(rng.standard_normal(n) * 0.1).astype(np.float32) for n in rows] if bias else [None] * 4
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norms else None
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norms else None
    sk = rng.standard_normal(nh).astype(np.float32) if sinks else None
    rc, rs = _rope_tables(kv_max, hd)
    kv_k = np.zeros((nkv, kv_max, hd), np.float32)
    kv_v = np.zeros((nkv, kv_max, hd), np.float32)
    kv_k[:, :kv_len] = rng.standard_normal((nkv, kv_len, hd))
    kv_v[:, :kv_len] = rng.standard_normal((nkv, kv_len, hd))
    x = (rng.standard_normal(D) * x_scale).astype(np.float32)
    return dict(fmts=fmts, w=w, b=b, qn=qn, kn=kn, sinks=sk, rc=rc, rs=rs, kv_k=kv_k, kv_v=kv_v, x=x, D=D, nh=nh,
                nkv=nkv, hd=hd, kv_max=kv_max, kv_len=kv_len)


def _oracle(orc, c, window):
    kk, vv = c["kv_k"].copy(), c["kv_v"].copy()
    out, att = orc.attention_v2(c["fmts"], c["w"], c["b"], c["qn"], c["kn"], c["sinks"], kk, vv, c["kv_len"],
                                c["kv_max"], window, c["rc"], c["rs"], c["x"], c["D"], c["nh"], c["nkv"], c["hd"],
                                c["kv_len"], 1e-6)
    return out, att, kk, vv


def _dev(tg, a):
    if a is None:
        return None
    d = tg.DeviceArray(a.nbytes)
    d.upload(np.ascontiguousarray(a))
    return d


def _gpu(tg, c, window):
    """tg_hip_attention_dev on device copies; returns output, attention output
    and the device caches read back."""
    lib = tg.lib()
    keep = []

    def dev(a):
        d = _dev(tg, a)
        keep.append(d)
        return d.ptr if d is not None else None

    w = [dev(m) for m in c["w"]]
    b = [dev(v) for v in c["b"]]
    qn, kn, sk = dev(c["qn"]), dev(c["kn"]), dev(c["sinks"])
    kk, vv = _dev(tg, c["kv_k"]), _dev(tg, c["kv_v"])
    keep += [kk, vv]
    rc, rs, x = dev(c["rc"]), dev(c["rs"]), dev(c["x"])
    out = tg.DeviceArray(c["D"] * 4)
    att = tg.DeviceArray(c["nh"] * c["hd"] * 4)
    sb = lib.tg_hip_attention_scratch_bytes(c["D"], c["nh"], c["nkv"], c["hd"], c["kv_max"])
    scr = tg.DeviceArray(sb)
    keep += [out, att, scr]
    lib.tg_hip_clear_error()
    lib.tg_hip_attention_dev(*c["fmts"], *w, *b, qn, kn, sk, kk.ptr, vv.ptr, c["kv_len"], c["kv_max"], window, rc, rs,
                             x, out.ptr, c["D"], c["nh"], c["nkv"], c["hd"], c["kv_len"], ctypes.c_float(1e-6),
                             att.ptr, scr.ptr, None)
    lib.tg_hip_synchronize()
    assert tg.last_error() == "", tg.last_error()
    r = (out.download(np.float32, c["D"]), att.download(np.float32, c["nh"] * c["hd"]),
         kk.download(np.float32, c["kv_k"].size).reshape(c["kv_k"].shape),
         vv.download(np.float32, c["kv_v"].size).reshape(c["kv_v"].shape))
    for a in keep:
        if a is not None:
            a.free()
    return r


def _rel(a, b):
    s = np.abs(b).max()
    return float(np.abs(a - b).max() / (s if s > 0 else 1.0))


def _check(orc, c, window, got, ref):
    out, att, kk, vv = got
    rout, ratt, rkk, rvv = ref
    L = c["kv_len"]
    assert _rel(kk[:, L], rkk[:, L]) <= 2e-5, ("k row", _rel(kk[:, L], rkk[:, L]))
    assert _rel(vv[:, L], rvv[:, L]) <= 2e-5, ("v row", _rel(vv[:, L], rvv[:, L]))
    # rows below kv_len are untouched
    assert np.array_equal(kk[:, :L], c["kv_k"][:, :L]) and np.array_equal(vv[:, :L], c["kv_v"][:, :L])
    assert _rel(att, ratt) <= 1e-4, ("attention", _rel(att, ratt))
    qd = c["nh"] * c["hd"]
    stage = orc.matmul(c["fmts"][3], c["w"][3], c["b"][3], att, c["D"], qd)
    assert _rel(out, stage) <= 1e-5, ("output from the GPU's attention", _rel(out, stage))
    if c["fmts"][3] != O.FMT_F16:
        flips = int(np.count_nonzero(orc.quantize_q8(att)["qs"] != orc.quantize_q8(ratt)["qs"]))
    else:
        flips = 0
    say(f"  attention rel {_rel(att, ratt):.2e}, output rel {_rel(out, rout):.2e}, q8 flips {flips}")
    if flips == 0:
        assert _rel(out, rout) <= 1e-5


Q4K, Q6K, Q80, F16 = O.FMT_Q4K, O.FMT_Q6K, O.FMT_Q80, O.FMT_F16


@pytest.mark.parametrize("kv_len", [0, 31, 300, 1023, 1500])
def test_attention_qwen3_shape(tg, orc, kv_len):
    """Qwen3-30B-A3B attention: D 2048, 32 query heads, 4 KV heads of 128,
    q4_K q/k/o, q6_K v, QK norm, no biases, full attention.  Spans up to 32
    chunks of 32 positions (1024 positions, kv_len 1023) combine inside the
    partial kernel; 1501 positions (47 chunks) take the separate combine
    kernel."""
    say("attention qwen3", kv_len)
    c = _case(10 + kv_len, 2048, 32, 4, 128, (Q4K, Q4K, Q6K, Q4K), max(512, kv_len + 1), kv_len, norms=True)
    got = _gpu(tg, c, 0)
    _check(orc, c, 0, got, _oracle(orc, c, 0))
    if kv_len == 0:
        # one position: each head's output is its KV head's new V row exactly
        _, att, _, vv = got
        for h in range(32):
            assert np.array_equal(att[h * 128:(h + 1) * 128], vv[h // 8, 0])


@pytest.mark.parametrize("kv_len", [300, 1500])
def test_attention_repeat_is_bit_identical(tg, kv_len):
    """The same call three times gives the same bits: the ticket counters of
    the folded combine are cleared by every call's projection launch, and no
    f32 result depends on which workgroup finishes last."""
    c = _case(80 + kv_len, 2048, 32, 4, 128, (Q4K, Q4K, Q6K, Q4K), kv_len + 1, kv_len, norms=True)
    runs = [_gpu(tg, c, 0) for _ in range(3)]
    for got in runs[1:]:
        for a, b in zip(got, runs[0]):
            assert a.tobytes() == b.tobytes()


@pytest.mark.parametrize("window,kv_len", [(128, 300), (0, 95), (1, 40)])
def test_attention_gptoss_shape(tg, orc, window, kv_len):
    """gpt-oss attention: D 2880, 64 query heads, 8 KV heads of 64, Q8_0
    projections with biases, per-head sinks, sliding window."""
    say("attention gpt-oss", window, kv_len)
    c = _case(20 + kv_len, 2880, 64, 8, 64, (Q80, Q80, Q80, Q80), 384, kv_len, bias=True, sinks=True, x_scale=0.02)
    got = _gpu(tg, c, window)
    _check(orc, c, window, got, _oracle(orc, c, window))
    if window == 1:
        _, att, _, vv = got
        # a window of 1 with a sink: weight exp(s - M) / (exp(s - M) + exp(sink - M)) on the new row only
        assert np.isfinite(att).all()


def test_attention_last_slot_and_f16(tg, orc):
    """kv_len = kv_max - 1 (the last cache slot), F16 projections, QK norm."""
    c = _case(30, 512, 8, 2, 64, (F16, F16, F16, F16), 70, 69, norms=True, bias=True)
    got = _gpu(tg, c, 0)
    _check(orc, c, 0, got, _oracle(orc, c, 0))


def test_attention_window_one_returns_new_v(tg, orc):
    """Without sinks, a window of 1 attends only the new row: the output is
    the stored V row bit for bit."""
    c = _case(40, 1024, 16, 4, 128, (Q4K, Q4K, Q4K, Q4K), 128, 77, norms=True)
    _, att, _, vv = _gpu(tg, c, 1)
    for h in range(16):
        assert np.array_equal(att[h * 128:(h + 1) * 128], vv[h // 4, 77])


def _host_call(tg, c, window, kv_k, kv_v, pos):
    lib = tg.lib()
    out = np.zeros(c["D"], np.float32)
    P = lambda a: None if a is None else a.ctypes.data  # noqa: E731
    lib.tg_hip_clear_error()
    lib.tg_attention_v2(*c["fmts"], *[m.ctypes.data for m in c["w"]], *[P(v) for v in c["b"]], P(c["qn"]),
                        P(c["kn"]), P(c["sinks"]), kv_k.ctypes.data, kv_v.ctypes.data, pos, c["kv_max"], window,
                        c["rc"].ctypes.data, c["rs"].ctypes.data, c["x"].ctypes.data, out.ctypes.data, c["D"],
                        c["nh"], c["nkv"], c["hd"], pos, ctypes.c_float(1e-6))
    assert tg.last_error() == "", tg.last_error()
    return out


def test_attention_v2_host_pointers_staged_equals_device(tg, orc):
    """The reference ABI on host arrays: the output equals the device entry
    point's bit for bit, and the new K/V rows land in the host cache."""
    c = _case(50, 2048, 32, 4, 128, (Q4K, Q4K, Q6K, Q4K), 256, 100, norms=True)
    dev_out, _, dkk, dvv = _gpu(tg, c, 0)
    kk, vv = c["kv_k"].copy(), c["kv_v"].copy()
    out = _host_call(tg, c, 0, kk, vv, 100)
    assert out.tobytes() == dev_out.tobytes()
    assert np.array_equal(kk, dkk) and np.array_equal(vv, dvv)


def test_attention_v2_registered_cache_two_steps(tg, orc):
    """Weights and KV arrays registered with tg_mlock: two consecutive
    positions, the second attending the first's row through the device copy;
    both match the oracle run in sequence."""
    c = _case(60, 1024, 16, 4, 64, (Q80, Q80, Q80, Q80), 96, 50, bias=True, sinks=True, x_scale=0.02)
    lib = tg.lib()
    kk, vv = c["kv_k"].copy(), c["kv_v"].copy()
    regs = [kk, vv] + list(c["w"])
    for a in regs:
        assert lib.tg_mlock(a.ctypes.data, a.nbytes) == 0
    try:
        out1 = _host_call(tg, c, 0, kk, vv, 50)
        c2 = dict(c)
        c2["x"] = (np.random.default_rng(61).standard_normal(c["D"]) * 0.02).astype(np.float32)
        out2 = _host_call(tg, c2, 0, kk, vv, 51)
    finally:
        for a in regs:
            lib.tg_hip_unregister(a.ctypes.data)
    ok, ov = c["kv_k"].copy(), c["kv_v"].copy()
    r1, _ = orc.attention_v2(c["fmts"], c["w"], c["b"], c["qn"], c["kn"], c["sinks"], ok, ov, 50, 96, 0, c["rc"],
                             c["rs"], c["x"], c["D"], c["nh"], c["nkv"], c["hd"], 50, 1e-6)
    r2, _ = orc.attention_v2(c["fmts"], c["w"], c["b"], c["qn"], c["kn"], c["sinks"], ok, ov, 51, 96, 0, c["rc"],
                             c["rs"], c2["x"], c["D"], c["nh"], c["nkv"], c["hd"], 51, 1e-6)
    say(f"  registered: step1 rel {_rel(out1, r1):.2e}, step2 rel {_rel(out2, r2):.2e}")
    assert _rel(out1, r1) <= 1e-4 and _rel(out2, r2) <= 1e-4
    assert _rel(kk[:, 50:52], ok[:, 50:52]) <= 2e-5 and _rel(vv[:, 50:52], ov[:, 50:52]) <= 2e-5


def test_attention_rejects_bad_shapes(tg):
    """Unsupported shapes set an error and leave the output untouched."""
    c = _case(70, 256, 8, 2, 32, (F16, F16, F16, F16), 16, 3)
    lib = tg.lib()
    out = np.full(256, 7.0, np.float32)
    lib.tg_hip_clear_error()
    lib.tg_attention_v2(*c["fmts"], *[m.ctypes.data for m in c["w"]], None, None, None, None, None, None, None,
                        c["kv_k"].ctypes.data, c["kv_v"].ctypes.data, 16, 16, 0, c["rc"].ctypes.data,
                        c["rs"].ctypes.data, c["x"].ctypes.data, out.ctypes.data, 256, 8, 2, 32, 16,
                        ctypes.c_float(1e-6))
    assert "kv_len" in tg.last_error()
    assert (out == 7.0).all()
