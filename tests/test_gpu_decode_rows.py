"""GPU parity of the multi-row persistent decode step: L Qwen3-30B-A3B expert
layers chained as h <- h + MoE_l(RMSNorm_l(h)) over k rows of h in one
cooperative launch (tinygiant/engine.py:281-282,335-341 applied to the rows
of forward_rows: a verify pass of K + 1 rows, tinygiant/specdec.py:66, or a
prefill chunk of 8 rows, engine.py:213-217).

Bars:
  * the persistent kernel gives the bits of the per-layer kernels (mode 0,
    which test_gpu_parity and test_gpu_decode hold to the oracle), over all
    48 layers and over repeated launches;
  * stage by stage against the oracle from the GPU's own per-layer records:
      N  RMSNorm(h) vs the oracle's                   <= 2e-6 of max|x|
      A  hidden vs oracle (from the GPU's x)           <= 1e-4 of max|row|
      B  layer output vs oracle down + combine from the GPU's x and hidden
                                                        <= 1e-5 of max|h|
"""

import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
D, I, E, TOPK = 2048, 768, 128, 8
GB_, DB_ = I * (D // 256) * 144, D * (I // 256) * 210


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class RowLayers:
    """L layers of k rows each: per layer every row's Zipf top-8 of 128
    experts, the union's weights resident on the device (synthesized from
    seeds), the plan, and host copies for the first `host` layers."""

    def __init__(self, tg, L, k, seed, host=0, same=False):
        import tinygiant_amd.synth as S
        self.tg, self.L, self.k = tg, L, k
        lib = tg.lib()
        rng = np.random.default_rng(seed)
        self.norm_host = [rng.uniform(0.5, 1.5, D).astype(np.float32) for _ in range(L)]
        self.norm = []
        for w in self.norm_host:
            a = tg.DeviceArray(D * 4)
            a.upload(w)
            self.norm.append(a)
        self.host, self.bufs, self.plans, self.rw, self.P = [], [], [], [], []
        for l in range(L):
            if same:   # every row picks the same 8 experts: 8 experts of k pairs each
                experts, rw1 = S.routing_rows(rng, 1, E, TOPK)
                rw = np.repeat(rw1, k, axis=1)
            else:
                experts, rw = S.routing_rows(rng, k, E, TOPK)
            n = len(experts)
            buf = tg.DeviceArray(n * (2 * GB_ + DB_))
            ptr = buf.ptr
            gp, up, dp = [], [], []
            for e in experts:
                for kind, w, nb, lst in ((0, 0, GB_, gp), (0, 1, GB_, up), (2, 2, DB_, dp)):
                    lib.tg_hip_synth_fill(kind, S.tensor_seed(seed, l, e, w), ptr, nb, None)
                    lst.append(ptr)
                    ptr += nb
            fm = np.full(n, 2, np.int32)
            a = [(ctypes.c_void_p * n)(*x) for x in (gp, up, dp)]
            rwc = np.ascontiguousarray(rw, np.float32)
            plan = lib.tg_hip_moe_plan_create(ctypes.addressof(a[0]), ctypes.addressof(a[1]), ctypes.addressof(a[2]),
                                              0, fm.ctypes.data, None, None, None, 0, n, rwc.ctypes.data, k, D, I)
            assert plan, tg.last_error()
            if l < host:
                self.host.append(([S.matrix_host(0, S.tensor_seed(seed, l, e, 0), I, D) for e in experts],
                                  [S.matrix_host(0, S.tensor_seed(seed, l, e, 1), I, D) for e in experts],
                                  [S.matrix_host(2, S.tensor_seed(seed, l, e, 2), D, I) for e in experts]))
            self.bufs.append(buf)
            self.plans.append(plan)
            self.rw.append(rwc)
            self.P.append(int((rwc != 0).sum()))
        lib.tg_hip_synchronize()

    def decode(self, h_dev, mode):
        lib = self.tg.lib()
        arr = (ctypes.c_void_p * self.L)(*self.plans)
        nw = (ctypes.c_void_p * self.L)(*[a.ptr for a in self.norm])
        d = lib.tg_hip_decode_create(ctypes.addressof(arr), self.L, ctypes.addressof(nw), ctypes.c_float(1e-6),
                                     h_dev, mode)
        assert d, self.tg.last_error()
        return d

    def close(self):
        lib = self.tg.lib()
        for p in self.plans:
            lib.tg_hip_moe_plan_destroy(p)
        for b in self.bufs + self.norm:
            b.free()


def _run(tg, layers, mode, h0, steps=1, debug=None):
    lib = tg.lib()
    k = layers.k
    h = tg.DeviceArray(k * D * 4)
    h.upload(h0)
    d = layers.decode(h.ptr, mode)
    if debug is not None:
        lib.tg_hip_decode_set_debug(d, debug.ptr)
    for _ in range(steps):
        lib.tg_hip_decode_run(d, None)
    lib.tg_hip_synchronize()
    status = lib.tg_hip_decode_status(d)
    rec = lib.tg_hip_decode_record_bytes(d)
    lib.tg_hip_decode_destroy(d)
    out = h.download(np.float32, k * D).reshape(k, D)
    h.free()
    return out, status, rec


def _h0(k, seed):
    return np.random.default_rng(seed).standard_normal((k, D)).astype(np.float32)


@pytest.mark.parametrize("k", [5, 9, 8])
def test_rows_persistent_equals_per_layer_kernels(tg, k):
    """48 layers: K + 1 = 5 and 9 verify rows and an 8-row prefill chunk,
    two launches in a row (the second starts from the first's h)."""
    say(f"multi-row step k={k}: 48 layers")
    ly = RowLayers(tg, 48, k, 9100 + k)
    try:
        say(f"  pairs per layer {min(ly.P)}..{max(ly.P)}; per-layer kernels")
        h0 = _h0(k, k)
        a, _, _ = _run(tg, ly, 0, h0, steps=2)
        say("  persistent")
        b, st, _ = _run(tg, ly, 2, h0, steps=2)
        assert st == 0, "a barrier wait timed out"
        assert np.isfinite(a).all()
        diff = np.argwhere(a != b)
        assert diff.size == 0, (diff[:4], a[tuple(diff[0])], b[tuple(diff[0])])
    finally:
        ly.close()


def test_rows_plain_launch_and_edges(tg):
    """A plain launch (mode 3) gives the cooperative launch's bits; k = 16
    with every row on the same 8 experts (16 pairs each) and k = 2 give the
    per-layer kernels' bits."""
    for k, same in ((16, True), (2, False), (16, False)):
        say(f"multi-row step k={k} same={same}: 6 layers")
        ly = RowLayers(tg, 6, k, 9200 + k + same, same=same)
        try:
            h0 = _h0(k, 100 + k)
            a, _, _ = _run(tg, ly, 0, h0)
            b, st, _ = _run(tg, ly, 2, h0)
            assert st == 0
            assert a.tobytes() == b.tobytes()
            if k == 16 and same:
                c, st, _ = _run(tg, ly, 3, h0)
                assert st == 0
                assert c.tobytes() == b.tobytes()
        finally:
            ly.close()


def test_rows_create_refuses_more_than_16_rows(tg):
    ly = RowLayers(tg, 1, 17, 9300)
    try:
        lib = tg.lib()
        h = tg.DeviceArray(17 * D * 4)
        arr = (ctypes.c_void_p * 1)(*ly.plans)
        d = lib.tg_hip_decode_create(ctypes.addressof(arr), 1, None, ctypes.c_float(1e-6), h.ptr, 2)
        assert not d
        assert "16" in tg.last_error()
        h.free()
    finally:
        ly.close()


@pytest.mark.parametrize("k", [5, 9])
def test_rows_persistent_stagewise(tg, orc, k):
    """Four layers checked stage by stage from the GPU's own inputs."""
    L = 4
    say(f"multi-row step k={k}: stage-wise, {L} layers")
    ly = RowLayers(tg, L, k, 9400 + k, host=L)
    try:
        rb = None
        h0 = _h0(k, 200 + k)
        lib = tg.lib()
        # record size from a throwaway step
        h = tg.DeviceArray(k * D * 4)
        d = ly.decode(h.ptr, 2)
        rb = lib.tg_hip_decode_record_bytes(d)
        lib.tg_hip_decode_destroy(d)
        h.free()
        pmax = (rb // 4 - 2 * k * D) // I
        assert pmax == max(ly.P)
        dbg = tg.DeviceArray(L * rb)
        h_final, st, _ = _run(tg, ly, 2, h0, debug=dbg)
        assert st == 0
        raw = dbg.download(np.uint8, L * rb).reshape(L, rb)
        dbg.free()
        for l in range(L):
            rec = raw[l]
            hin = rec[:k * D * 4].view(np.float32).reshape(k, D)
            x = rec[k * D * 4:2 * k * D * 4].view(np.float32).reshape(k, D)
            P = ly.P[l]
            hid = rec[2 * k * D * 4:].view(np.float32).reshape(pmax, I)[:P]
            if l == 0:
                assert np.array_equal(hin, h0)
            for r in range(k):   # N
                x_ref = orc.rms_norm(hin[r], ly.norm_host[l], 1e-6)
                assert np.abs(x[r] - x_ref).max() <= 2e-6 * np.abs(x_ref).max(), (l, r)
            g, u, dm = ly.host[l]
            n = len(g)
            h_ref = np.zeros((P, I), np.float32)   # A
            orc.moe_v2(g, u, dm, 0, [2] * n, None, None, None, 0, ly.rw[l], x, np.zeros((k, D), np.float32), I,
                       hidden_out=h_ref)
            for p in range(P):
                assert np.abs(hid[p] - h_ref[p]).max() <= 1e-4 * np.abs(h_ref[p]).max(), (l, p)
            out_ref = orc.moe_v2(g, u, dm, 0, [2] * n, None, None, None, 0, ly.rw[l], x, hin.copy(), I,
                                 hidden_in=np.ascontiguousarray(hid))   # B
            h_out = h_final if l == L - 1 else raw[l + 1][:k * D * 4].view(np.float32).reshape(k, D)
            err = np.abs(h_out - out_ref).max() / np.abs(out_ref).max()
            say(f"  layer {l}: {n} experts, {P} pairs, output rel {err:.2e}")
            assert err <= 1e-5, (l, err)
    finally:
        ly.close()
