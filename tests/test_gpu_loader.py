"""The on-disk expert cache in HBM (tinygiant_amd/loader.py over
tg_hip_upload_file): the reference's layer files (tinygiant/relayout.py:
147-162, read by tinygiant/cache.py:29-54) land in device memory byte for
byte, and a MoE plan over the loaded experts gives the same bits as the
host-pointer call tg_moe_forward_rows_v2 over the same tensors."""

import ctypes
import sys

import numpy as np
import pytest

import oracle as O
from tests._expert_cache import synth_layers, write_cache
from tests.test_gpu_parity import close

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _run_plan(tg, plan, x):
    L = tg.lib()
    k, D = x.shape
    xin, out = tg.DeviceArray(x.nbytes), tg.DeviceArray(x.nbytes)
    xin.upload(x)
    out.upload(np.zeros_like(x))
    L.tg_hip_moe_plan_run(plan, xin.ptr, out.ptr, None)
    L.tg_hip_synchronize()
    return out.download(np.float32, k * D).reshape(k, D)


@pytest.mark.parametrize("shape", ["qwen", "mxfp4"])
def test_loaded_experts_bytes_and_forward(tg, orc, tmp_path, shape):
    from tinygiant_amd.loader import HBMExpertCache
    if shape == "qwen":
        D, I, fm, rows, act = 2048, 768, {"gate": O.FMT_Q4K, "up": O.FMT_Q4K, "down": O.FMT_Q6K}, 0, O.ACT_SILU
    else:
        D, I, fm, rows, act = 1024, 1024, {"gate": O.FMT_MXFP4, "up": O.FMT_MXFP4, "down": O.FMT_MXFP4}, 1, O.ACT_GPTOSS
    E = 6
    layers = synth_layers(2, E, D, I, fm, 404)
    write_cache(tmp_path, layers, E, D, I, fm)
    say(f"loader {shape}: 2 layers x {E} experts")
    cache = HBMExpertCache(tmp_path, chunk_mb=1)       # 1 MiB chunks: many pinned-buffer round trips
    try:
        for layer in range(2):
            blob = np.fromfile(tmp_path / f"layer_{layer:03d}.q4.bin", np.uint8)
            got = cache._bufs[layer].download(np.uint8, blob.size)
            assert got.tobytes() == blob.tobytes()
            assert cache.formats(layer) == fm
        assert cache.bytes_loaded == sum((tmp_path / f"layer_{l:03d}.q4.bin").stat().st_size for l in range(2))
        # a plan over experts 5, 0, 3 of layer 1 (any order), 12 rows
        experts, k = [5, 0, 3], 12
        rng = np.random.default_rng(12)
        rw = rng.uniform(0.1, 1.0, (len(experts), k)).astype(np.float32)
        rw[1, ::3] = 0
        x = rng.uniform(-1, 1, (k, D)).astype(np.float32)
        g = [layers[1][e]["gate"] for e in experts]
        u = [layers[1][e]["up"] for e in experts]
        d = [layers[1][e]["down"] for e in experts]
        L = tg.lib()
        prev = L.tg_hip_set_moe_grouped_min_rows(rows if rows else 1 << 20)
        try:
            want = tg.moe_forward_rows_v2(g, u, d, fm["gate"], [fm["down"]] * len(experts), None, None, None, act, rw,
                                          x, np.zeros((k, D), np.float32), I)
            plan = cache.plan(1, experts, rw, k, D, I, act)
            try:
                got = _run_plan(tg, plan, x)
            finally:
                L.tg_hip_moe_plan_destroy(plan)
        finally:
            L.tg_hip_set_moe_grouped_min_rows(prev)
        assert got.tobytes() == want.tobytes()
        ref = orc.moe_v2(g, u, d, fm["gate"], [fm["down"]] * len(experts), None, None, None, act, rw, x,
                         np.zeros((k, D), np.float32), I)
        ok, rel = close(got, ref, tol=1e-3)    # end to end, q8 roundings of the hidden may flip
        assert ok, rel
    finally:
        cache.close()


def test_loader_missing_and_short_files(tg, tmp_path):
    from tinygiant_amd.loader import HBMExpertCache
    D, I, fm = 256, 256, {"gate": O.FMT_Q4K, "up": O.FMT_Q4K, "down": O.FMT_Q4K}
    write_cache(tmp_path, synth_layers(2, 2, D, I, fm, 5), 2, D, I, fm)
    say("loader errors")
    f1 = tmp_path / "layer_001.q4.bin"
    data = f1.read_bytes()
    f1.write_bytes(data[:-100])                        # shorter than total_bytes
    with pytest.raises(IOError, match="short"):
        HBMExpertCache(tmp_path)
    (tmp_path / "layer_000.q4.bin").unlink()
    with pytest.raises(IOError, match="cannot open"):
        HBMExpertCache(tmp_path, layers=[0])
    # the library stays usable after the errors
    c = HBMExpertCache(tmp_path, layers=[], chunk_mb=2)
    assert c.bytes_loaded == 0
    f1.write_bytes(data)
    c = HBMExpertCache(tmp_path, layers=[1])
    assert c._bufs[1].download(np.uint8, len(data)).tobytes() == data
    c.close()
