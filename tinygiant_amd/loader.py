"""The reference's on-disk expert cache, uploaded whole into HBM.

The cache is what tinygiant/relayout.py writes (write_expert_cache_q4,
relayout.py:147-162, and the index, :287-300): a directory with index.json
and one file per layer, layer_NNN.q4.bin, holding every expert of the layer
in expert-id order, each as its gate, up and down tensors back to back in
their GGUF block format.  tinygiant/cache.py:29-54 reads it through mmap
views and mlocks the hot experts; with 288 GB of HBM the whole cache fits
(Qwen3-30B-A3B: 18.8 GB, gpt-oss-120b: 61 GB), so HBMExpertCache copies each
layer file once, straight into device memory (tg_hip_upload_file: pread into
pinned buffers overlapped with the host-to-device copies), and hands out
device pointers per expert for the device-resident MoE plans.

The bytes in HBM are the file's bytes: the reference's expert sizes are
multiples of 16 bytes, so every tensor starts 16-byte aligned when the layer
buffer does, which the MXFP4 MFMA phases need and HBMExpertCache checks.
"""

import json
from pathlib import Path


# tinygiant/engine.py:21 (format names of index.json -> the library's codes)
FMT_NAMES = {"q4_k": 0, "float16": 1, "q6_k": 2, "mxfp4": 3, "q8_0": 4}
EXPERT_KEYS = ("gate", "up", "down")   # tinygiant/_constants.py:13


def read_index(cache_dir):
    """index.json of an expert cache directory."""
    with open(Path(cache_dir) / "index.json") as f:
        return json.load(f)


def layer_layout(index, layer):
    """(file name, total bytes, {key: format code}, [(expert id, offset,
    {key: size})]) of one layer, as cache.py:35-54 reads them; a missing
    format is q4_k (engine.py:326-327)."""
    info = index["layers"][str(layer)]
    names = info.get("tensor_formats", {})
    fmts = {k: FMT_NAMES[names.get(k, "q4_k")] for k in EXPERT_KEYS}
    experts = []
    for key, e in info["expert_offsets"].items():
        experts.append((int(key), int(e["offset"]), {k: int(e["sizes"][k]) for k in EXPERT_KEYS}))
    experts.sort()
    return info["file"], int(info["total_bytes"]), fmts, experts


class HBMExpertCache:
    """Every expert of an on-disk cache resident in HBM.

    ptrs(layer, expert) -> {"gate", "up", "down"}: device addresses;
    formats(layer) -> {"gate", "up", "down"}: format codes;
    plan(layer, experts, row_weights, k, ...) -> a tg_hip_moe_plan over them.
    """

    def __init__(self, cache_dir, index=None, layers=None, chunk_mb=64):
        from . import DeviceArray, last_error, lib as _lib_handle
        self.cache_dir = Path(cache_dir)
        self.index = index if index is not None else read_index(cache_dir)
        self.n_layers = int(self.index["n_layers"])
        self.n_experts = int(self.index["n_experts"])
        lib = _lib_handle()
        self._bufs, self._ptrs, self._fmts = {}, {}, {}
        self.bytes_loaded = 0
        keys = sorted(int(k) for k in self.index["layers"])
        for layer in keys if layers is None else layers:
            fname, total, fmts, experts = layer_layout(self.index, layer)
            buf = DeviceArray(total)
            n = lib.tg_hip_upload_file(str(self.cache_dir / fname).encode(), 0, total, buf.ptr, chunk_mb << 20)
            if n != total:
                buf.free()
                raise IOError(f"loading {fname}: {last_error()}")
            self._bufs[layer] = buf
            self._fmts[layer] = fmts
            for eid, off, sizes in experts:
                p, d = buf.ptr + off, {}
                for k in EXPERT_KEYS:
                    if p % 16:
                        raise ValueError(f"layer {layer} expert {eid} {k} is not 16-byte aligned in HBM")
                    d[k] = p
                    p += sizes[k]
                self._ptrs[(layer, eid)] = d
            self.bytes_loaded += total

    def ptrs(self, layer, expert):
        return self._ptrs[(layer, expert)]

    def formats(self, layer):
        return self._fmts[layer]

    def plan(self, layer, experts, row_weights, k, embed_dim, inter_dim, act=0, biases=None):
        """tg_hip_moe_plan_create over the given experts of a layer
        (row_weights [len(experts)][k], float32); biases: optional (gate, up,
        down) lists of device pointers."""
        import ctypes
        import numpy as np
        from . import last_error, lib as _lib_handle
        lib = _lib_handle()
        n = len(experts)
        f = self._fmts[layer]
        arrs = [(ctypes.c_void_p * n)(*[self._ptrs[(layer, e)][key] for e in experts]) for key in EXPERT_KEYS]
        bias = [None] * 3 if biases is None else [(ctypes.c_void_p * n)(*b) for b in biases]
        fm = np.full(n, f["down"], np.int32)
        rw = np.ascontiguousarray(row_weights, np.float32)
        p = lib.tg_hip_moe_plan_create(*[ctypes.addressof(a) for a in arrs], f["gate"], fm.ctypes.data,
                                       *[None if b is None else ctypes.addressof(b) for b in bias], act, n,
                                       rw.ctypes.data, k, embed_dim, inter_dim)
        if not p:
            raise RuntimeError(last_error())
        return p

    def close(self):
        for b in self._bufs.values():
            b.free()
        self._bufs.clear()
        self._ptrs.clear()
