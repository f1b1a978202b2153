"""Seeded synthetic workloads of the fused MoE expert path.

Weights come from the library's integer generator (csrc/tg_synth.h), which
gives the same bytes on the host and on the GPU; activations and router
logits come from numpy's PCG64 with recorded seeds.  Shapes:

  Qwen3-30B-A3B  D=2048, I=768, 128 experts, top-8, 48 layers
                 (tinygiant/_constants.py:1-13), gate/up q4_K, down q6_K
  gpt-oss-120b   D=I=2880, 128 experts, top-4, 36 layers, mxfp4, biases,
                 gpt-oss activation (csrc/test_libtinygiant.c:561)
"""

import numpy as np

from . import FMT_MXFP4, FMT_Q4K, FMT_Q6K, FMT_Q80, lib

QWEN = dict(D=2048, I=768, E=128, top_k=8, L=48, gate_fmt=FMT_Q4K, down_fmt=FMT_Q6K)
GPTOSS = dict(D=2880, I=2880, E=128, top_k=4, L=36, gate_fmt=FMT_MXFP4, down_fmt=FMT_MXFP4)

SYN_KIND = {FMT_Q4K: 0, FMT_Q6K: 2, FMT_MXFP4: 3, FMT_Q80: 4}
MASK64 = (1 << 64) - 1


def tensor_seed(base, layer, expert, which):
    """Seed of one weight tensor (which: 0 gate, 1 up, 2 down, 3 head)."""
    z = (base * 0x9E3779B97F4A7C15 + (layer << 24) + (expert << 4) + which) & MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def matrix_host(fmt, seed, nrows, ncols):
    """nrows x ncols weight matrix in `fmt`, as a uint8 array of its bytes."""
    rb = lib().tg_row_bytes(fmt, ncols)
    out = np.empty(nrows * rb, np.uint8)
    lib().tg_hip_synth_fill_host(SYN_KIND.get(fmt, -1), seed, out.ctypes.data, out.nbytes)
    return out


def zipf_topk(rng, n_experts, top_k, s=1.1, perm=None):
    """top_k distinct experts from a Zipf(s) popularity over a permutation of
    the experts (Gumbel-top-k sampling without replacement)."""
    if perm is None:
        perm = np.arange(n_experts)
    logp = -s * np.log(np.arange(1, n_experts + 1, dtype=np.float64))
    g = rng.gumbel(size=n_experts)
    order = np.argsort(-(logp + g))[:top_k]
    return perm[order]


def router_weights(rng, top_k):
    """Softmax over the selected logits only (tinygiant/router.py:39-42)."""
    l = rng.standard_normal(top_k).astype(np.float32)
    e = np.exp(l - l.max())
    return (e / e.sum()).astype(np.float32)


def routing_rows(rng, k, n_experts, top_k, s=1.1, perm=None):
    """Per-row top-k choices -> (sorted expert union, row_weights [n, k])
    exactly as NWSEngine.forward_rows builds them (tinygiant/engine.py:285-318)."""
    union = {}
    for r in range(k):
        idx = zipf_topk(rng, n_experts, top_k, s, perm)
        w = router_weights(rng, top_k)
        for e, wt in zip(idx, w):
            union.setdefault(int(e), {})[r] = float(wt)
    experts = sorted(union)
    rw = np.zeros((len(experts), k), np.float32)
    for i, e in enumerate(experts):
        for r, wt in union[e].items():
            rw[i, r] = wt
    return experts, rw
