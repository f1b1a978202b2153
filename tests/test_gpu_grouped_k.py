"""GPU parity of the Q4_K gate/up and Q6_K down expert phases on int8 MFMA
(v_mfma_i32_16x16x32_i8, tg_grouped_k.hip): moe_phase_a / moe_phase_b
(csrc/libtinygiant.c:1279-1384) over many pairs per expert, as a prefill or
a long verify batch routes them.

The MFMA phases form the reference's integer sums per sub-block (dot_q4k_q8
:223-272, dot_q6k_q8 :384-443) and only group the f32 additions differently,
so the bars are those of the v_dot4 phases (stage-wise, see _check_moe):
hidden <= 1e-4 per pair row, q8(hidden) bit-exact, down + combine <= 1e-5 of
max|out|.  The cases cover one and several passes of 16 pairs, rows of more
blocks than a workgroup has waves (a wave takes several blocks or
half-blocks), biases with the gpt-oss activation, a non-zero base output,
and the same layer through the v_dot4 phases.
"""

import sys

import numpy as np
import pytest

import oracle as O
from tests.test_gpu_parity import _check_moe, _experts, close

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class _qk_rows:
    """Sets the pair count from which Q4_K / Q6_K layers take the MFMA phases."""

    def __init__(self, tg, rows):
        self.lib, self.rows = tg.lib(), rows

    def __enter__(self):
        self.prev = self.lib.tg_hip_set_moe_qk_min_rows(self.rows)

    def __exit__(self, *exc):
        self.lib.tg_hip_set_moe_qk_min_rows(self.prev)


def _route(rng, k, n, top):
    rw = np.zeros((n, k), np.float32)
    for r in range(k):
        chosen = rng.choice(n, top, replace=False)
        w = rng.uniform(0.1, 1.0, top).astype(np.float32)
        rw[chosen, r] = w / w.sum()
    return rw


def test_qk_qwen3_prefill_64_tokens(tg, orc):
    """Qwen3-30B-A3B expert shape (D 2048, I 768, q4_K gate/up, q6_K down,
    SiLU), 64 tokens routed top-8 over 32 experts (Zipf): the busiest expert
    holds more than 16 pairs (several passes over its resident slab)."""
    import tinygiant_amd.synth as S
    rng = np.random.default_rng(2048)
    experts, rw = S.routing_rows(rng, 64, 32, 8, 1.1)
    n = len(experts)
    most = int(np.count_nonzero(rw, axis=1).max())
    say(f"qk prefill: {n} experts, busiest {most} pairs")
    assert most > 16
    x = rng.standard_normal((64, 2048)).astype(np.float32)
    with _qk_rows(tg, 1):
        _check_moe(tg, orc, n, 64, 2048, 768, O.FMT_Q4K, [O.FMT_Q6K] * n, O.ACT_SILU, False, rw, x)


@pytest.mark.parametrize("k,n,top", [(12, 4, 2), (40, 4, 2), (150, 2, 1)])
def test_qk_pass_counts(tg, orc, k, n, top):
    """Busiest expert <= 16 pairs (one pass), <= 32 (two), and 150 rows on
    two experts (ten passes, the last partial)."""
    rng = np.random.default_rng(k + 7)
    rw = _route(rng, k, n, top)
    most = int(np.count_nonzero(rw, axis=1).max())
    say(f"qk passes: k={k} n={n} busiest {most}")
    D, I = 1024, 512
    x = rng.standard_normal((k, D)).astype(np.float32)
    with _qk_rows(tg, 1):
        _check_moe(tg, orc, n, k, D, I, O.FMT_Q4K, [O.FMT_Q6K] * n, O.ACT_SILU, False, rw, x)


def test_qk_wide_rows_biases_base(tg, orc):
    """D = 2560 (10 blocks: two waves take two blocks each) and I = 2304 (18
    half-blocks over 8 waves), gate/up/down biases with the gpt-oss clamped
    activation, and a non-zero base output."""
    rng = np.random.default_rng(2560)
    k, n, D, I = 24, 3, 2560, 2304
    rw = np.zeros((n, k), np.float32)
    rw[0, :] = 0.5
    rw[1, ::2] = 0.3
    rw[2, 1::3] = 0.25
    x = rng.uniform(-1, 1, (k, D)).astype(np.float32)
    base = rng.standard_normal((k, D)).astype(np.float32)
    say("qk wide rows, biases, base")
    with _qk_rows(tg, 1):
        _check_moe(tg, orc, n, k, D, I, O.FMT_Q4K, [O.FMT_Q6K] * n, O.ACT_GPTOSS, True, rw, x, base)


def test_qk_equals_dot4_phases(tg, orc):
    """The same Qwen3-shaped layer through the MFMA phases and through the
    v_dot4 expert-major phases: equal to the f32 bar (both sum the same
    integer sub-block sums, in different f32 orders)."""
    import tinygiant_amd.synth as S
    rng = np.random.default_rng(99)
    experts, rw = S.routing_rows(rng, 32, 16, 8, 1.1)
    n = len(experts)
    D, I = 2048, 768
    g, u, d = _experts(n, D, I, O.FMT_Q4K, [O.FMT_Q6K] * n, 11)
    x = rng.standard_normal((32, D)).astype(np.float32)
    outs = {}
    hid = {}
    P = int(np.count_nonzero(rw))
    for name, rows in (("mfma", 1), ("dot4", 0)):
        with _qk_rows(tg, rows):
            h = np.zeros((P, I), np.float32)
            outs[name] = tg.moe_forward_rows_v2(g, u, d, O.FMT_Q4K, [O.FMT_Q6K] * n, None, None, None, O.ACT_SILU,
                                                rw, x, np.zeros((32, D), np.float32), I, hidden_out=h)
            hid[name] = h
    for p in range(P):
        ok, rel = close(hid["mfma"][p], hid["dot4"][p], tol=1e-4)
        assert ok, ("hidden", p, rel)
    # the down phase from identical hidden rows: run the reference on the MFMA path's hidden
    ref_b = orc.moe_v2(g, u, d, O.FMT_Q4K, [O.FMT_Q6K] * n, None, None, None, O.ACT_SILU, rw, x,
                       np.zeros((32, D), np.float32), I, hidden_in=hid["mfma"])
    ok, rel = close(outs["mfma"], ref_b)
    assert ok, ("down+combine", rel)
    say(f"  mfma vs dot4 end-to-end rel {np.abs(outs['mfma'] - outs['dot4']).max() / np.abs(outs['dot4']).max():.2e}")
