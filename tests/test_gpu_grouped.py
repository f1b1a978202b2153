"""GPU parity of the MXFP4 expert phases on block-scaled f8f6f4 MFMA
(v_mfma_scale_f32_16x16x128_f8f6f4, tg_grouped.hip):
moe_phase_a / moe_phase_b (csrc/libtinygiant.c:1279-1384) over many pairs
per expert, as a prefill or a long verify batch routes them.

The MFMA phases form the same per-block integer sums as dot_mxfp4_q8
(:533-547) and accumulate the f32 terms block by block in the reference's
order, so the bars are those of the per-pair kernels (stage-wise, see
_check_moe): hidden <= 1e-4 per pair row, q8(hidden) bit-exact, down + combine
<= 1e-5 of max|out|.  Each case covers one of the pass shapes: one, two or
four 16-row tiles per pass, more pairs than one pass holds, weight rows past
the matrix end, a block count that is not a multiple of the four-block
pipeline stage, and experts whose down matrix is not MXFP4.
"""

import sys

import numpy as np
import pytest

import oracle as O
from tests.test_gpu_parity import _check_moe, close

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class _grouped_rows:
    """Sets the pair count from which MXFP4 layers take the MFMA phases."""

    def __init__(self, tg, rows):
        self.lib, self.rows = tg.lib(), rows

    def __enter__(self):
        self.prev = self.lib.tg_hip_set_moe_grouped_min_rows(self.rows)

    def __exit__(self, *exc):
        self.lib.tg_hip_set_moe_grouped_min_rows(self.prev)


def _rows(rng, k, n, top, s=1.1):
    import tinygiant_amd.synth as S
    experts, rw = S.routing_rows(rng, k, n, top, s)
    return len(experts), rw, int(np.count_nonzero(rw, axis=1).max())


def test_grouped_gptoss_prefill_64_rows(tg, orc):
    """gpt-oss shape (D = I = 2880, biases, clamped activation), 64 rows, top-4
    over 16 experts: the busiest expert holds more than 32 pairs (4 tiles)."""
    rng = np.random.default_rng(2880)
    n, rw, most = _rows(rng, 64, 16, 4)
    say(f"grouped gptoss prefill: {n} experts, busiest {most} pairs")
    assert most > 32
    x = rng.uniform(-1, 1, (64, 2880)).astype(np.float32)
    with _grouped_rows(tg, 1):
        _check_moe(tg, orc, n, 64, 2880, 2880, O.FMT_MXFP4, [O.FMT_MXFP4] * n, O.ACT_GPTOSS, True, rw, x)


@pytest.mark.parametrize("k,n,top", [(12, 4, 2), (40, 4, 2), (150, 2, 1)])
def test_grouped_tile_counts(tg, orc, k, n, top):
    """Busiest expert <= 16 (1 tile), <= 32 (2 tiles), and 150 rows on two
    experts: more pairs than one 64-pair pass, so the weights are walked
    twice with a partial last tile."""
    rng = np.random.default_rng(k)
    rw = np.zeros((n, k), np.float32)
    for r in range(k):
        chosen = rng.choice(n, top, replace=False)
        w = rng.uniform(0.1, 1.0, top).astype(np.float32)
        rw[chosen, r] = w / w.sum()
    most = int(np.count_nonzero(rw, axis=1).max())
    say(f"grouped tiles: k={k} n={n} busiest {most}")
    D = I = 1024
    x = rng.standard_normal((k, D)).astype(np.float32)
    with _grouped_rows(tg, 1):
        _check_moe(tg, orc, n, k, D, I, O.FMT_MXFP4, [O.FMT_MXFP4] * n, O.ACT_SILU, False, rw, x)


def test_grouped_ragged_rows_and_blocks(tg, orc):
    """D = I = 1056: 33 blocks per row (a partial four-block stage) and 66
    row groups of 16 (the last workgroup's waves run past the matrix end);
    a non-zero base output; one expert with a q4_K down matrix."""
    rng = np.random.default_rng(1056)
    k, n, D, I = 24, 3, 1056, 1056
    rw = np.zeros((n, k), np.float32)
    rw[0, :] = 0.5
    rw[1, ::2] = 0.3
    rw[2, 1::3] = 0.25
    x = rng.standard_normal((k, D)).astype(np.float32)
    base = rng.standard_normal((k, D)).astype(np.float32)
    say("grouped ragged")
    with _grouped_rows(tg, 1):
        _check_moe(tg, orc, n, k, D, I, O.FMT_MXFP4, [O.FMT_MXFP4, O.FMT_MXFP4, O.FMT_MXFP4], O.ACT_GPTOSS, True,
                   rw, x, base)
    # q4_K down requires I % 256 == 0: a separate shape
    k, D, I = 20, 1056, 1024
    fmts = [O.FMT_MXFP4, O.FMT_Q4K, O.FMT_MXFP4]
    x = rng.standard_normal((k, D)).astype(np.float32)
    rw = rng.uniform(0.1, 1.0, (n, k)).astype(np.float32)
    say("grouped mixed down formats")
    with _grouped_rows(tg, 1):
        _check_moe(tg, orc, n, k, D, I, O.FMT_MXFP4, fmts, O.ACT_SILU, False, rw, x)


def test_grouped_equals_per_pair_kernels(tg, orc):
    """The same layer through the MFMA phases and through the per-pair
    kernels: equal to the f32 bar (the two sum the same integer block sums in
    different f32 orders)."""
    from tests.test_gpu_parity import _experts
    rng = np.random.default_rng(77)
    n, rw, most = _rows(rng, 32, 8, 4)
    D = I = 2880
    g, u, d = _experts(n, D, I, O.FMT_MXFP4, [O.FMT_MXFP4] * n, 5)
    gb = [rng.uniform(-0.5, 0.5, I).astype(np.float32) for _ in range(n)]
    ub = [rng.uniform(-0.5, 0.5, I).astype(np.float32) for _ in range(n)]
    db = [rng.uniform(-0.05, 0.05, D).astype(np.float32) for _ in range(n)]
    x = rng.uniform(-1, 1, (32, D)).astype(np.float32)
    P = int(np.count_nonzero(rw))
    outs, hids = [], []
    for rows in (0, 1):
        h = np.zeros((P, I), np.float32)
        with _grouped_rows(tg, rows):
            outs.append(tg.moe_forward_rows_v2(g, u, d, O.FMT_MXFP4, [O.FMT_MXFP4] * n, gb, ub, db, O.ACT_GPTOSS, rw,
                                               x, np.zeros((32, D), np.float32), I, hidden_out=h))
        hids.append(h)
    say(f"grouped vs per-pair: {n} experts, busiest {most}")
    for p in range(P):
        ok, rel = close(hids[1][p], hids[0][p], tol=1e-4)
        assert ok, ("hidden", p, rel)
    flips = int(np.count_nonzero(orc.quantize_q8(hids[0])["qs"] != orc.quantize_q8(hids[1])["qs"]))
    ok, rel = close(outs[1], outs[0], tol=1e-5 if flips == 0 else 1e-3)
    assert ok, (rel, flips)


def test_grouped_run_to_run_identical(tg):
    """The MFMA phases are deterministic: two calls give the same bits."""
    from tests.test_gpu_parity import _experts
    rng = np.random.default_rng(3)
    n, rw, _ = _rows(rng, 48, 6, 4)
    D = I = 1024
    g, u, d = _experts(n, D, I, O.FMT_MXFP4, [O.FMT_MXFP4] * n, 8)
    x = rng.standard_normal((48, D)).astype(np.float32)
    with _grouped_rows(tg, 1):
        a = tg.moe_forward_rows_v2(g, u, d, O.FMT_MXFP4, [O.FMT_MXFP4] * n, None, None, None, O.ACT_SILU, rw, x,
                                   np.zeros((48, D), np.float32), I)
        b = tg.moe_forward_rows_v2(g, u, d, O.FMT_MXFP4, [O.FMT_MXFP4] * n, None, None, None, O.ACT_SILU, rw, x,
                                   np.zeros((48, D), np.float32), I)
    assert a.tobytes() == b.tobytes()
