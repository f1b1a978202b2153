"""GPU parity of a greedy self-speculative round (tinygiant_amd.specdec) over
one Qwen3-30B-A3B-shaped layer with all 128 experts in HBM and the full
151936 x 2048 q6_K head, against the oracle running the same round.

The oracle round restates the reference: the draft passes route with
Router.select(restrict=True) over the resident experts (tinygiant/router.py:
46-54, engine.py:287), the verify pass routes [t0] + drafts exactly
(specdec.py:66), each pass is forward_rows for one MoE layer (engine.py:
281-282, 285-341: RMSNorm * ffn_norm, per-row top-8, the union of experts
with row weights, moe_out zero-filled then X += moe_out) followed by
RMSNorm * output_norm and tg_matmul over the head per row (engine.py:
347-354), and the drafts are accepted while argmax(P[r]) == drafts[r]
(specdec.py:73-77), the round emitting the accepted drafts and the target's
next token (specdec.py:91-104).

Bars: every pass's union of experts, every draft token, every target argmax
and the accepted count equal the oracle's.  Argmax parity needs each
oracle argmax to win by more than the logit tolerance (1e-4 of the largest
logit: the GPU's RMSNorm'd rows may differ from the oracle's by an ulp and
flip one q8 rounding); the test asserts that margin first, so a near tie
shows as a failed precondition, not as a parity failure.
"""

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

V, D, I, E, TOPK = 151936, 2048, 768, 128, 8
EPS = 1e-6
LOGIT_TOL = 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class OracleLayer:
    """The same model on the host, run through the oracle."""

    def __init__(self, orc, seed):
        import tinygiant_amd.specdec as SD
        import tinygiant_amd.synth as S
        self.orc, self.SD = orc, SD
        self.m = SD.model_host(seed)
        self.g = [S.matrix_host(0, self.m["seeds"][(e, 0)], I, D) for e in range(E)]
        self.u = [S.matrix_host(0, self.m["seeds"][(e, 1)], I, D) for e in range(E)]
        self.d = [S.matrix_host(2, self.m["seeds"][(e, 2)], D, I) for e in range(E)]
        self.head = S.matrix_host(2, self.m["head_seed"], V, D)
        self.margins = []

    def forward_rows(self, tokens, draft):
        o, m = self.orc, self.m
        X = np.stack([self.SD.embed(m["seed"], t) for t in tokens]).astype(np.float32)
        k = len(tokens)
        N = np.stack([o.rms_norm(X[r], m["ffn_norm"], EPS) for r in range(k)])
        idx = np.zeros((k, TOPK), np.int64)
        w = np.zeros((k, TOPK), np.float32)
        for r in range(k):
            _, idx[r], w[r] = o.route(m["router"], m["bias"], N[r], TOPK, resident=m["resident"] if draft else None)
        experts, rw = self.SD.union_rows(idx, w)
        moe_out = np.zeros((k, D), np.float32)
        o.moe_v2([self.g[e] for e in experts], [self.u[e] for e in experts], [self.d[e] for e in experts],
                 o.FMT_Q4K, [o.FMT_Q6K] * len(experts), None, None, None, o.ACT_SILU, rw, N, moe_out, I)
        X += moe_out
        out = []
        for r in range(k):
            logits = o.matmul(o.FMT_Q6K, self.head, None, o.rms_norm(X[r], m["out_norm"], EPS), V, D)
            top2 = np.sort(logits)[-2:]
            self.margins.append(float((top2[1] - top2[0]) / np.abs(logits).max()))
            out.append(int(np.argmax(logits)))
        say(f"  oracle pass: {k} rows, {len(experts)} experts")
        return out, experts

    def verify_round(self, t0, n_draft):
        drafts, draft_experts = [], []
        inp = t0
        for _ in range(n_draft):
            (d,), ex = self.forward_rows([inp], draft=True)
            drafts.append(d)
            draft_experts.append(ex)
            inp = d
        target, union = self.forward_rows([t0] + drafts, draft=False)
        n_acc = 0
        while n_acc < n_draft and target[n_acc] == drafts[n_acc]:
            n_acc += 1
        return {"drafts": drafts, "target": target, "accepted": n_acc, "emitted": drafts[:n_acc] + [target[n_acc]],
                "union": union, "draft_experts": draft_experts}


@pytest.mark.parametrize("n_draft", [4, 8])
def test_spec_round_matches_oracle(tg, orc, n_draft):
    """K = 4 and 8 drafts (K + 1 = 5 and 9 verify rows) over 128 experts with
    Zipf-skewed top-8 routing, draft routing restricted to the 64 most
    popular experts, and the full q6_K head."""
    import tinygiant_amd.specdec as SD
    seed, t0 = 4242 + n_draft, 1234 + n_draft
    say(f"spec round K={n_draft}: oracle")
    oracle_layer = OracleLayer(orc, seed)
    ref = oracle_layer.verify_round(t0, n_draft)
    # preconditions on the oracle: no near tie at any argmax, drafts route
    # over resident experts only
    assert min(oracle_layer.margins) > LOGIT_TOL, min(oracle_layer.margins)
    for ex in ref["draft_experts"]:
        assert all(oracle_layer.m["resident"][e] for e in ex)
    del oracle_layer
    say(f"spec round K={n_draft}: gpu")
    layer = SD.SpecLayer(seed)
    try:
        got = layer.verify_round(t0, n_draft)
    finally:
        layer.free()
    say(f"  union {len(ref['union'])} experts, accepted {ref['accepted']} of {n_draft}")
    assert got["draft_experts"] == ref["draft_experts"]
    assert got["drafts"] == ref["drafts"]
    assert got["union"] == ref["union"]
    assert got["target"] == ref["target"]
    assert got["accepted"] == ref["accepted"] and got["emitted"] == ref["emitted"]
    # the verify batch is the grouped case: 1..K+1 rows per expert
    assert len(ref["union"]) > TOPK

