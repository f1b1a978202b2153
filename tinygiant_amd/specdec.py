"""Self-speculative decoding round (greedy) on the device: the verify batch
of the fused MoE expert path end to end.

The reference drafts K tokens with the same model restricted to resident
experts (zero I/O), then runs one exact pass over [t0] + drafts and accepts
the drafts while the target's argmax agrees (tinygiant/specdec.py:51-108 at
temperature 0; draft routing Router.select(restrict=True),
tinygiant/router.py:46-54, engine.py:287; the verify pass engine.py:232-359;
the head engine.py:347-354).  Here the model is one Qwen3-30B-A3B-shaped MoE
layer and its q6_K output head, all resident in HBM:

    x_r = embed(token_r)                       synthetic, seeded per token
    n_r = RMSNorm(x_r) * ffn_norm              tg_hip_rms_norm_dev
    experts, weights = route(n_r)              tg_hip_route_dev / _restricted_dev
    h_r = x_r + MoE(n_r)                       tg_hip_moe_plan_run over the union
    logits_r = head(RMSNorm(h_r) * out_norm)   tg_hip_head_argmax_dev (argmax fused)

A pass runs its rows in one batch, as forward_rows does: the union of the
rows' experts is read once, each with 1..k rows (engine.py:285-334).  The
router is 128 x 2048 f32 rows N(0, 1/2048) plus a per-expert bias
log(p_e), p a Zipf(1.1) popularity over a seeded permutation of the experts,
so every row picks its top-8 with Zipf skew; the draft's resident experts
are the most popular ones.

Routing and the union are formed on the host from the device router's
top-k (the reference routes in Python, engine.py:285-318); every weight byte
and every matrix product stays on the device.
"""

import ctypes

import numpy as np

from . import FMT_Q4K, FMT_Q6K, ACT_SILU, DeviceArray, last_error, lib

D, I, E, TOPK = 2048, 768, 128, 8
VOCAB = 151936
GATE_B = I * (D // 256) * 144          # 884,736
DOWN_B = D * (I // 256) * 210          # 1,290,240
EXPERT_B = 2 * GATE_B + DOWN_B         # 3,059,712
EPS = 1e-6
ZIPF_S = 1.1


def embed(seed, token):
    """Synthetic embedding of a token id: D float32 values N(0, 1) from
    PCG64 seeded with (seed, token)."""
    return np.random.default_rng([seed, int(token)]).standard_normal(D, dtype=np.float32)


def model_host(seed, vocab=VOCAB, n_resident=64):
    """The model's float tensors and seeds (numpy, host): router [E][D],
    router bias [E], ffn_norm [D], output_norm [D], the resident mask [E],
    the popularity permutation, and the weight seeds (tensor_seed(seed,
    0, e, which) for expert e; the head is tensor_seed(seed, 0, 0, 3))."""
    from .synth import tensor_seed
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)                  # perm[r] is the expert of popularity rank r
    logp = -ZIPF_S * np.log(np.arange(1, E + 1, dtype=np.float64))
    logp -= np.log(np.exp(logp).sum())
    bias = np.zeros(E, np.float32)
    bias[perm] = logp.astype(np.float32)
    router = (rng.standard_normal((E, D)) / np.sqrt(D)).astype(np.float32)
    ffn_norm = rng.uniform(0.5, 1.5, D).astype(np.float32)
    out_norm = rng.uniform(0.5, 1.5, D).astype(np.float32)
    resident = np.zeros(E, bool)
    resident[perm[:n_resident]] = True
    seeds = {(e, w): tensor_seed(seed, 0, e, w) for e in range(E) for w in range(3)}
    return dict(seed=seed, vocab=vocab, router=router, bias=bias, ffn_norm=ffn_norm, out_norm=out_norm,
                resident=resident, perm=perm, seeds=seeds, head_seed=tensor_seed(seed, 0, 0, 3))


def union_rows(idx, w):
    """Per-row top-k -> (sorted expert union, row_weights [n][k]), as
    NWSEngine.forward_rows builds them (tinygiant/engine.py:285-318)."""
    k = idx.shape[0]
    union = {}
    for r in range(k):
        for e, wt in zip(idx[r], w[r]):
            union.setdefault(int(e), {})[r] = float(wt)
    experts = sorted(union)
    rw = np.zeros((len(experts), k), np.float32)
    for i, e in enumerate(experts):
        for r, wt in union[e].items():
            rw[i, r] = wt
    return experts, rw


class SpecLayer:
    """One MoE layer + q6_K output head resident in HBM (see the module
    docstring), with the draft and the exact forward passes."""

    def __init__(self, seed, vocab=VOCAB, n_resident=64, max_rows=16):
        self.lib = lib()
        self.m = model_host(seed, vocab, n_resident)
        self.vocab = vocab
        self.max_rows = max_rows
        L = self.lib
        self.experts = DeviceArray(E * EXPERT_B)
        base = self.experts.ptr
        for e in range(E):
            L.tg_hip_synth_fill(0, self.m["seeds"][(e, 0)], self.gate_ptr(e), GATE_B, None)
            L.tg_hip_synth_fill(0, self.m["seeds"][(e, 1)], self.up_ptr(e), GATE_B, None)
            L.tg_hip_synth_fill(2, self.m["seeds"][(e, 2)], self.down_ptr(e), DOWN_B, None)
        del base
        self.head_bytes = vocab * (D // 256) * 210
        self.head = DeviceArray(self.head_bytes)
        L.tg_hip_synth_fill(2, self.m["head_seed"], self.head.ptr, self.head_bytes, None)
        self.router = self._put(self.m["router"])
        self.bias = self._put(self.m["bias"])
        self.ffn_norm = self._put(self.m["ffn_norm"])
        self.out_norm = self._put(self.m["out_norm"])
        self.resident = self._put(self.m["resident"].astype(np.uint8))
        k = max_rows
        self.x = DeviceArray(k * D * 4)          # the rows' hidden state (h after the layer)
        self.n = DeviceArray(k * D * 4)          # RMSNorm(x) * ffn_norm
        self.idx = DeviceArray(k * TOPK * 4)
        self.w = DeviceArray(k * TOPK * 4)
        self.rsc = DeviceArray(L.tg_hip_route_scratch_bytes(k, E))
        self.am = DeviceArray(k * 4)
        self.val = DeviceArray(k * 4)
        self.hsc = DeviceArray(L.tg_hip_head_scratch_bytes(k, vocab, D))
        L.tg_hip_synchronize()
        self.last = {}

    def _put(self, a):
        d = DeviceArray(a.nbytes)
        d.upload(np.ascontiguousarray(a))
        return d

    def gate_ptr(self, e):
        return self.experts.ptr + e * GATE_B

    def up_ptr(self, e):
        return self.experts.ptr + E * GATE_B + e * GATE_B

    def down_ptr(self, e):
        return self.experts.ptr + 2 * E * GATE_B + e * DOWN_B

    def weight_bytes(self):
        return E * EXPERT_B + self.head_bytes

    def plan(self, experts, rw):
        """A MoE plan over the union's experts and their row weights."""
        L = self.lib
        n = len(experts)
        k = rw.shape[1]
        gp = (ctypes.c_void_p * n)(*[self.gate_ptr(e) for e in experts])
        up = (ctypes.c_void_p * n)(*[self.up_ptr(e) for e in experts])
        dp = (ctypes.c_void_p * n)(*[self.down_ptr(e) for e in experts])
        fm = np.full(n, FMT_Q6K, np.int32)
        rw = np.ascontiguousarray(rw, np.float32)
        p = L.tg_hip_moe_plan_create(ctypes.addressof(gp), ctypes.addressof(up), ctypes.addressof(dp), FMT_Q4K,
                                     fm.ctypes.data, None, None, None, ACT_SILU, n, rw.ctypes.data, k, D, I)
        if not p:
            raise RuntimeError(f"moe plan: {last_error()}")
        return p

    def route(self, k, draft):
        """Top-8 experts and weights of the k normalized rows in self.n."""
        L = self.lib
        if draft:
            L.tg_hip_route_restricted_dev(self.router.ptr, self.bias.ptr, self.n.ptr, k, E, D, TOPK,
                                          self.resident.ptr, self.idx.ptr, self.w.ptr, self.rsc.ptr, None)
        else:
            L.tg_hip_route_dev(self.router.ptr, self.bias.ptr, self.n.ptr, k, E, D, TOPK, self.idx.ptr, self.w.ptr,
                               self.rsc.ptr, None)
        idx = self.idx.download(np.int32, k * TOPK).reshape(k, TOPK)
        w = self.w.download(np.float32, k * TOPK).reshape(k, TOPK)
        return idx, w

    def forward_rows(self, tokens, draft=False):
        """The tokens' rows through the layer and the head; returns the
        argmax token of each row (forward_rows + numpy.argmax of its logits,
        tinygiant/specdec.py:60-77)."""
        L = self.lib
        k = len(tokens)
        if not 1 <= k <= self.max_rows:
            raise ValueError(f"1 <= rows <= {self.max_rows}")
        X = np.stack([embed(self.m["seed"], t) for t in tokens]).astype(np.float32)
        self.x.upload(X)
        L.tg_hip_rms_norm_dev(self.x.ptr, self.ffn_norm.ptr, self.n.ptr, k, D, ctypes.c_float(EPS), None)
        idx, w = self.route(k, draft)
        experts, rw = union_rows(idx, w)
        p = self.plan(experts, rw)
        try:
            L.tg_hip_moe_plan_run(p, self.n.ptr, self.x.ptr, None)    # x += MoE(n)
        finally:
            L.tg_hip_moe_plan_destroy(p)
        L.tg_hip_head_argmax_dev(FMT_Q6K, self.head.ptr, self.x.ptr, self.out_norm.ptr, ctypes.c_float(EPS), k,
                                 self.vocab, D, None, self.am.ptr, self.val.ptr, self.hsc.ptr, None)
        am = self.am.download(np.int32, k)
        err = last_error()
        if err:
            raise RuntimeError(err)
        self.last = {"experts": experts, "idx": idx, "w": w, "rows": k}
        return am

    def verify_round(self, t0, n_draft):
        """One greedy speculative round (tinygiant/specdec.py:57-108): n_draft
        draft passes of one row each, then the exact pass over [t0] + drafts;
        the drafts are accepted while the target argmax agrees, and the
        round emits the accepted drafts plus the target's next token."""
        drafts, draft_experts = [], []
        inp = t0
        for _ in range(n_draft):
            d = int(self.forward_rows([inp], draft=True)[0])
            drafts.append(d)
            draft_experts.append(self.last["experts"])
            inp = d
        target = [int(t) for t in self.forward_rows([t0] + drafts, draft=False)]
        n_acc = 0
        while n_acc < n_draft and target[n_acc] == drafts[n_acc]:
            n_acc += 1
        emitted = drafts[:n_acc] + [target[n_acc]]
        return {"drafts": drafts, "target": target, "accepted": n_acc, "emitted": emitted,
                "union": self.last["experts"], "draft_experts": draft_experts}

    def prepare_pass(self, tokens, draft):
        """Device state of one pass ready to replay: the rows' embeddings
        uploaded and the MoE plan of their routing.  Returns the plan (the
        caller destroys it) and the number of union experts."""
        k = len(tokens)
        X = np.stack([embed(self.m["seed"], t) for t in tokens]).astype(np.float32)
        self.x.upload(X)
        self.lib.tg_hip_rms_norm_dev(self.x.ptr, self.ffn_norm.ptr, self.n.ptr, k, D, ctypes.c_float(EPS), None)
        idx, w = self.route(k, draft)
        experts, rw = union_rows(idx, w)
        return self.plan(experts, rw), len(experts)

    def launch_pass(self, plan, k, draft):
        """One pass's device work, queued on the library stream: RMSNorm,
        routing, the MoE over the planned union (accumulated into the rows),
        and the head with its argmax."""
        L = self.lib
        L.tg_hip_rms_norm_dev(self.x.ptr, self.ffn_norm.ptr, self.n.ptr, k, D, ctypes.c_float(EPS), None)
        if draft:
            L.tg_hip_route_restricted_dev(self.router.ptr, self.bias.ptr, self.n.ptr, k, E, D, TOPK,
                                          self.resident.ptr, self.idx.ptr, self.w.ptr, self.rsc.ptr, None)
        else:
            L.tg_hip_route_dev(self.router.ptr, self.bias.ptr, self.n.ptr, k, E, D, TOPK, self.idx.ptr, self.w.ptr,
                               self.rsc.ptr, None)
        L.tg_hip_moe_plan_run(plan, self.n.ptr, self.x.ptr, None)
        L.tg_hip_head_argmax_dev(FMT_Q6K, self.head.ptr, self.x.ptr, self.out_norm.ptr, ctypes.c_float(EPS), k,
                                 self.vocab, D, None, self.am.ptr, self.val.ptr, self.hsc.ptr, None)

    def free(self):
        for a in (self.experts, self.head, self.router, self.bias, self.ffn_norm, self.out_norm, self.resident,
                  self.x, self.n, self.idx, self.w, self.rsc, self.am, self.val, self.hsc):
            a.free()


def time_passes(layers, tokens, draft, iters=20):
    """Device time of one pass (HIP events on the library stream), the
    passes alternating over `layers` (models of distinct weights, so that
    the bytes a pass reads are not served from the last one's cache): the
    same tokens' routing is planned once per model, then iters passes are
    queued back to back.  Returns (us per pass, weight bytes per pass on
    average: the union's experts, the router and the head)."""
    L = lib()
    k = len(tokens)
    plans, nexp = [], []
    for m in layers:
        p, n = m.prepare_pass(tokens, draft)
        plans.append(p)
        nexp.append(n)
    try:
        for i in range(2 * len(layers)):
            layers[i % len(layers)].launch_pass(plans[i % len(layers)], k, draft)
        L.tg_hip_mark(0)
        for i in range(iters):
            j = i % len(layers)
            layers[j].launch_pass(plans[j], k, draft)
        L.tg_hip_mark(1)
        us = L.tg_hip_marks_ms(0, 1) * 1e3 / iters
        err = last_error()
        if err:
            raise RuntimeError(err)
    finally:
        for p in plans:
            L.tg_hip_moe_plan_destroy(p)
    head = layers[0].head_bytes
    nbytes = float(np.mean([n * EXPERT_B + head + E * D * 4 for n in nexp]))
    return us, nbytes, nexp
