"""Independent pin of the oracle's composed decode step (``orc_step_lanes``).

``Restatement.lane_step`` below is a float64 numpy restatement of one decode step
written from the reference's op order, not from the oracle's code:

  embed            decoder.clj:195-204 (scale sqrt(d) in double, rounded to float;
                   prescaled table decoder_gpu.clj:80-91)
  per layer        decoder.clj:291-345: attn norm -> Q/K/V -> qk-norm (per head)
                   -> RoPE at p with theta per layer (rope-theta :222-227,
                   global-layer? :214-220: layer l is global iff (l+1) % p == 0)
                   -> append -> attention over the visible window (sliding only
                   on local layers, :306-310) -> O -> sandwich post-attn norm ->
                   residual -> pre-FFN norm -> act(gate) * up -> down -> sandwich
                   post-FFN norm -> residual
  head + tail      final norm (:347), tied head (lm-logits :369-373, the head is
                   always the quantised embedding, decoder_gpu.clj:445-455),
                   greedy argmax, next input row = embed(token) (decode-tail!
                   decoder_gpu.clj:73-78)

Everything is float64 except the two quantisers the path defines: weights are
the oracle's packed blocks dequantised exactly, and each linear input is
int8-quantised per 32-block (d = amax/127 rounded up to a 4-bit significand,
q = rint(x/d)) in float64.  The
oracle runs the same descriptors in its f32-KV mode (the reference CPU path's
f32 kc/vc, decoder.clj:304-310) and in the fp16-KV product mode.

Tolerance: the north star's logits bound, max-abs 2e-2 and cosine >= 0.9999,
applied to the logits and to every appended K/V row.  Why the faithful
restatement sits well inside it: the two sides differ by fp32 rounding (~1e-7
relative) plus, rarely, an activation element whose fp32 and float64 values
straddle an int8 quantisation boundary.  One such flip moves every output of
that linear by d_x * w (d_x = amax/127 of its block, |w| <= 8 d_w), ~1e-3 of
the output scale here, and what it perturbs downstream is bounded by the
activation quantisation noise itself (~1/254 of an element, averaged over the
dot product); fp16 KV adds half an fp16 ulp per appended element.  Measured:
at most 8.3e-3 (Gemma flags, fp16 KV), 5e-4 or less otherwise.  Each mutation
below (a plausible op-order mistake) must miss the bound by at least three
times (measured: 8.7x for the mildest, swapping qk-norm and RoPE), which shows
the check bites.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle as O
from lanes import Routes
from rstr import configs

TOL = 2e-2      # max-abs, logits and K/V rows
COS = 0.9999


# ---- float64 building blocks ------------------------------------------------------

def dequant(wq: np.ndarray, ws: np.ndarray, bits: int) -> np.ndarray:
    """Packed blocks -> float64 [n][k]: Q4 byte j = q[2j] | q[2j+1] << 4, value q - 8;
    Q8 int8 q; times the fp16 block scale."""
    n, nb = ws.shape
    if bits == 4:
        q = np.stack([wq & 15, wq >> 4], -1).reshape(n, nb, 32).astype(np.float64) - 8.0
    else:
        q = wq.reshape(n, nb, 32).astype(np.float64)
    return (q * ws.view(np.float16).astype(np.float64)[..., None]).reshape(n, nb * 32)


def quant_act64(x: np.ndarray) -> np.ndarray:
    """Per-32-block symmetric int8 of a float64 row (decoder.clj:206-213), dequantised;
    the block scale is amax/127 rounded up to a 4-bit significand, kept in
    [2^-21, 480]."""
    b = x.reshape(-1, 32)
    a = np.abs(b).max(-1, keepdims=True) / 127.0
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    d = np.ceil(a / 2.0 ** (e - 3)) * 2.0 ** (e - 3)
    d = np.where(a > 0, np.clip(d, 2.0 ** -21, 480.0), 0.0)
    q = np.where(d > 0, np.clip(np.rint(b / np.where(d > 0, d, 1.0)), -127, 127), 0.0)
    return (q * d).reshape(x.shape)


def rms64(x: np.ndarray, g: np.ndarray, goff: float, eps: float) -> np.ndarray:
    """RMSNorm over the last axis: x / sqrt(mean(x^2) + eps) * (goff + g)."""
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * (goff + g.astype(np.float64))


def rope64(x: np.ndarray, pos: int, theta: float) -> np.ndarray:
    """HF rotate-half RoPE of [heads][hd] at absolute position pos, angles in float64."""
    hd = x.shape[-1]
    h = hd // 2
    ang = pos * theta ** (-2.0 * np.arange(h) / hd)
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[..., :h], x[..., h:]
    return np.concatenate([a * c - b * s, b * c + a * s], -1)


def gelu64(g):
    return 0.5 * g * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (g + 0.044715 * g ** 3)))


def silu64(g):
    return g / (1.0 + np.exp(-g))


# ---- the restatement ----------------------------------------------------------------

class Restatement:
    """Weights of an oracle model, dequantised once; ``mutate`` names one planted
    op-order mistake (None for the faithful restatement)."""

    def __init__(self, om: "O.Model", cfg: dict, mutate: str | None = None):
        self.cfg, self.mutate, self.om = cfg, mutate, om
        bits = cfg["weight_bits"]
        self.W = {}
        for l in range(cfg["n_layers"]):
            for role in ("q", "k", "v", "o", "gate", "up", "down"):
                self.W[(l, role)] = dequant(*om.tensor(l, role), bits)
        self.W[(-1, "embed")] = dequant(*om.tensor(-1, "embed"), bits)
        self.N = {}
        for l in range(cfg["n_layers"]):
            for role in ("attn_norm", "ffn_pre_norm", "q_norm", "k_norm", "post_attn_norm", "ffn_post_norm"):
                try:
                    self.N[(l, role)] = om.norm(l, role).astype(np.float64)
                except KeyError:
                    pass
        self.N[(-1, "final_norm")] = om.norm(-1, "final_norm").astype(np.float64)
        self.key = O.tensor_key(om.seed, -1, O.ROLE["embed"])

    def embed_source(self, token: int) -> np.ndarray:
        """The embedding row as bound (f32, before any scale)."""
        d = self.cfg["d_model"]
        return O.normal(self.key, token * d, d, 0.0, 0.02)

    def embed(self, token: int) -> np.ndarray:
        """decoder.clj:195-204: (float) (scale * (double) e), scale sqrt(d) or 1."""
        e = self.embed_source(token).astype(np.float64)
        scale = math.sqrt(self.cfg["d_model"]) if self.cfg["embed_scale_sqrt_d"] else 1.0
        if self.mutate == "drop_embed_scale":
            scale = 1.0
        return (scale * e).astype(np.float32)

    def global_layer(self, l: int) -> bool:
        p = self.cfg["global_pattern"]
        if p <= 0:
            return True
        if self.mutate == "flip_global":
            return l % p == 0
        return (l + 1) % p == 0

    def lin(self, l, role, x):
        return self.W[(l, role)] @ quant_act64(x)

    def lane_step(self, token, pos, length, page_row, ps, kslabs, vslabs, kv_f16=False):
        """One step of one lane.  kslabs/vslabs[l]: the pool before the step as
        float64 [pages][ps][n_kv][hd]; the lane's visible route is tokens
        [0, length) of page_row, the last one being this step's own row, which
        is rounded to fp16 before attending when the pool holds fp16
        (paged_append.clj:44-57).  length 0 is an inactive lane: an empty route
        whose attention output is 0 and which appends nothing; its row still
        runs through the layers and the tail (the whole batch does,
        paged_decoder.clj:562-578).  Returns (logits, K rows, V rows)."""
        c, mu = self.cfg, self.mutate
        n_q, n_kv, hd, eps = c["n_q"], c["n_kv"], c["head_dim"], c["eps"]
        goff = 1.0 if c["gain_offset"] else 0.0
        x = self.embed(token).astype(np.float64)
        krows, vrows = [], []
        for l in range(c["n_layers"]):
            glob = self.global_layer(l)
            theta = c["rope_local"] if (c["rope_dual"] and not glob) else c["rope_global"]
            window = c["sliding_window"] if (c["sliding_window"] > 0 and not glob) else 0
            if mu == "no_window":
                window = 0
            h = rms64(x, self.N[(l, "attn_norm")], goff, eps)
            q = self.lin(l, "q", h).reshape(n_q, hd)
            k = self.lin(l, "k", h).reshape(n_kv, hd)
            v = self.lin(l, "v", h).reshape(n_kv, hd)
            if c["qk_norm"] and mu == "swap_qknorm_rope":
                q = rms64(rope64(q, pos, theta), self.N[(l, "q_norm")], goff, eps)
                k = rms64(rope64(k, pos, theta), self.N[(l, "k_norm")], goff, eps)
            else:
                if c["qk_norm"]:
                    q = rms64(q, self.N[(l, "q_norm")], goff, eps)
                    k = rms64(k, self.N[(l, "k_norm")], goff, eps)
                q = rope64(q, pos, theta)
                k = rope64(k, pos, theta)
            if kv_f16:
                k = k.astype(np.float16).astype(np.float64)
                v = v.astype(np.float16).astype(np.float64)
            krows.append(k.reshape(-1))
            vrows.append(v.reshape(-1))
            att = np.zeros((n_q, hd))
            if length > 0:
                lo = max(0, length - window) if window else 0
                ks = np.stack([kslabs[l][page_row[t // ps], t % ps] for t in range(lo, length - 1)] + [k])
                vs = np.stack([vslabs[l][page_row[t // ps], t % ps] for t in range(lo, length - 1)] + [v])
                scale = float(np.float32(c["attn_scale"]))
                G = n_q // n_kv
                for hq in range(n_q):
                    s = ks[:, hq // G] @ q[hq] * scale
                    w = np.exp(s - s.max())
                    att[hq] = (w / w.sum()) @ vs[:, hq // G]
            o = self.lin(l, "o", att.reshape(-1))
            if c["sandwich"] and mu != "drop_post_attn_norm":
                o = rms64(o, self.N[(l, "post_attn_norm")], goff, eps)
            x = (h if mu == "residual_from_norm" else x) + o
            f = rms64(x, self.N[(l, "ffn_pre_norm")], goff, eps)
            g, u = self.lin(l, "gate", f), self.lin(l, "up", f)
            if mu == "swap_gate_up":
                g, u = u, g
            act = gelu64(g) if c["ffn_geglu"] else silu64(g)
            dn = self.lin(l, "down", act * u)
            if c["sandwich"]:
                dn = rms64(dn, self.N[(l, "ffn_post_norm")], goff, eps)
            x = x + dn
        fin = rms64(x, self.N[(-1, "final_norm")], goff, eps)
        return self.lin(-1, "embed", fin), krows, vrows


# ---- driving the oracle and the restatement over the same descriptors -----------------

CASES = {
    # model, bits, lanes, restored prefix per lane, active lanes per step
    "tiny_gemma": (4, 4, [9, 30, 2, 51], [[0, 1, 2, 3], [0, 1, 3], [2, 3], [0, 1, 2, 3]]),
    "tiny_qwen": (8, 3, [5, 40, 17], [[0, 1, 2], [0, 2], [1], [0, 1, 2]]),
    "tiny_llama": (4, 3, [12, 33, 7], [[0, 1, 2], [1, 2], [0], [0, 1, 2]]),
}
PS, PAGES, PPS, MAXPOS, SPLIT, SEED, KV_SEED = 16, 40, 6, 128, 16, 3, 17


def _err(got, want):
    return float(np.max(np.abs(got - want)))


def _cos(a, b):
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def run_case(name: str, kv_f16: bool, mutate: str | None = None):
    """Returns (worst K/V max-abs error, worst logits max-abs error, worst logits
    cosine, token agreements) over every lane of every step."""
    bits, B, prefix, sched = CASES[name]
    cfg = configs.with_bits(configs.MODELS[name], bits)
    om = O.Model(cfg, seed=SEED)
    od = O.Decoder(om, B, PS, PAGES, PPS, MAXPOS, kv_f16=kv_f16, split=SPLIT)
    rs = Restatement(om, cfg, mutate)
    routes = Routes(B, PS, PAGES, PPS, seed=SEED)
    worst_kv = worst_lg = 0.0
    worst_cos = 1.0
    agree = []
    try:
        for b, n in enumerate(prefix):
            for pg in routes.prefix(b, n):
                od.fill_synthetic(pg, KV_SEED)
        toks = np.array([(37 * b + 5) % cfg["vocab"] for b in range(B)], np.int32)
        od.prime_lanes(np.arange(B), toks)
        if mutate is None:
            assert np.array_equal(od.r0(), np.stack([rs.embed(int(t)) for t in toks]))
        for active in sched:
            before = [(od.slab(0, l).astype(np.float64), od.slab(1, l).astype(np.float64))
                      for l in range(cfg["n_layers"])]
            desc = routes.step(active)
            out = od.step_lanes(**desc)
            logits = od.logits()
            for b in range(B):
                L = int(desc["lengths"][b])
                lg, krows, vrows = rs.lane_step(int(toks[b]), int(desc["positions"][b]), L,
                                                desc["page_table"][b], PS,
                                                [s[0] for s in before], [s[1] for s in before], kv_f16)
                slot = int(desc["slots"][b])
                for l in range(cfg["n_layers"] if L > 0 else 0):
                    ko = od.slab(0, l).reshape(-1, cfg["n_kv"] * cfg["head_dim"])[slot].astype(np.float64)
                    vo = od.slab(1, l).reshape(-1, cfg["n_kv"] * cfg["head_dim"])[slot].astype(np.float64)
                    worst_kv = max(worst_kv, _err(ko, krows[l]), _err(vo, vrows[l]))
                worst_lg = max(worst_lg, _err(logits[b].astype(np.float64), lg))
                worst_cos = min(worst_cos, _cos(logits[b].astype(np.float64), lg))
                agree.append(int(out[b]) == int(np.argmax(lg)))
                if mutate is None:
                    # the tail: the next input row is the prescaled embedding of the token
                    assert np.array_equal(od.r0()[b], rs.embed(int(out[b])))
                toks[b] = out[b]
    finally:
        od.close()
        om.close()
    return worst_kv, worst_lg, worst_cos, agree


@pytest.mark.parametrize("kv_f16", [False, True])
@pytest.mark.parametrize("name", list(CASES))
def test_oracle_step_matches_float64_restatement(name, kv_f16):
    kv, lg, cos, agree = run_case(name, kv_f16)
    assert kv <= TOL, kv
    assert lg <= TOL, lg
    assert cos >= COS, cos
    assert all(agree), agree


MUTATIONS = {
    "tiny_gemma": ["swap_qknorm_rope", "drop_post_attn_norm", "flip_global", "drop_embed_scale",
                   "no_window", "swap_gate_up", "residual_from_norm"],
    "tiny_qwen": ["swap_qknorm_rope", "swap_gate_up", "residual_from_norm"],
    "tiny_llama": ["swap_gate_up", "residual_from_norm"],
}


@pytest.mark.parametrize("name,mutate", [(n, m) for n, ms in MUTATIONS.items() for m in ms])
def test_planted_op_order_mistakes_fail_the_bound(name, mutate):
    """Each plausible mistake, planted in the restatement, misses the tolerance by
    at least 3x against the oracle: the float64 check would catch the same
    mistake in the oracle (and, through the bit-exact GPU tests, in the kernels)."""
    kv, lg, cos, _ = run_case(name, kv_f16=False, mutate=mutate)
    assert max(kv, lg) >= 3 * TOL, (mutate, kv, lg, cos)


def test_head_is_the_quantised_embedding():
    """The tied head (decoder_gpu.clj:445-455) is the block quantisation of the
    same embedding table the input rows are gathered from."""
    for name, bits in (("tiny_gemma", 4), ("tiny_qwen", 8)):
        cfg = configs.with_bits(configs.MODELS[name], bits)
        om = O.Model(cfg, seed=SEED)
        try:
            rs = Restatement.__new__(Restatement)
            rs.cfg, rs.mutate, rs.om = cfg, None, om
            rs.key = O.tensor_key(om.seed, -1, O.ROLE["embed"])
            emb = np.stack([rs.embed_source(t) for t in range(cfg["vocab"])])
            want = O.quant_q4(emb) if bits == 4 else O.quant_q8(emb)
            got = om.tensor(-1, "embed")
            assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
        finally:
            om.close()
