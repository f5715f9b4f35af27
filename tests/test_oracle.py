"""Pins of the CPU oracle (``oracle/rstr_oracle.c``) against the reference's own
known answers and against what the mathematics fixes.  None of these retypes
the oracle's formula: each compares it with an independent source -- IEEE
conversions in numpy, float64 closed forms, brute force, or the literal
values of the reference tests -- chosen so that a plausible mistake (a dropped
term, a wrong sign, a transposed operand, a wrong RoPE pairing, an off-by-one
window) fails at least one of them.
"""
import math

import numpy as np
import pytest

import oracle as O

RNG = np.random.default_rng(1234)


# ---- IEEE half conversions --------------------------------------------------

def test_f16_to_f32_matches_ieee_for_every_bit_pattern():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([O.lib().orc_f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rounds_to_nearest_even():
    edge = np.array([0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.1e-5, 5.96e-8, 2.98e-8,
                     2.99e-8, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 2049.0, 2051.0, np.inf, -np.inf], np.float32)
    mags = np.exp(RNG.uniform(np.log(1e-9), np.log(7e4), 200_000)).astype(np.float32)
    x = np.concatenate([edge, mags * RNG.choice([-1.0, 1.0], mags.size).astype(np.float32)])
    got = O.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---- transcendental helpers ------------------------------------------------

def _ulp_err(got: np.ndarray, want64: np.ndarray) -> np.ndarray:
    want = want64.astype(np.float32)
    ulp = np.spacing(np.abs(want)).astype(np.float64)
    return np.abs(got.astype(np.float64) - want64) / ulp


def test_exp_within_two_ulp_of_correctly_rounded():
    x = np.concatenate([RNG.uniform(-87.0, 88.0, 20_000), RNG.uniform(-1.0, 1.0, 5_000),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 88.7, -87.3])]).astype(np.float32)
    got = np.array([O.exp(float(v)) for v in x], np.float32)
    err = _ulp_err(got, np.exp(x.astype(np.float64)))
    assert err.max() <= 2.0, err.max()
    assert O.exp(0.0) == 1.0
    assert O.exp(89.0) == math.inf
    assert O.exp(-104.0) == 0.0
    assert math.isnan(O.exp(math.nan))


def test_gelu_tanh_and_silu_against_float64_closed_forms():
    g = np.concatenate([RNG.uniform(-10, 10, 4000), np.linspace(-0.1, 0.1, 101)]).astype(np.float32)
    gelu = np.array([O.lib().orc_gelu_tanh(float(v)) for v in g], np.float64)
    silu = np.array([O.lib().orc_silu(float(v)) for v in g], np.float64)
    g64 = g.astype(np.float64)
    gelu64 = 0.5 * g64 * (1 + np.tanh(math.sqrt(2 / math.pi) * (g64 + 0.044715 * g64 ** 3)))
    silu64 = g64 / (1 + np.exp(-g64))
    # fp32 evaluation: absolute error below 2.5e-7 * max(1, |g|) (the erf form
    # of GELU differs from the tanh form by up to ~1e-3)
    bound = 2.5e-7 * np.maximum(1.0, np.abs(g64))
    assert (np.abs(gelu - gelu64) <= bound).all()
    assert (np.abs(silu - silu64) <= bound).all()
    assert O.lib().orc_gelu_tanh(0.0) == 0.0 and O.lib().orc_silu(0.0) == 0.0


# ---- synthetic weights --------------------------------------------------------

def test_splitmix64_published_sequence():
    """Vigna's splitmix64 from state 0 emits 0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4."""
    g = 0x9E3779B97F4A7C15
    assert O.lib().orc_splitmix64(0) == 0xE220A8397B1DCDAF
    assert O.lib().orc_splitmix64(g) == 0x6E789E6AA1B965F4


def test_synthetic_normal_moments_and_support():
    x = O.normal(O.tensor_key(7, 0, 3), 0, 1_000_000, 0.0, 1.0).astype(np.float64)
    assert abs(x.mean()) < 5e-3 and abs(x.std() - 1.0) < 5e-3
    assert np.abs(x).max() <= 6.0


# ---- weight and activation quantisation -----------------------------------------

def test_q4_ggml_known_block_and_bounds():
    """GGML Q4_0 rule: d = (signed max-magnitude)/-8, q = min(15, trunc(w/d + 8.5))."""
    w = np.concatenate([np.arange(-8, 8), np.arange(-8, 8)]).astype(np.float32)[None, :]
    nib, sc = O.quant_q4(w)
    q = np.stack([nib[0, 0] & 15, nib[0, 0] >> 4], 1).ravel()
    assert np.array_equal(q, np.concatenate([np.arange(16), np.arange(16)]))
    assert np.float16(1.0).view(np.uint16) == sc[0, 0]
    w = RNG.standard_normal((64, 256)).astype(np.float32)
    nib, sc = O.quant_q4(w)
    q = np.stack([nib & 15, nib >> 4], -1).reshape(64, 8, 32).astype(np.float64) - 8
    d = sc.view(np.float16).astype(np.float64)[:, :, None]
    err = np.abs(w.reshape(64, 8, 32) - q * d)
    assert (err <= np.abs(d) * 1.001 + 1e-12).all()
    top = np.abs(w.reshape(64, 8, 32)).argmax(-1)
    assert (np.take_along_axis(q, top[..., None], -1) == -8).all()
    nib, sc = O.quant_q4(np.zeros((1, 32), np.float32))
    assert sc[0, 0] == 0 and ((nib & 15) == 8).all() and ((nib >> 4) == 8).all()


def test_symmetric_int8_q8_block_quantisation():
    w = (RNG.standard_normal((32, 256)) * RNG.uniform(0.01, 10, (32, 1))).astype(np.float32)
    q, sc = O.quant_q8(w)
    d = sc.view(np.float16).astype(np.float64)
    q = q.reshape(32, 8, 32)
    assert np.abs(q).max() <= 127
    wb = w.reshape(32, 8, 32).astype(np.float64)
    top = np.abs(wb).argmax(-1)
    assert (np.abs(np.take_along_axis(q, top[..., None], -1)) == 127).all()
    assert (np.abs(wb - q * d[..., None]) <= 0.6 * d[..., None] + 1e-12).all()
    zq, zs = O.quant_q8(np.zeros((1, 32), np.float32))
    assert (zq == 0).all() and np.asarray(zs).view(np.uint8).max() == 0


def _prev4(d: float) -> float:
    """The largest value below d with a 4-bit significand (d itself has one)."""
    e = math.floor(math.log2(d))
    return d - 2.0 ** (e - 4) if d == 2.0 ** e else d - 2.0 ** (e - 3)


def test_activation_scale_rounding():
    """The activation block scale is the smallest value with a 4-bit significand
    that is >= RN(amax/127), kept in [2^-21, 480]; every q*d with |q| <= 127 is
    then exact in fp16 (the property the linear relies on)."""
    amax = np.concatenate([np.exp(RNG.uniform(np.log(1e-9), np.log(1e5), 20000)),
                           [1e-30, 2.0 ** -21 * 127, 127.0, 60960.0, 1e6, 0.0]]).astype(np.float32)
    for a in amax:
        d = O.lib().orc_act_scale(float(a))
        if a == 0:
            assert d == 0.0
            continue
        base = float(np.float32(a) / np.float32(127))
        assert 2.0 ** -21 <= d <= 480.0
        m = d / 2.0 ** math.floor(math.log2(d)) * 8
        assert m == int(m) and 8 <= m <= 15, (a, d)               # 4 significant bits
        if 2.0 ** -21 < base <= 480.0:
            assert _prev4(d) < base <= d                               # the smallest such value
            assert d < base * 1.125 + 1e-300
        q = np.arange(-127, 128, dtype=np.float64)
        assert np.array_equal(np.float16(q * d).astype(np.float64), q * d), d
    assert O.lib().orc_act_scale(1e-30) == 2.0 ** -21
    assert O.lib().orc_act_scale(1e6) == 480.0


def test_activation_block_quantisation():
    x = (RNG.standard_normal((32, 256)) * RNG.uniform(0.01, 10, (32, 1))).astype(np.float32)
    q, d = O.quant_act(x)
    q = q.reshape(32, 8, 32).astype(np.float64)
    d = d.astype(np.float64)
    xb = x.reshape(32, 8, 32).astype(np.float64)
    assert np.abs(q).max() <= 127
    top = np.abs(xb).argmax(-1)
    qt = np.abs(np.take_along_axis(q, top[..., None], -1))
    assert (qt >= 112).all() and (qt <= 127).all()    # the scale exceeds amax/127 by < 1/8
    assert (np.abs(xb - q * d[..., None]) <= 0.5 * d[..., None] * (1 + 1e-6)).all()
    zq, zs = O.quant_act(np.zeros((1, 32), np.float32))
    assert (zq == 0).all() and np.asarray(zs).view(np.uint8).max() == 0


def test_qlinear_single_block_is_exact_and_matches_float64():
    """One nonzero block: y = fmaf(isum*dx, dw, 0) = RN(isum * dx * dw) exactly
    (isum*dx is exact).  Random: float64."""
    k = 128
    w = np.zeros((16, k), np.float32)
    x = np.zeros((3, k), np.float32)
    w[:, 64:96] = RNG.standard_normal((16, 32))
    x[:, 64:96] = RNG.standard_normal((3, 32))
    for bits in (4, 8):
        wq, ws = O.quant_q4(w) if bits == 4 else O.quant_q8(w)
        xq, xs = O.quant_act(x)
        y = O.qlinear(bits, wq, ws, xq, xs)
        wint = (np.stack([wq & 15, wq >> 4], -1).reshape(16, k).astype(np.int64) - 8) if bits == 4 \
            else wq.reshape(16, k).astype(np.int64)
        isum = xq.astype(np.int64)[:, 64:96] @ wint[:, 64:96].T
        exact = isum.astype(np.float64) * xs[:, 2].astype(np.float64)[:, None] \
            * ws.view(np.float16)[:, 2].astype(np.float64)[None, :]      # <= 30 significant bits
        assert np.array_equal(y, exact.astype(np.float32))
    # general case vs float64 (dropped blocks, a transposed operand or a sign
    # error are far outside this tolerance)
    w = RNG.standard_normal((24, 512)).astype(np.float32)
    x = RNG.standard_normal((5, 512)).astype(np.float32)
    for bits in (4, 8):
        wq, ws = O.quant_q4(w) if bits == 4 else O.quant_q8(w)
        xq, xs = O.quant_act(x)
        y = O.qlinear(bits, wq, ws, xq, xs)
        wint = (np.stack([wq & 15, wq >> 4], -1).reshape(24, 512).astype(np.float64) - 8) if bits == 4 \
            else wq.reshape(24, 512).astype(np.float64)
        wd = (wint.reshape(24, 16, 32) * ws.view(np.float16).astype(np.float64)[..., None]).reshape(24, 512)
        xd = (xq.astype(np.float64).reshape(5, 16, 32) * xs.astype(np.float64)[..., None]).reshape(5, 512)
        y64 = xd @ wd.T
        assert np.allclose(y, y64, rtol=1e-5, atol=1e-5 * np.abs(y64).max())


# ---- RMSNorm and RoPE ------------------------------------------------------------

def test_rmsnorm_closed_forms():
    n, eps = 256, 1e-6
    for c in (0.5, 3.0, -2.0):
        y = O.rmsnorm(np.full((1, n), c, np.float32), np.zeros(n, np.float32), 1.0, eps)
        assert np.allclose(y, c / math.sqrt(c * c + eps), rtol=3e-7)
    x = np.arange(1, 257, dtype=np.float32)[None, :]
    assert O.lib().orc_sumsq(O.ptr(np.ascontiguousarray(x)), 256) == float(sum(i * i for i in range(1, 257)))
    x = RNG.standard_normal((4, 640)).astype(np.float32)
    g = RNG.standard_normal(640).astype(np.float32) * 0.02
    for goff in (0.0, 1.0):
        y = O.rmsnorm(x, g, goff, eps)
        x64 = x.astype(np.float64)
        y64 = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + eps) * (goff + g.astype(np.float64))
        assert np.allclose(y, y64, rtol=2e-6, atol=1e-7)


def test_rope_identity_norms_and_rotate_half_pairing():
    hd, theta = 128, 10000.0
    cos_t, sin_t = O.rope_table(theta, hd, 64)
    x = RNG.standard_normal((3, 2, hd)).astype(np.float32)
    assert np.array_equal(O.rope(x, [0, 0, 0], cos_t, sin_t), x)
    pos = [5, 17, 63]
    y = O.rope(x, pos, cos_t, sin_t).astype(np.float64)
    h = hd // 2
    n_in = x[..., :h].astype(np.float64) ** 2 + x[..., h:].astype(np.float64) ** 2
    n_out = y[..., :h] ** 2 + y[..., h:] ** 2
    assert np.allclose(n_in, n_out, rtol=1e-5)
    e = np.zeros((1, 1, hd), np.float32)
    e[0, 0, 1] = 1.0
    p = 9
    y = O.rope(e, [p], cos_t, sin_t)[0, 0]
    ang = p * theta ** (-2.0 / hd)
    assert abs(y[1] - math.cos(ang)) < 1e-6 and abs(y[1 + h] - math.sin(ang)) < 1e-6
    assert np.count_nonzero(y) == 2, "HF rotate-half pairs dim i with dim i + head_dim/2"


# ---- attention ----------------------------------------------------------------------

def _pages(rows_per_lane, hd=8, ps=2, n_kv=1):
    """Lay lanes' K/V rows into consecutive pages; returns kpages, vpages, table, lengths."""
    npages = sum(-(-len(r[0]) // ps) for r in rows_per_lane) + 1
    kp = np.zeros((npages, ps, n_kv, hd), np.float16)
    vp = np.zeros_like(kp)
    pps = max(-(-len(r[0]) // ps) for r in rows_per_lane)
    table = -np.ones((len(rows_per_lane), pps), np.int32)
    nxt = 0
    for b, (ks, vs) in enumerate(rows_per_lane):
        for t, (k, v) in enumerate(zip(ks, vs)):
            if t % ps == 0:
                table[b, t // ps] = nxt
                nxt += 1
            kp[table[b, t // ps], t % ps, 0, :len(k)] = k
            vp[table[b, t // ps], t % ps, 0, :len(v)] = v
    return kp, vp, table, np.array([len(r[0]) for r in rows_per_lane], np.int32)


def test_attention_reference_known_answer():
    """continuation_paged_attention_device_test.clj:42-174: lane a holds
    K=[[1,0],[0,1]], V=[[10,20],[30,40]]; lane b holds K=[[1,1]], V=[[5,7]];
    q=[1,0], scale 1/sqrt(2) -> [16.6048 26.6048] and [5 7]; window-left 0
    (only the current token visible) -> [30 40] and [5 7]."""
    kp, vp, table, lengths = _pages([([[1, 0], [0, 1]], [[10, 20], [30, 40]]), ([[1, 1]], [[5, 7]])])
    q = np.zeros((2, 1, 8), np.float32)
    q[:, 0, 0] = 1.0
    for split in (256, 4):
        out = O.attention(q, kp, vp, table, lengths, 0, 1 / math.sqrt(2), split)
        assert np.allclose(out[0, 0, :2], [16.6048, 26.6048], atol=1e-4)
        assert np.allclose(out[1, 0, :2], [5.0, 7.0], atol=1e-6)
    out = O.attention(q, kp, vp, table, lengths, 1, 1 / math.sqrt(2), 256)
    assert out[0, 0, :2].tolist() == [30.0, 40.0] and out[1, 0, :2].tolist() == [5.0, 7.0]


def _attn64(q, ks, vs, scale):
    s = (ks.astype(np.float64) @ q.astype(np.float64)) * scale
    p = np.exp(s - s.max())
    return (p[:, None] * vs.astype(np.float64)).sum(0) / p.sum()


@pytest.mark.parametrize("window", [0, 2, 4])
def test_attention_brute_force_and_sliding_window(window):
    """Window w keeps the last w tokens (decoder_test.clj:6-34 compaction;
    window-left = size-1, continuation_paged_decoder_test.clj:110-125)."""
    hd, G, n_kv, ps = 16, 2, 2, 4
    lens = [1, 6, 9]
    ks = [RNG.standard_normal((n, n_kv, hd)).astype(np.float16) for n in lens]
    vs = [RNG.standard_normal((n, n_kv, hd)).astype(np.float16) for n in lens]
    pps = -(-max(lens) // ps)
    table = -np.ones((len(lens), pps), np.int32)
    P = sum(-(-n // ps) for n in lens)
    perm = RNG.permutation(P)
    kp = np.zeros((P, ps, n_kv, hd), np.float16)
    vp = np.zeros_like(kp)
    c = 0
    for b, n in enumerate(lens):
        for pg in range(-(-n // ps)):
            table[b, pg] = perm[c]
            c += 1
        for t in range(n):
            kp[table[b, t // ps], t % ps] = ks[b][t]
            vp[table[b, t // ps], t % ps] = vs[b][t]
    q = RNG.standard_normal((len(lens), n_kv * G, hd)).astype(np.float32)
    scale = 0.3
    for split in (256, 4):
        out = O.attention(q, kp, vp, table, np.array(lens, np.int32), window, scale, split)
        for b, n in enumerate(lens):
            lo = max(0, n - window) if window else 0
            for h in range(n_kv * G):
                want = _attn64(q[b, h], ks[b][lo:, h // G], vs[b][lo:, h // G], scale)
                assert np.allclose(out[b, h], want, rtol=2e-5, atol=2e-6)


def test_attention_empty_route_outputs_zero():
    kp, vp, table, lengths = _pages([([[1, 0]], [[3, 4]]), ([[1, 0]], [[3, 4]])])
    lengths[1] = 0
    out = O.attention(np.ones((2, 1, 8), np.float32), kp, vp, table, lengths, 0, 1.0, 256)
    assert (out[1] == 0).all()


# ---- greedy tail ----------------------------------------------------------------------

def test_argmax_reference_known_answer():
    """decoder_gpu_composition_test.clj:9-20: ties and multiple NaNs both select
    the lowest matching column."""
    logits = np.array([[1.0, 5.0, 5.0, 2.0], [9.0, np.nan, 8.0, np.nan]], np.float32)
    assert O.argmax_rows(logits).tolist() == [1, 1]
    assert O.argmax_rows(np.array([[-np.inf, -np.inf, -1.0]], np.float32)).tolist() == [2]


def test_host_tensor_model_equals_the_synthetic_model():
    """``Model.set_tensor`` (host f32 tensors: a checkpoint's) quantises and
    stores exactly as the synthetic build does: a model whose every tensor is
    set to the synthetic generator's f32 values equals the synthetic model in
    packed weights, norms, embedding rows and a decode step's logits."""
    from rstr import configs
    cfg = configs.TINY_GEMMA
    syn = O.Model(cfg, seed=4)
    host = O.Model(cfg, seed=99)
    try:
        roles = ["q", "k", "v", "o", "gate", "up", "down", "attn_norm", "ffn_pre_norm", "q_norm", "k_norm",
                 "post_attn_norm", "ffn_post_norm"]
        for layer in list(range(cfg["n_layers"])) + [-1]:
            for role in (roles if layer >= 0 else ["embed", "final_norm"]):
                key = O.tensor_key(4, layer, O.ROLE[role])
                if role.endswith("norm"):
                    n = cfg["head_dim"] if role in ("q_norm", "k_norm") else cfg["d_model"]
                    vals = O.normal(key, 0, n, 0.0 if cfg["gain_offset"] else 1.0, 0.02)
                else:
                    n, k = O.linear_shape(cfg, role)
                    vals = O.normal(key, 0, n * k, 0.0, 0.02)
                host.set_tensor(layer, role, vals)
        with pytest.raises(ValueError):
            host.set_tensor(0, "q", np.zeros(5, np.float32))
        for layer in range(cfg["n_layers"]):
            for role in ("q", "k", "v", "o", "gate", "up", "down"):
                for a, b in zip(syn.tensor(layer, role), host.tensor(layer, role)):
                    assert np.array_equal(a, b), (layer, role)
            for role in roles[7:]:
                assert np.array_equal(syn.norm(layer, role), host.norm(layer, role))
        for a, b in zip(syn.tensor(-1, "embed"), host.tensor(-1, "embed")):
            assert np.array_equal(a, b)
        for tok in (0, 5, cfg["vocab"] - 1):
            assert np.array_equal(syn.embed_row(tok), host.embed_row(tok))
        outs = []
        for m in (syn, host):
            d = O.Decoder(m, 1, 16, 2, 2, 32, kv_f16=True, split=16)
            d.prime_lanes([0], [9])
            d.step_lanes([0], [0, 1], [0], [0, -1], [1], [0])
            outs.append(d.logits())
            d.close()
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    finally:
        syn.close()
        host.close()
