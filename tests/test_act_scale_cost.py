"""The cost of this build's activation block scale, on record (CPU only).

The reference int8-quantises every linear's input per 32-block with
d = amax/127 (``qlinear-i8``, decoder.clj:206-213; Raster's exact rule is
parity unpinned).  This build rounds d up to a 4-bit significand and keeps it in
[2^-21, 480] so that q*d is an exact fp16 MFMA operand.  Three deviations follow,
each pinned here:

1. the quantisation step is up to 2^-4 coarser (|q_max| in [112, 127]);
2. blocks with amax above 127*480 = 60960 saturate: q = +-127, the block
   dequantises to +-60960 instead of its own values;
3. blocks with amax below 2^-22 quantise to all zeros (below ~6e-5 they keep
   fewer than 7 bits), where amax/127 keeps full precision.

``test_config1_scale_cost_teacher_forced`` measures (1) end to end on
BASELINE.json configs[0] (Gemma-3-270M-shaped Q8, 32-token prompt, 64 greedy
tokens) with the oracle's measurement hook ``orc_set_act_scale_plain``: logits of
the 4-bit-significand scale against the plain scale on the same token sequence."""
import numpy as np

import oracle as O
from lanes import Routes
from rstr import configs

CFG = configs.with_bits(configs.GEMMA3_270M, 8)
PS, MAXPOS, SPLIT = 16, 112, 64
PPS = MAXPOS // PS


def test_blocks_above_the_scale_range_saturate():
    """amax 1e5 > 60960: d clamps to 480, q saturates at +-127 where |x| > 60960, so
    the block dequantises to +-60960 there; the plain scale keeps the block."""
    x = np.zeros((1, 64), np.float32)
    x[0, :32] = np.linspace(-1e5, 1e5, 32, dtype=np.float32)
    x[0, 32:] = np.linspace(-1.0, 1.0, 32, dtype=np.float32)
    q, d = O.quant_act(x)
    assert d[0, 0] == 480.0
    deq = q[0, :32].astype(np.float64) * 480.0
    big = np.abs(x[0, :32]) > 60960
    assert big.sum() == 14
    assert np.array_equal(deq[big], np.sign(x[0, :32][big]) * 60960.0)
    assert (np.abs(deq[~big] - x[0, :32][~big]) <= 240.0).all()
    O.lib().orc_set_act_scale_plain(1)
    try:
        qp, dp = O.quant_act(x)
    finally:
        O.lib().orc_set_act_scale_plain(0)
    assert dp[0, 0] == np.float32(np.float32(1e5) / np.float32(127))
    assert (np.abs(qp[0, :32].astype(np.float64) * dp[0, 0] - x[0, :32]) <= 0.5 * dp[0, 0] * (1 + 1e-6)).all()


def test_blocks_below_the_scale_range_vanish():
    """amax 1e-8 < 2^-22: d clamps up to 2^-21 and every q rounds to 0; at amax
    1e-6 the block keeps about 2 of its 7 bits (|q| <= 2); the plain scale keeps
    |q_max| = 127 in both."""
    x = np.zeros((1, 128), np.float32)
    x[0, :32] = np.linspace(-1e-8, 1e-8, 32, dtype=np.float32)
    x[0, 32:64] = np.linspace(-1e-6, 1e-6, 32, dtype=np.float32)
    x[0, 64:96] = np.linspace(-1.0, 1.0, 32, dtype=np.float32)
    q, d = O.quant_act(x)
    assert d[0, 0] == 2.0 ** -21 and d[0, 1] == 2.0 ** -21
    assert (q[0, :32] == 0).all()
    assert np.abs(q[0, 32:64]).max() == 2
    O.lib().orc_set_act_scale_plain(1)
    try:
        qp, dp = O.quant_act(x)
    finally:
        O.lib().orc_set_act_scale_plain(0)
    assert np.abs(qp[0, :32]).max() == 127 and np.abs(qp[0, 32:64]).max() == 127


def _teacher_forced(model, seq, greedy_from=None, split=SPLIT):
    od = O.Decoder(model, 1, PS, PPS + 1, PPS, MAXPOS, kv_f16=False, split=split)
    routes = Routes(1, PS, PPS + 1, PPS, seed=0, permute=False)
    out = []
    try:
        for i in range(96):
            od.prime_lanes([0], [seq[i]])
            tok = od.step_lanes(**routes.step([0]))
            out.append(np.array(od.logits()[0], dtype=np.float64, copy=True))
            if greedy_from is not None and i >= greedy_from and len(seq) < 96:
                seq.append(int(tok[0]))
    finally:
        od.close()
    return out


def test_config1_scale_cost_teacher_forced():
    """configs[0] with f32 K/V (the reference CPU path's KV precision): the
    prompt, then the 4-bit-scale run's own 64 greedy tokens, fed to both scales,
    and, as the yardstick, to the 4-bit scale with the attention split at 16
    instead of 64 (a change of summation order only).  Measured on the last
    prompt step and the 64 generated ones: scale cost max-abs 0.098, min cosine
    0.99925, argmax agreement 63/65; summation-order floor max-abs 0.045, min
    cosine 0.99983, 63/65.  The bounds sit above the measurement."""
    prompt = [int(x) for x in np.random.default_rng(0).integers(0, CFG["vocab"], 32)]
    om = O.Model(CFG, seed=0)
    seq = list(prompt)
    try:
        ours = _teacher_forced(om, seq, greedy_from=31)
        floor = _teacher_forced(om, seq, split=16)
        O.lib().orc_set_act_scale_plain(1)
        try:
            plain = _teacher_forced(om, seq)
        finally:
            O.lib().orc_set_act_scale_plain(0)
    finally:
        om.close()

    def stats(xs, ys):
        ma, cs, ag = [], [], []
        for a, b in zip(xs[31:], ys[31:]):
            ma.append(float(np.max(np.abs(a - b))))
            cs.append(float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b))))
            ag.append(int(np.argmax(a)) == int(np.argmax(b)))
        return max(ma), min(cs), sum(ag), len(ag)

    sm, sc, sa, n = stats(ours, plain)
    fm, fc, fa, _ = stats(ours, floor)
    print(f"  4-bit-significand scale vs amax/127: max-abs {sm:.4f}, min cosine {sc:.6f}, argmax agreement "
          f"{sa}/{n}; split 16 vs 64 (floor): max-abs {fm:.4f}, min cosine {fc:.6f}, {fa}/{n}", flush=True)
    assert sm < 0.2 and sc > 0.9985 and sa >= n - 4
    assert fm < sm
