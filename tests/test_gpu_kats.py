"""GPU cases the decode-step tests leave open: the reference's tail KAT and its
corners on the step's own tail kernel, the isolated-attention workload of
BASELINE configs[3] at its full size, merges of more than 128 splits, and the
north star's per-kernel tolerance for fp16 KV against f32 KV.  Everything runs
through the C ABI and is checked against the CPU oracle (bit for bit) or a
float64 restatement (within the stated tolerance)."""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle as O
from rstr import configs, hip, workload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sess():
    s = hip.Session(0)
    yield s
    s.close()


def _attn_cfg(n_q, n_kv, hd):
    c = dict(configs.TINY_LLAMA)
    c.update(n_layers=1, d_model=128, d_ff=128, vocab=64, n_q=n_q, n_kv=n_kv, head_dim=hd)
    return c


# ---------------------------------------------------------------------------
# tail: argmax (ties -> lowest id, NaN wins, lowest NaN) + embedding gather
# ---------------------------------------------------------------------------
def test_tail_reference_kat(sess):
    """decoder_gpu_composition_test.clj:9-20: tokens [1 1], rows [1 11 1 11]."""
    print("case tail KAT", flush=True)
    nan = np.float32("nan")
    logits = np.array([[1.0, 5.0, 5.0, 2.0], [9.0, nan, 8.0, nan]], np.float32)
    emb = np.array([[0.0, 10.0], [1.0, 11.0], [2.0, 12.0], [3.0, 13.0]], np.float32)
    tok, rows = sess.tail(logits, emb)
    assert tok.tolist() == [1, 1]
    assert rows.ravel().tolist() == [1.0, 11.0, 1.0, 11.0]


def _tail_rows(V, rng):
    rows = []
    r = rng.standard_normal(V).astype(np.float32)
    r[:] = -1.0
    r[V - 1] = 0.0
    r[V // 2] = -0.0            # +0 and -0 tie: the lower id
    rows.append(r)
    r = rng.standard_normal(V).astype(np.float32)
    r[V - 1] = np.nan           # NaN in the last element (last float4 chunk)
    rows.append(r)
    r = rng.standard_normal(V).astype(np.float32)
    r[V - 3] = np.nan
    r[min(7, V - 1)] = np.nan   # two NaNs: the lower id
    rows.append(r)
    r = rng.standard_normal(V).astype(np.float32)
    for i in (V - 1, V // 3, min(11, V - 1)):
        r[i] = 5.0              # a three-way tie of the maximum
    rows.append(r)
    rows.append(np.full(V, -np.inf, np.float32))   # all -inf: id 0
    r = rng.standard_normal(V).astype(np.float32)
    r[0] = 9.0                  # the maximum at id 0
    rows.append(r)
    r = rng.standard_normal(V).astype(np.float32)
    r[V - 1] = np.nan
    r[max(V - 4, 0)] = np.nan   # both NaNs inside the last float4 chunk
    rows.append(r)
    r = rng.standard_normal(V).astype(np.float32)
    r[max(V - 2, 0)] = np.inf
    r[V - 1] = np.inf           # +inf tie
    rows.append(r)
    return np.stack(rows)


@pytest.mark.parametrize("V", [262144, 151936, 128256, 4099, 4])
def test_tail_ties_signed_zeros_nans_and_last_chunk(sess, V):
    """numpy's argmax returns the first NaN, else the first maximum (-0 == +0):
    exactly the tail's contract.  Vocabularies of the three configs (float4
    path), an odd one (scalar path) and the KAT's 4."""
    print(f"case tail corners V={V}", flush=True)
    rng = np.random.default_rng(V)
    logits = _tail_rows(V, rng)
    d = 8
    emb = rng.standard_normal((V, d)).astype(np.float32)
    tok, rows = sess.tail(logits, emb)
    want = np.argmax(logits, axis=1)
    assert tok.tolist() == want.tolist()
    assert tok.tolist() == O.argmax_rows(logits).tolist()
    assert np.array_equal(rows, emb[want])


# ---------------------------------------------------------------------------
# attention: BASELINE configs[3] at its own size, and merges past 128 splits
# ---------------------------------------------------------------------------
def test_config4_full_workload_matches_oracle(sess):
    """128 lanes, 32/8 heads, hd 128, contexts lognormal(7, 1.2) clipped to
    [16, 32768] (seed 4), permuted page ids, 25% of full pages shared across
    lanes, split 256: the bench's own routes, bit for bit against the oracle."""
    print("case config4 full workload", flush=True)
    B, seed, ps = 128, 4, 16
    lengths, pt, physical, _, rng = workload.shared_prefix_routes(B, seed, page_size=ps)
    cfg = _attn_cfg(32, 8, 128)
    m = hip.Model(sess, cfg, seed=1)
    p = hip.Pool(m, ps, physical)
    try:
        p.fill_synthetic(np.arange(physical, dtype=np.int32), seed)
        kp, vp = p.pages(0, 0), p.pages(1, 0)
        q = rng.standard_normal((B, 32, 128)).astype(np.float32)
        scale = 1.0 / math.sqrt(128)
        got = p.attention(0, q, pt, lengths, scale=scale, split=256)
        print(f"  lanes {B}, mean ctx {lengths.mean():.0f}, max {lengths.max()}, {physical} pages", flush=True)
        want = O.attention(q, kp, vp, pt, lengths, 0, scale, 256)
        assert np.array_equal(got, want)
    finally:
        p.close()
        m.close()


@pytest.mark.parametrize("window", [0, 2090, 4000])
def test_attention_past_128_splits_matches_oracle(sess, window):
    """Split 16 over routes of 2100 and 4100 tokens: 132 and 257 splits, i.e. the
    merge's third to fifth 64-split groups of the maximum and of the exp-weight
    rounds; windows keep 131-251 splits."""
    print(f"case attention >128 splits window={window}", flush=True)
    cfg = _attn_cfg(8, 2, 128)
    lengths = np.array([2100, 4100, 300, 0, 2049], np.int32)
    B, ps = len(lengths), 16
    npg = -(-lengths // ps)
    pps, pages = int(npg.max()), int(npg.sum()) + 3
    rng = np.random.default_rng(window + 129)
    m = hip.Model(sess, cfg, seed=2)
    p = hip.Pool(m, ps, pages)
    try:
        kp = rng.standard_normal((pages, ps, 2, 128)).astype(np.float16)
        vp = rng.standard_normal((pages, ps, 2, 128)).astype(np.float16)
        p.upload(0, 0, 0, kp)
        p.upload(1, 0, 0, vp)
        perm = rng.permutation(pages).astype(np.int32)
        pt = np.full((B, pps), -1, np.int32)
        used = 0
        for b in range(B):
            pt[b, :npg[b]] = perm[used:used + npg[b]]
            used += int(npg[b])
        q = rng.standard_normal((B, 8, 128)).astype(np.float32)
        scale = 1.0 / math.sqrt(128)
        got = p.attention(0, q, pt, lengths, window=window, scale=scale, split=16)
        want = O.attention(q, kp, vp, pt, lengths, window, scale, 16)
        assert np.array_equal(got, want)
        assert np.all(got[3] == 0)
    finally:
        p.close()
        m.close()


def test_attention_fp16_kv_within_north_star_tolerance(sess):
    """The north star's per-kernel bound, max-abs 2e-2 and cosine >= 0.9999:
    attention over fp16 pages (the routed append's RNE rounding) against float64
    attention over the same K/V before rounding (the reference CPU path's f32
    kc/vc, decoder.clj:304-310).  Llama geometry, contexts to 5000."""
    print("case attention fp16 vs f32 KV tolerance", flush=True)
    cfg = _attn_cfg(32, 8, 128)
    lengths = np.array([1, 37, 900, 5000, 2048, 333], np.int32)
    B, ps = len(lengths), 16
    npg = -(-lengths // ps)
    pps, pages = int(npg.max()), int(npg.sum())
    rng = np.random.default_rng(77)
    k32 = rng.standard_normal((pages, ps, 8, 128)).astype(np.float32)
    v32 = rng.standard_normal((pages, ps, 8, 128)).astype(np.float32)
    m = hip.Model(sess, cfg, seed=2)
    p = hip.Pool(m, ps, pages)
    try:
        p.upload(0, 0, 0, k32.astype(np.float16))
        p.upload(1, 0, 0, v32.astype(np.float16))
        pt = np.full((B, pps), -1, np.int32)
        used = 0
        for b in range(B):
            pt[b, :npg[b]] = np.arange(used, used + npg[b])
            used += int(npg[b])
        q = rng.standard_normal((B, 32, 128)).astype(np.float32)
        scale = 1.0 / math.sqrt(128)
        got = p.attention(0, q, pt, lengths, scale=scale, split=256)
        worst, cos_min = 0.0, 1.0
        for b in range(B):
            ks = np.concatenate([k32[pt[b, i]] for i in range(npg[b])])[:lengths[b]].astype(np.float64)
            vs = np.concatenate([v32[pt[b, i]] for i in range(npg[b])])[:lengths[b]].astype(np.float64)
            for h in range(32):
                s = ks[:, h // 4] @ q[b, h].astype(np.float64) * scale
                w = np.exp(s - s.max())
                ref = (w / w.sum()) @ vs[:, h // 4]
                g = got[b, h].astype(np.float64)
                worst = max(worst, float(np.max(np.abs(g - ref))))
                cos_min = min(cos_min, float(g @ ref / (np.linalg.norm(g) * np.linalg.norm(ref))))
        print(f"  fp16 KV vs f32 KV: max-abs {worst:.3e}, min cosine {cos_min:.8f}", flush=True)
        assert worst <= 2e-2 and cos_min >= 0.9999
    finally:
        p.close()
        m.close()
