"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Integer/byte/index results (packed weights, page contents, token ids) must be
bit-exact; this build also holds every float intermediate bit-exact (logits,
resident rows, attention outputs) because the kernels follow the oracle's
canonical operation order.  The reference's own device KATs are reproduced
first (continuation_paged_attention_device_test.clj:42-174,
continuation_paged_append_device_test.clj:30-119).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle as O
from lanes import Routes
from rstr import configs, hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sess():
    s = hip.Session(0)
    yield s
    s.close()


def _cfg(name, **kw):
    c = dict(configs.MODELS[name])
    c.update(kw)
    return c


# ---------------------------------------------------------------------------
# weights
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("name,bits", [("tiny_gemma", 4), ("tiny_llama", 4), ("tiny_qwen", 8),
                                       ("tiny_llama", 8)])
def test_synthetic_weights_bit_exact(sess, name, bits):
    cfg = configs.with_bits(configs.MODELS[name], bits)
    print(f"case weights {name} q{bits}", flush=True)
    m = hip.Model(sess, cfg, seed=5)
    om = O.Model(cfg, seed=5)
    try:
        for layer in range(cfg["n_layers"]):
            for role in ("q", "k", "v", "o", "gate", "up", "down"):
                gw, gs = m.export_linear(layer, role)
                ow, osc = om.tensor(layer, role)
                assert np.array_equal(gw, ow), (layer, role)
                assert np.array_equal(gs, osc), (layer, role)
        gw, gs = m.export_linear(-1, "embed")
        ow, osc = om.tensor(-1, "embed")
        assert np.array_equal(gw, ow) and np.array_equal(gs, osc)
    finally:
        m.close()


def _edge_matrix(n, k, seed):
    """Weights with the quantiser's edge cases: zero blocks, signed ties, tiny and
    huge magnitudes, exact multiples of the step."""
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.02)
    w[0, :32] = 0.0
    w[1, :32] = 0.5
    w[1, 5] = -0.5                     # |max| tie between signs: first occurrence wins
    w[2, :32] = np.linspace(-8, 7, 32, dtype=np.float32)   # exact grid
    w[3, :32] = 1e-30
    w[4, :32] = 6e4
    w[5, 32:64] = -rng.random(32).astype(np.float32)
    return w


@pytest.mark.parametrize("bits", [4, 8])
def test_host_tensor_bind_quantises_like_the_oracle(sess, bits):
    cfg = configs.with_bits(configs.TINY_LLAMA, bits)
    print(f"case host-bind q{bits}", flush=True)
    tensors = []
    expect = {}
    seed = 11
    for layer in range(cfg["n_layers"]):
        for role in ("q", "k", "v", "o", "gate", "up", "down"):
            n, k = O.linear_shape(cfg, role)
            w = _edge_matrix(n, k, seed)
            seed += 1
            tensors.append((layer, role, w))
            expect[(layer, role)] = O.quant_q4(w) if bits == 4 else O.quant_q8(w)
        for role in ("attn_norm", "ffn_pre_norm"):
            tensors.append((layer, role, np.ones(cfg["d_model"], np.float32)))
    emb = _edge_matrix(cfg["vocab"], cfg["d_model"], 99)
    tensors.append((-1, "embed", emb))
    tensors.append((-1, "final_norm", np.ones(cfg["d_model"], np.float32)))
    expect[(-1, "embed")] = O.quant_q4(emb) if bits == 4 else O.quant_q8(emb)
    m = hip.Model(sess, cfg, tensors=tensors)
    try:
        for (layer, role), (ew, es) in expect.items():
            gw, gs = m.export_linear(layer, role)
            assert np.array_equal(gw, ew), (layer, role)
            assert np.array_equal(gs, es), (layer, role)
    finally:
        m.close()


def test_host_bind_rejects_missing_tensor(sess):
    cfg = configs.TINY_LLAMA
    with pytest.raises(hip.RstrError, match="missing"):
        hip.Model(sess, cfg, tensors=[(-1, "final_norm", np.ones(cfg["d_model"]))])


# ---------------------------------------------------------------------------
# reference KATs: append and attention
# ---------------------------------------------------------------------------
def _kat_pool(sess, page_size=4, pages=4):
    cfg = configs.TINY_GEMMA      # n_kv 1, head_dim 64: the KAT's 2/4-wide rows embed in dims 0..3
    m = hip.Model(sess, cfg, seed=1)
    return m, hip.Pool(m, page_size, pages)


def _row(vals, hd=64):
    r = np.zeros(hd, np.float32)
    r[:len(vals)] = vals
    return r


def test_reference_attention_kat(sess):
    """continuation_paged_attention_device_test.clj:42-174: K=[[1,0],[0,1]],
    V=[[10,20],[30,40]], q=[1,0], scale 1/sqrt(2) -> [16.6048 26.6048]; a
    one-token lane gives [5 7]; window-left 0 gives [30 40] and [5 7]."""
    print("case attention KAT", flush=True)
    m, p = _kat_pool(sess)
    try:
        # route a: pages [0] tokens 0,1 ; route b: page [1] token 0
        p.append(0, [_row([1, 0]), _row([0, 1]), _row([1, 1])],
                 [_row([10, 20]), _row([30, 40]), _row([5, 7])], [0, 1, 4])
        q = np.stack([_row([1, 0]), _row([1, 0])])[:, None, :]
        pt = np.array([[0, -1], [1, -1]], np.int32)
        lengths = np.array([2, 1], np.int32)
        out = p.attention(0, q, pt, lengths, scale=1 / math.sqrt(2.0))
        got = np.concatenate([out[0, 0, :2], out[1, 0, :2]])
        assert np.all(np.abs(got - np.array([16.6048, 26.6048, 5.0, 7.0])) < 1e-4), got
        assert np.all(out[:, :, 2:] == 0)
        # several history tiles (split 4 > route) give the same value
        out2 = p.attention(0, q, pt, lengths, scale=1 / math.sqrt(2.0), split=4)
        assert np.array_equal(out, out2)
        win = p.attention(0, q, pt, lengths, scale=1 / math.sqrt(2.0), window=1)
        assert np.array_equal(np.concatenate([win[0, 0, :2], win[1, 0, :2]]),
                              np.array([30.0, 40.0, 5.0, 7.0], np.float32))
    finally:
        p.close()
        m.close()


def test_reference_append_kat(sess):
    """continuation_paged_append_device_test.clj:30-119: rows land in fp16
    (round to nearest even) exactly at their slots, every other element keeps
    the sentinel 42.0, and append -> attention over the fresh row returns the
    value row exactly."""
    print("case append KAT", flush=True)
    m, p = _kat_pool(sess, page_size=4, pages=3)
    try:
        hd = 64
        sentinel = np.float16(42.0).view(np.uint16)
        for slab in (0, 1):
            p.upload(slab, 0, 0, np.full(3 * 4 * hd, sentinel, np.uint16))
        k_rows = [_row([1.1, -2.2, 3.3, -4.4]), _row([5.5, -6.6, 7.7, -8.8])]
        v_rows = [_row([0.25, -0.5, 0.75, -1.0]), _row([1.25, -1.5, 1.75, -2.0])]
        slots = [4, 3]
        p.append(0, k_rows, v_rows, slots)
        kk = p.download(0, 0).reshape(12, hd)
        vv = p.download(1, 0).reshape(12, hd)
        for slot in range(12):
            if slot in slots:
                lane = slots.index(slot)
                assert np.array_equal(kk[slot], k_rows[lane].astype(np.float16).view(np.uint16))
                assert np.array_equal(vv[slot], v_rows[lane].astype(np.float16).view(np.uint16))
            else:
                assert np.all(kk[slot] == sentinel) and np.all(vv[slot] == sentinel)
        # append then attention over the one-row route at slot 8 (page 2)
        p.append(0, [k_rows[0]], [v_rows[0]], [8])
        out = p.attention(0, np.array([[_row([1, 0, 0, 0])]]), np.array([[2]], np.int32),
                          np.array([1], np.int32))
        assert np.array_equal(out[0, 0, :4], np.array([0.25, -0.5, 0.75, -1.0], np.float32))
    finally:
        p.close()
        m.close()


def test_append_rejects_duplicate_slots(sess):
    m, p = _kat_pool(sess)
    try:
        with pytest.raises(hip.RstrError, match="distinct"):
            p.append(0, [_row([1])] * 2, [_row([1])] * 2, [3, 3])
    finally:
        p.close()
        m.close()


# ---------------------------------------------------------------------------
# attention vs the oracle on random ragged inputs
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("hd,n_q,n_kv", [(128, 8, 2), (64, 4, 4)])
@pytest.mark.parametrize("split,window", [(16, 0), (32, 700)])
def test_attention_many_splits_matches_oracle(sess, hd, n_q, n_kv, split, window):
    """Routes of up to 69 splits: the merge's rounds of 16 splits and its second
    group of 64 (exp weights read from the lane that computed them)."""
    print(f"case attention many splits hd{hd} q{n_q} kv{n_kv} split{split} window{window}", flush=True)
    _many_splits_case(sess, hd, n_q, n_kv, split, window, 6)


@pytest.mark.parametrize("hd,n_q,n_kv,B", [(128, 32, 8, 63), (128, 32, 8, 64), (256, 8, 2, 255),
                                           (256, 8, 2, 256)])
def test_attention_merge_forms_match_oracle(sess, hd, n_q, n_kv, B):
    """Both merge forms on routes of up to 69 splits: one wave per (lane, head)
    from 2048 (lane, head) pairs on, one wave per 64 dims of a head below (32
    or 64 splits per load round, the second group of 64 splits)."""
    print(f"case attention merge forms hd{hd} q{n_q} kv{n_kv} B{B}", flush=True)
    _many_splits_case(sess, hd, n_q, n_kv, 16, 0, B)


@pytest.mark.parametrize("lo,hi", [(1024, 1800), (2100, 2600)])
def test_attention_long_lists_match_oracle(sess, lo, hi):
    """Long lists on the one-wave split kernel (128 lanes, 32/8 heads, hd 128,
    split 256): 4-10 full splits per lane are 2-5 rounds of full items on
    MI355X's 2048 resident waves, so static rounds and the claim phase both
    run.  Pages are drawn with repetition from a small pool (lanes share
    pages).  Bit-exact against the oracle."""
    print(f"case attention long lists ctx [{lo}, {hi})", flush=True)
    hd, n_q, n_kv, B, ps, split = 128, 32, 8, 128, 16, 256
    cfg = _cfg("tiny_llama", n_layers=1, d_model=128, d_ff=128, vocab=64, n_q=n_q, n_kv=n_kv, head_dim=hd)
    rng = np.random.default_rng(lo)
    lengths = rng.integers(lo, hi, B).astype(np.int32)
    pages, pps = 384, int(-(-lengths.max() // ps))
    m = hip.Model(sess, cfg, seed=2)
    p = hip.Pool(m, ps, pages)
    try:
        kp = rng.standard_normal((pages, ps, n_kv, hd)).astype(np.float16)
        vp = rng.standard_normal((pages, ps, n_kv, hd)).astype(np.float16)
        p.upload(0, 0, 0, kp)
        p.upload(1, 0, 0, vp)
        pt = rng.integers(0, pages, (B, pps)).astype(np.int32)
        q = rng.standard_normal((B, n_q, hd)).astype(np.float32)
        scale = 1.0 / math.sqrt(hd)
        got = p.attention(0, q, pt, lengths, window=0, scale=scale, split=split)
        want = O.attention(q, kp, vp, pt, lengths, 0, scale, split)
        assert np.array_equal(got, want)
    finally:
        p.close()
        m.close()


@pytest.mark.parametrize("window", [0, 40])
def test_attention_over_1024_lanes_matches_oracle(sess, window):
    """1100 lanes: past the one-workgroup list kernel's 1024 lanes, so the work
    list comes from the lane-table kernel (a scan carried across two 1024-lane
    chunks) and the item writer; contexts 0..160 at split 32 (empty lanes,
    partial first and last splits, windows).  Bit-exact against the oracle."""
    print(f"case attention 1100 lanes window {window}", flush=True)
    hd, n_q, n_kv, B, ps, split = 64, 4, 2, 1100, 16, 32
    cfg = _cfg("tiny_llama", n_layers=1, d_model=128, d_ff=128, vocab=64, n_q=n_q, n_kv=n_kv, head_dim=hd)
    rng = np.random.default_rng(1100 + window)
    lengths = rng.integers(0, 161, B).astype(np.int32)
    lengths[::97] = 0
    pages, pps = 256, int(-(-lengths.max() // ps))
    m = hip.Model(sess, cfg, seed=2)
    p = hip.Pool(m, ps, pages)
    try:
        kp = rng.standard_normal((pages, ps, n_kv, hd)).astype(np.float16)
        vp = rng.standard_normal((pages, ps, n_kv, hd)).astype(np.float16)
        p.upload(0, 0, 0, kp)
        p.upload(1, 0, 0, vp)
        pt = rng.integers(0, pages, (B, pps)).astype(np.int32)
        q = rng.standard_normal((B, n_q, hd)).astype(np.float32)
        scale = 1.0 / math.sqrt(hd)
        got = p.attention(0, q, pt, lengths, window=window, scale=scale, split=split)
        want = O.attention(q, kp, vp, pt, lengths, window, scale, split)
        assert np.array_equal(got, want)
        assert np.all(got[lengths == 0] == 0)
    finally:
        p.close()
        m.close()


def _many_splits_case(sess, hd, n_q, n_kv, split, window, B):
    cfg = _cfg("tiny_llama", n_layers=1, d_model=128, d_ff=128, vocab=64, n_q=n_q, n_kv=n_kv,
               head_dim=hd)
    lengths = np.resize(np.array([1100, 300, 0, 1025, 17, 257], np.int32), B)
    ps, pps = 16, 72
    pages = int(sum(-(-n // ps) for n in lengths)) + 4
    rng = np.random.default_rng(hd * 7 + split + window + B)
    m = hip.Model(sess, cfg, seed=2)
    p = hip.Pool(m, ps, pages)
    try:
        kp = rng.standard_normal((pages, ps, n_kv, hd)).astype(np.float16)
        vp = rng.standard_normal((pages, ps, n_kv, hd)).astype(np.float16)
        p.upload(0, 0, 0, kp)
        p.upload(1, 0, 0, vp)
        perm = rng.permutation(pages).astype(np.int32)
        pt = np.full((B, pps), -1, np.int32)
        used = 0
        for b in range(B):
            n = -(-lengths[b] // ps)
            pt[b, :n] = perm[used:used + n]
            used += n
        q = rng.standard_normal((B, n_q, hd)).astype(np.float32)
        scale = 1.0 / math.sqrt(hd)
        got = p.attention(0, q, pt, lengths, window=window, scale=scale, split=split)
        want = O.attention(q, kp, vp, pt, lengths, window, scale, split)
        assert np.array_equal(got, want)
        assert np.all(got[2] == 0) and np.isfinite(got).all()
    finally:
        p.close()
        m.close()


@pytest.mark.parametrize("hd,n_q,n_kv", [(128, 32, 8), (256, 4, 1), (64, 8, 2), (128, 16, 8), (128, 4, 1)])
@pytest.mark.parametrize("split,window", [(256, 0), (32, 0), (16, 24)])
def test_attention_matches_oracle(sess, hd, n_q, n_kv, split, window):
    print(f"case attention hd{hd} q{n_q} kv{n_kv} split{split} window{window}", flush=True)
    cfg = _cfg("tiny_llama", n_layers=1, d_model=128, d_ff=128, vocab=64, n_q=n_q, n_kv=n_kv,
               head_dim=hd)
    B, ps, pages, pps = 7, 16, 96, 16
    rng = np.random.default_rng(hd + split + window)
    m = hip.Model(sess, cfg, seed=2)
    p = hip.Pool(m, ps, pages)
    try:
        kp = rng.standard_normal((pages, ps, n_kv, hd)).astype(np.float16)
        vp = rng.standard_normal((pages, ps, n_kv, hd)).astype(np.float16)
        p.upload(0, 0, 0, kp)
        p.upload(1, 0, 0, vp)
        lengths = np.array([1, 0, 17, 255, 256, 100, 233], np.int32)
        perm = rng.permutation(pages).astype(np.int32)
        pt = np.full((B, pps), -1, np.int32)
        used = 0
        for b in range(B):
            n = -(-lengths[b] // ps)
            pt[b, :n] = perm[used:used + n]
            used += n
        q = rng.standard_normal((B, n_q, hd)).astype(np.float32)
        scale = 1.0 / math.sqrt(hd)
        got = p.attention(0, q, pt, lengths, window=window, scale=scale, split=split)
        want = O.attention(q, kp, vp, pt, lengths, window, scale, split)
        assert np.array_equal(got, want)
        # float64 softmax restatement: the canonical order stays within fp32 rounding
        for b in range(B):
            L = lengths[b]
            if L == 0:
                assert np.all(got[b] == 0)
                continue
            lo = max(0, L - window) if window else 0
            ks = np.stack([kp[pt[b, t // ps], t % ps] for t in range(lo, L)]).astype(np.float64)
            vs = np.stack([vp[pt[b, t // ps], t % ps] for t in range(lo, L)]).astype(np.float64)
            for h in range(n_q):
                kvh = h // (n_q // n_kv)
                s = ks[:, kvh] @ q[b, h].astype(np.float64) * scale
                w = np.exp(s - s.max())
                ref = (w / w.sum()) @ vs[:, kvh]
                assert np.max(np.abs(ref - got[b, h])) < 2e-5 * (1 + np.max(np.abs(ref)))
    finally:
        p.close()
        m.close()


@pytest.mark.parametrize("hd,n_q,n_kv", [(128, 32, 8), (64, 8, 2)])
@pytest.mark.parametrize("ps,split", [(4, 20), (8, 64), (12, 256), (32, 20), (48, 64), (64, 256), (32, 256),
                                      (64, 36)])
@pytest.mark.parametrize("window", [0, 24])
def test_attention_page_sizes_and_splits_match_oracle(sess, hd, n_q, n_kv, ps, split, window):
    """Page sizes that are and are not powers of two times 16 (whole-page chunks
    or per-row page lookups) and splits that are not multiples of the 16-token
    chunk: the routed attention equals the oracle bit for bit on permuted pages,
    with empty, one-token, page-boundary and multi-split lanes."""
    print(f"case attention ps{ps} split{split} window{window} hd{hd}", flush=True)
    cfg = _cfg("tiny_llama", n_layers=1, d_model=128, d_ff=128, vocab=64, n_q=n_q, n_kv=n_kv,
               head_dim=hd)
    lengths = np.array([1, 0, ps, ps + 1, 3 * ps - 1, 300, 129], np.int32)
    B = len(lengths)
    npg = -(-lengths // ps)
    pps = int(npg.max())
    pages = int(npg.sum()) + 3
    rng = np.random.default_rng(ps * 1000 + split + window + hd)
    m = hip.Model(sess, cfg, seed=2)
    p = hip.Pool(m, ps, pages)
    try:
        kp = rng.standard_normal((pages, ps, n_kv, hd)).astype(np.float16)
        vp = rng.standard_normal((pages, ps, n_kv, hd)).astype(np.float16)
        p.upload(0, 0, 0, kp)
        p.upload(1, 0, 0, vp)
        perm = rng.permutation(pages).astype(np.int32)
        pt = np.full((B, pps), -1, np.int32)
        used = 0
        for b in range(B):
            pt[b, :npg[b]] = perm[used:used + npg[b]]
            used += npg[b]
        q = rng.standard_normal((B, n_q, hd)).astype(np.float32)
        scale = 1.0 / math.sqrt(hd)
        got = p.attention(0, q, pt, lengths, window=window, scale=scale, split=split)
        want = O.attention(q, kp, vp, pt, lengths, window, scale, split)
        assert np.array_equal(got, want)
    finally:
        p.close()
        m.close()


@pytest.mark.parametrize("ps,pps,pages", [(8, 40, 200), (32, 10, 60), (12, 26, 130)])
def test_decode_steps_page_sizes(sess, ps, pps, pages):
    """Decode steps on pools of 8-, 32- and 12-token pages (whole-page chunks,
    per-row lookups, routed appends across page boundaries): tokens and logits
    equal the oracle's on every step."""
    print(f"case decode ps{ps}", flush=True)
    cfg = configs.TINY_LLAMA
    r = _run_lanes(sess, cfg, 4, [5, 0, ps - 1, 2 * ps + 3], [[0, 1, 2, 3], [0, 2, 3], [0, 1, 2, 3], [1, 3]],
                   split=32, ps=ps, pages=pages, pps=pps, maxpos=pps * ps)
    _close(r)


@pytest.mark.parametrize("hd,n_q,n_kv", [(128, 32, 8), (128, 16, 8), (128, 8, 1), (256, 4, 1), (256, 8, 8),
                                         (128, 8, 8)])
@pytest.mark.parametrize("split,window", [(256, 0), (64, 40)])
def test_attention_few_and_many_item_kernels_agree(sess, hd, n_q, n_kv, split, window):
    """Short work lists run one 4-wave workgroup per item, long ones one wave per
    item.  The same seven lanes run alone (short list) and beside a long eighth
    lane that reuses their pages (its list forces the one-wave kernel): their
    outputs agree bit for bit, and with the oracle."""
    print(f"case attention kernels agree hd{hd} q{n_q} kv{n_kv} split{split} window{window}", flush=True)
    cfg = _cfg("tiny_llama", n_layers=1, d_model=128, d_ff=128, vocab=64, n_q=n_q, n_kv=n_kv,
               head_dim=hd)
    B, ps, pages = 7, 16, 96
    long_len = split * (-(-4200 // n_kv))  # > 4200 items of its own: more than two rounds of workgroups
    pps = -(-long_len // ps)
    rng = np.random.default_rng(7 * hd + split + window + n_q)
    m = hip.Model(sess, cfg, seed=2)
    p = hip.Pool(m, ps, pages)
    try:
        kp = rng.standard_normal((pages, ps, n_kv, hd)).astype(np.float16)
        vp = rng.standard_normal((pages, ps, n_kv, hd)).astype(np.float16)
        p.upload(0, 0, 0, kp)
        p.upload(1, 0, 0, vp)
        lengths = np.array([1, 0, 17, 255, 256, 100, 233], np.int32)
        perm = rng.permutation(pages).astype(np.int32)
        pt = np.full((B + 1, pps), -1, np.int32)
        used = 0
        for b in range(B):
            n = -(-lengths[b] // ps)
            pt[b, :n] = perm[used:used + n]
            used += n
        pt[B, :] = np.arange(pps, dtype=np.int32) % pages
        q = rng.standard_normal((B + 1, n_q, hd)).astype(np.float32)
        scale = 1.0 / math.sqrt(hd)
        few = p.attention(0, q[:B], pt[:B], lengths, window=window, scale=scale, split=split)
        many = p.attention(0, q, pt, np.append(lengths, np.int32(long_len)), window=window, scale=scale,
                           split=split)
        assert np.array_equal(few, many[:B])
        want = O.attention(q[:B], kp, vp, pt[:B], lengths, window, scale, split)
        assert np.array_equal(few, want)
    finally:
        p.close()
        m.close()


def test_attention_long_shared_routes_match_oracle(sess):
    """Config-4 geometry (32/8 heads, hd 128): long routes (many splits), pages
    shared across lanes (a common prefix run), permuted page ids."""
    print("case attention long shared routes", flush=True)
    cfg = _cfg("tiny_llama", n_layers=1, d_model=128, d_ff=128, vocab=64, n_q=32, n_kv=8, head_dim=128)
    ps = 16
    lengths = np.array([16, 300, 5000, 4097, 33, 8000, 0, 2049], np.int32)
    B = len(lengths)
    rng = np.random.default_rng(44)
    shared = 40  # the first min(40, full pages) pages of every lane are one shared run
    npg = -(-lengths // ps)
    priv = int(np.maximum(npg - np.minimum(lengths // ps, shared), 0).sum())
    pages = shared + priv
    perm = rng.permutation(pages).astype(np.int32)
    pps = int(npg.max())
    pt = np.full((B, pps), -1, np.int32)
    used = shared
    for b in range(B):
        k = int(min(lengths[b] // ps, shared))
        pt[b, :k] = perm[:k]
        n = int(npg[b]) - k
        pt[b, k:npg[b]] = perm[used:used + n]
        used += n
    m = hip.Model(sess, cfg, seed=2)
    p = hip.Pool(m, ps, pages)
    try:
        kp = rng.standard_normal((pages, ps, 8, 128)).astype(np.float16)
        vp = rng.standard_normal((pages, ps, 8, 128)).astype(np.float16)
        p.upload(0, 0, 0, kp)
        p.upload(1, 0, 0, vp)
        q = rng.standard_normal((B, 32, 128)).astype(np.float32)
        scale = 1.0 / math.sqrt(128)
        got = p.attention(0, q, pt, lengths, scale=scale, split=256)
        want = O.attention(q, kp, vp, pt, lengths, 0, scale, 256)
        assert np.array_equal(got, want)
        assert np.all(got[6] == 0)
    finally:
        p.close()
        m.close()


# ---------------------------------------------------------------------------
# full decode steps
# ---------------------------------------------------------------------------
def _run_lanes(sess, cfg, B, prefix, schedule, graph=True, split=16, ps=16, pages=80, pps=10,
               maxpos=160, seed=3, kv_seed=17, tokens=None):
    """Drive GPU and oracle decoders through the same descriptors; return both
    token histories plus the decoders for further checks."""
    routes = Routes(B, ps, pages, pps, seed=seed)
    m = hip.Model(sess, cfg, seed=seed)
    p = hip.Pool(m, ps, pages)
    d = hip.Decoder(m, p, B, pps, maxpos, split)
    d.set_graph(graph)
    om = O.Model(cfg, seed=seed)
    od = O.Decoder(om, B, ps, pages, pps, maxpos, kv_f16=True, split=split)
    r = dict(m=m, p=p, d=d, om=om, od=od, routes=routes)
    try:
        return _drive(r, cfg, B, prefix, schedule, kv_seed, tokens)
    except BaseException:
        _close(r)
        raise


def _drive(r, cfg, B, prefix, schedule, kv_seed, tokens):
    m, p, d, om, od, routes = r["m"], r["p"], r["d"], r["om"], r["od"], r["routes"]
    for b, n in enumerate(prefix):
        new = routes.prefix(b, n)
        if new:
            p.fill_synthetic(new, kv_seed)
            for pg in new:
                od.fill_synthetic(pg, kv_seed)
    toks = tokens if tokens is not None else (np.arange(B) * 37 + 5) % cfg["vocab"]
    d.prime_lanes(np.arange(B), toks)
    od.prime_lanes(np.arange(B), toks)
    hist_g, hist_o = [], []
    for active in schedule:
        desc = routes.step(active)
        g = d.step_lanes(**desc)
        o = od.step_lanes(**desc)
        act = np.array(sorted(active))
        assert np.array_equal(g[act], o[act]), (g, o)
        gl, ol = d.logits(), od.logits()
        assert np.array_equal(gl[act], ol[act])
        hist_g.append(g)
        hist_o.append(o)
    r.update(g=hist_g, o=hist_o)
    return r


def _close(r):
    r["d"].close()
    r["p"].close()
    r["m"].close()
    r["od"].close()
    r["om"].close()


@pytest.mark.parametrize("name", ["tiny_gemma", "tiny_llama", "tiny_qwen"])
@pytest.mark.parametrize("graph", [True, False])
def test_decode_steps_bit_exact(sess, name, graph):
    print(f"case decode {name} graph={graph}", flush=True)
    cfg = configs.MODELS[name]
    B = 6
    prefix = [0, 17, 40, 3, 0, 60]
    sched = [[0, 1, 2, 3, 5], [0, 1, 2, 3, 5], [1, 2, 5], [0, 1, 2, 3, 4, 5]] + [list(range(6))] * 4
    r = _run_lanes(sess, cfg, B, prefix, sched, graph=graph)
    try:
        # every resident row and every page of every layer matches bit for bit
        assert np.array_equal(r["d"].rows(), r["od"].r0())
        for layer in range(cfg["n_layers"]):
            for slab in (0, 1):
                assert np.array_equal(r["p"].pages(slab, layer).view(np.uint16),
                                      r["od"].slab(slab, layer).view(np.uint16)), (layer, slab)
    finally:
        _close(r)


def test_lane_results_do_not_depend_on_the_batch(sess):
    """A lane decoded alone and inside a batch of ragged neighbours yields the same
    tokens and logits (the canonical orders are per row)."""
    print("case batch invariance", flush=True)
    cfg = configs.TINY_LLAMA
    sched = [[0, 1, 2, 3, 4, 5, 6, 7, 8]] * 5
    big = _run_lanes(sess, cfg, 9, [33, 5, 0, 70, 12, 1, 2, 44, 9], sched, tokens=np.full(9, 77))
    one = _run_lanes(sess, cfg, 1, [33], [[0]] * 5, tokens=np.array([77]))
    try:
        assert [h[0] for h in big["g"]] == [h[0] for h in one["g"]]
    finally:
        _close(big)
        _close(one)


@pytest.mark.parametrize("B", [40, 60, 100, 130])
def test_wide_batches_bit_exact(sess, B):
    """Row-tile groupings of the projection kernel (32 x 32 wave tiles at 40 rows,
    32 x 16 at 60, 64 x 16 in 2 and 3 row groups at 100 and 130; split-K slices)
    against the oracle."""
    print(f"case wide batch B={B}", flush=True)
    cfg = configs.TINY_QWEN
    rng = np.random.default_rng(B)
    prefix = [int(x) for x in rng.integers(0, 40, B)]
    sched = [list(range(B))] * 2
    r = _run_lanes(sess, cfg, B, prefix, sched, pages=B * 4 + 8, pps=4, maxpos=60)
    try:
        assert np.array_equal(r["d"].rows(), r["od"].r0())
    finally:
        _close(r)


@pytest.mark.parametrize("name,d_model,bits,B", [("tiny_llama", 512, 4, 100), ("tiny_gemma", 256, 4, 65),
                                                  ("tiny_qwen", 256, 8, 130), ("tiny_llama", 512, 8, 80)])
def test_fused_gate_up_activation_bit_exact(sess, name, d_model, bits, B):
    """A feed-forward width of 32768 at 65..130 rows (2048..3072 workgroups) takes the
    gate/up launch with the gated activation and its quantisation in the epilogue
    (one K slice, workgroup = one 32-column activation block of gate and up): SiLU
    and GeLU, Q4 and Q8, 4-block and 1-block chunks (d_model 512 / 256), 2 and 3 row
    groups; rows and tokens equal the oracle's, which runs gate/up and the
    activation as separate steps."""
    print(f"case fused act {name} d={d_model} q{bits} B={B}", flush=True)
    cfg = configs.with_bits(_cfg(name, d_model=d_model, d_ff=32768, vocab=512), bits)
    rng = np.random.default_rng(B + d_model)
    prefix = [int(x) for x in rng.integers(0, 40, B)]
    sched = [list(range(B)), [b for b in range(B) if b % 3]]
    r = _run_lanes(sess, cfg, B, prefix, sched, pages=B * 4 + 8, pps=4, maxpos=60)
    try:
        assert np.array_equal(r["d"].rows(), r["od"].r0())
    finally:
        _close(r)


@pytest.mark.parametrize("n_q,n_kv,hd", [(8, 1, 128), (2, 2, 128), (8, 1, 256), (4, 4, 256)])
def test_few_item_attention_with_qkv_prologue_group_sizes(sess, n_q, n_kv, hd):
    """Small batches run qk-norm, RoPE and the K/V append inside the few-item
    attention kernel; its prologue maps query heads to waves (head h on wave
    h mod 4), so GQA groups of 8 and of 1 take other paths than the shipped
    configs' groups of 2 and 4.  Decode steps with qk-norm (Qwen flags) and
    sandwich/GeLU flags (Gemma) equal the oracle bit for bit."""
    print(f"case qkv prologue n_q={n_q} n_kv={n_kv} hd={hd}", flush=True)
    base = "tiny_qwen" if hd == 128 else "tiny_gemma"
    cfg = _cfg(base, n_q=n_q, n_kv=n_kv, head_dim=hd, attn_scale=1.0 / math.sqrt(hd))
    B = 5
    prefix = [0, 21, 44, 3, 60]
    sched = [[0, 1, 2, 3, 4], [1, 2, 4], [0, 1, 2, 3, 4]]
    r = _run_lanes(sess, cfg, B, prefix, sched, pages=60, pps=10, maxpos=160)
    try:
        assert np.array_equal(r["d"].rows(), r["od"].r0())
        for layer in range(cfg["n_layers"]):
            for slab in (0, 1):
                assert np.array_equal(r["p"].pages(slab, layer).view(np.uint16),
                                      r["od"].slab(slab, layer).view(np.uint16)), (layer, slab)
    finally:
        _close(r)


@pytest.mark.parametrize("name,split", [("tiny_gemma", 16), ("tiny_qwen", 16), ("tiny_qwen", 128)])
def test_lanes_that_read_each_others_appends(sess, name, split):
    """Small batches run the qkv post-processing inside the few-item attention
    kernel, where each lane appends its own new K/V row.  A step whose lanes read
    each other's new rows (three causal lanes over one route, as a prefill tile
    lays them out) must still see every append, as the oracle's append-then-attend
    order does: the decoder runs such a step with the separate qkv launch.  Later
    steps on private routes return to the fused form.  At split 128 >= maxpos
    (head dim 128) both forms also write the attention output from the split
    kernel, without a merge launch."""
    print(f"case shared appends {name} split {split}", flush=True)
    cfg = configs.MODELS[name]
    B, ps, pages, pps, maxpos = 3, 16, 12, 6, 96
    start_len = 37
    pt = np.full((B, pps), -1, np.int32)
    route = np.array([7, 2, 9, 4], np.int32)
    for b in range(B):
        pt[b, :4] = route
    m = hip.Model(sess, cfg, seed=4)
    p = hip.Pool(m, ps, pages)
    d = hip.Decoder(m, p, B, pps, maxpos, split)
    om = O.Model(cfg, seed=4)
    od = O.Decoder(om, B, ps, pages, pps, maxpos, kv_f16=True, split=split)
    try:
        for pg in route[:3]:
            p.fill_synthetic([int(pg)], 23)
            od.fill_synthetic(int(pg), 23)
        toks = np.array([11, 12, 13], np.int32)
        d.prime_lanes(np.arange(B), toks)
        od.prime_lanes(np.arange(B), toks)
        # causal step: lane b's new token sits at position start_len + b and lane
        # b reads positions 0..start_len + b, i.e. the new rows of lanes < b
        lengths = np.array([start_len + b + 1 for b in range(B)], np.int32)
        pos = lengths - 1
        slots = np.array([route[t // ps] * ps + t % ps for t in pos], np.int32)
        desc = dict(slots=slots, row_offsets=np.arange(B + 1, dtype=np.int32), positions=pos.astype(np.int32),
                    page_table=pt, lengths=lengths, start_positions=np.zeros(B, np.int32))
        g = d.step_lanes(**desc)
        o = od.step_lanes(**desc)
        assert np.array_equal(g, o)
        assert np.array_equal(d.logits(), od.logits())
        for layer in range(cfg["n_layers"]):
            for slab in (0, 1):
                assert np.array_equal(p.pages(slab, layer).view(np.uint16), od.slab(slab, layer).view(np.uint16))
        # then one lane alone on its route (private append): the fused form
        lengths2 = np.array([start_len + 4, 0, 0], np.int32)
        t = int(lengths2[0]) - 1
        slots2 = np.array([route[t // ps] * ps + t % ps, -1, -1], np.int32)
        desc2 = dict(slots=slots2, row_offsets=np.arange(B + 1, dtype=np.int32),
                     positions=np.array([t, 0, 0], np.int32), page_table=pt, lengths=lengths2,
                     start_positions=np.zeros(B, np.int32))
        d.prime_lanes([0], [5])
        od.prime_lanes([0], [5])
        assert d.step_lanes(**desc2)[0] == od.step_lanes(**desc2)[0]
        assert np.array_equal(d.logits()[0], od.logits()[0])
    finally:
        d.close()
        p.close()
        m.close()
        od.close()
        om.close()


@pytest.mark.parametrize("bits", [4, 8])
def test_one_lane_long_k_weight_streaming(sess, bits):
    """One lane at Llama-3-8B width (first layer, full vocabulary): the MLP down
    projection (K = 14336) runs through the weight-streaming GEMV, which computes
    act(gate)*up and its quantisation while staging its input (no separate
    activation launch); tokens and logits equal the oracle's on every step, for
    Q4 and Q8 weights."""
    print(f"case one lane llama3_8b q{bits}", flush=True)
    cfg = configs.with_bits(_cfg("llama3_8b", n_layers=1), bits)
    r = _run_lanes(sess, cfg, 1, [300], [[0], [0], [0]], split=256, ps=16, pages=40, pps=30, maxpos=400)
    _close(r)


@pytest.mark.parametrize("name,B,bits", [("llama3_8b", 2, 4), ("llama3_8b", 2, 8), ("llama3_8b", 4, 4),
                                         ("qwen3_06b", 4, 8), ("qwen3_06b", 2, 4), ("gemma3_270m", 3, 8)])
def test_few_lane_weight_streaming(sess, name, B, bits):
    """Two to four lanes at full config width (first layer, full vocabulary):
    projections with four K slices run on the workgroup GEMV at two rows, and at
    three or four rows for matrices up to 4M weights, and the Qwen3 head (one
    slice, K = 1024) at two rows (the rest on the MFMA tile); a down projection
    on the workgroup GEMV computes the gated activation in its staging.  Tokens
    and logits equal the oracle's on every step."""
    print(f"case few lanes {name} B={B} q{bits}", flush=True)
    cfg = configs.with_bits(_cfg(name, n_layers=1), bits)
    prefix = [300, 0, 17, 120][:B]
    r = _run_lanes(sess, cfg, B, prefix, [list(range(B))] * 3, split=256, ps=16, pages=80, pps=30, maxpos=400)
    try:
        assert np.array_equal(r["d"].rows(), r["od"].r0())
    finally:
        _close(r)


@pytest.mark.parametrize("name,layers", [("llama3_8b", 1), ("gemma3_270m", 6), ("qwen3_06b", 1)])
def test_config_shapes_first_layers(sess, name, layers):
    """Full-width config shapes (vocabulary included) with the first layers only:
    one step of ragged lanes matches the oracle bit for bit."""
    print(f"case shape {name} layers={layers}", flush=True)
    cfg = _cfg(name, n_layers=layers)
    B = 4
    r = _run_lanes(sess, cfg, B, [700, 0, 33, 1500], [[0, 2, 3], [0, 1, 2, 3]], split=256,
                   ps=16, pages=200, pps=100, maxpos=1600)
    _close(r)


@pytest.mark.parametrize("graph", [True, False])
def test_step_timing_reports_the_last_call(sess, graph):
    """rstr_decoder_step_timing after rstr_step_lanes calls: every phase is a
    finite non-negative time, the step's device time is positive, and the host
    phases of the call fit inside the call's own duration."""
    print(f"case step timing graph={graph}", flush=True)
    cfg = configs.TINY_LLAMA
    r = _run_lanes(sess, cfg, 3, [5, 0, 19], [[0, 1, 2], [0, 2], [0, 1, 2]], graph=graph)
    try:
        t = r["d"].step_timing()
        assert set(t) == set(hip.Decoder.STEP_TIMING)
        assert all(np.isfinite(v) and v >= 0.0 for v in t.values()), t
        assert t["device_step"] > 0.0 and t["call"] > 0.0, t
        host = sum(t[k] for k in ("validate", "prior_sync", "pack", "enqueue", "device_wait", "handback"))
        assert host <= t["call"] * 1.05 + 1e-3, t
    finally:
        _close(r)


def test_step_rejects_bad_descriptors(sess):
    cfg = configs.TINY_LLAMA
    m = hip.Model(sess, cfg, seed=1)
    p = hip.Pool(m, 16, 8)
    d = hip.Decoder(m, p, 2, 4, 64, 16)
    try:
        rows = np.arange(3)
        pt = np.array([[0, -1, -1, -1], [-1] * 4])
        good = dict(slots=[0, -1], row_offsets=rows, positions=[0, 0], page_table=pt,
                    lengths=[1, 0], start_positions=[0, 0])
        d.step_lanes(**good)
        bad = dict(good, slots=[5, -1])
        with pytest.raises(hip.RstrError, match="last token"):
            d.step_lanes(**bad)
        bad = dict(good, lengths=[1, 0], slots=[0, 3])
        with pytest.raises(hip.RstrError, match="inactive"):
            d.step_lanes(**bad)
        bad = dict(good, page_table=np.array([[9, -1, -1, -1], [-1] * 4]), slots=[144, -1])
        with pytest.raises(hip.RstrError):
            d.step_lanes(**bad)
        bad = dict(good, positions=[3, 0])
        with pytest.raises(hip.RstrError, match="position"):
            d.step_lanes(**bad)
        # an idle lane's row is still rotated at its position: it must lie in
        # [0, maxpos) (maxpos 64 here)
        for p_idle in (64, -3, 1 << 30):
            with pytest.raises(hip.RstrError, match="maxpos"):
                d.step_lanes(**dict(good, positions=[0, p_idle]))
        # a route starts at a non-negative position (page_pool.clj:647), even
        # when the query position itself is in range
        bad = dict(good, slots=[2, -1], lengths=[3, 0], start_positions=[-2, 0], positions=[0, 0])
        with pytest.raises(hip.RstrError, match="extents"):
            d.step_lanes(**bad)
        with pytest.raises(hip.RstrError, match="extents"):
            d.step_lanes(**dict(good, start_positions=[0, -1]))
        # the decoder still steps after the rejections
        d.step_lanes(**good)
    finally:
        d.close()
        p.close()
        m.close()


def test_copy_page_copies_every_layer_and_slab(sess):
    cfg = configs.TINY_GEMMA
    m = hip.Model(sess, cfg, seed=1)
    p = hip.Pool(m, 16, 6)
    try:
        p.fill_synthetic([2], seed=5)
        p.copy_page(2, 4)
        for layer in range(cfg["n_layers"]):
            for slab in (0, 1):
                a = p.pages(slab, layer)
                assert np.array_equal(a[2].view(np.uint16), a[4].view(np.uint16))
                assert np.any(a[2] != 0)
    finally:
        p.close()
        m.close()


@pytest.mark.parametrize("case", ["tiny_gemma_q4", "tiny_qwen_q8", "tiny_llama_q4"])
def test_decode_matches_golden_fixture(sess, case):
    """The HIP decoder reproduces the committed oracle digests without running
    the oracle (tests/golden/decode_*.json)."""
    import hashlib
    import json
    import os
    from golden.make_golden import GEOM, schedule_descriptors
    print(f"case golden {case}", flush=True)
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", f"decode_{case}.json")) as f:
        want = json.load(f)["oracle"]
    cfg, B, fills, steps = schedule_descriptors(case)
    g = GEOM
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    m = hip.Model(sess, cfg, seed=g["seed"])
    p = hip.Pool(m, g["ps"], g["pages"])
    d = hip.Decoder(m, p, B, g["pps"], g["maxpos"], g["split"])
    try:
        if fills:
            p.fill_synthetic(fills, g["kv_seed"])
        d.prime_lanes(np.arange(B), (np.arange(B) * 37 + 5) % cfg["vocab"])
        for (active, desc), ws in zip(steps, want["steps"]):
            t = d.step_lanes(**desc)
            act = np.array(active)
            assert [int(x) for x in t[act]] == ws["tokens"]
            assert sha(d.logits()[act]) == ws["logits_sha256"]
        assert sha(d.rows()) == want["rows_sha256"]
        for layer in range(cfg["n_layers"]):
            for slab in (0, 1):
                assert sha(p.pages(slab, layer).view(np.uint16)) == want["pages_sha256"][layer][slab]
    finally:
        d.close()
        p.close()
        m.close()


# ---------------------------------------------------------------------------
# activation blocks outside the scale's [2^-21, 480] range
# ---------------------------------------------------------------------------
def _clamp_case(sess, v_big, plain=False, hip_side=True):
    """Two lanes of tiny_llama.  Lane 0 attends over 60 restored rows whose V
    holds v_big in dims 0..31 of kv head 0 (every layer), so its attention
    output there -- the O projection's input -- lies above 127*480 = 60960.  Lane
    1's input row has a block of 1e-9 (dims 32..63) and one of 1e-6 (64..95), so
    its first normed row carries blocks below 2^-22 and near 2^-20."""
    cfg = configs.TINY_LLAMA
    B, ps, pages, pps, maxpos, split = 2, 16, 8, 4, 64, 16
    pt = np.array([[0, 1, 2, 3], [4, 5, -1, -1]], np.int32)
    lengths = np.array([61, 21], np.int32)
    pos = lengths - 1
    slots = np.array([pt[b, pos[b] // ps] * ps + pos[b] % ps for b in range(B)], np.int32)
    rows = np.arange(B + 1, dtype=np.int32)
    row1 = np.random.default_rng(3).standard_normal(cfg["d_model"]).astype(np.float32)
    row1[32:64] = np.linspace(-1e-9, 1e-9, 32, dtype=np.float32)
    row1[64:96] = np.linspace(-1e-6, 1e-6, 32, dtype=np.float32)
    big = np.zeros((4, ps, cfg["head_dim"]), np.float16)

    def setup(fill, vset, prime_tok, prime_row):
        for pg in range(pages):
            fill(pg)
        for layer in range(cfg["n_layers"]):
            vset(layer)
        prime_tok()
        prime_row()

    out = {}
    om = O.Model(cfg, seed=2)
    od = O.Decoder(om, B, ps, pages, pps, maxpos, kv_f16=True, split=split)
    try:
        if plain:
            O.lib().orc_set_act_scale_plain(1)

        def o_vset(layer):
            v = od.slab(1, layer)
            v[0:4, :, 0, 0:32] = np.float16(v_big)

        setup(lambda pg: od.fill_synthetic(pg, 5), o_vset, lambda: od.prime_lanes([0], [7]),
              lambda: od.prime_rows([1], row1[None]))
        out["oracle"] = (od.step_lanes(slots, rows, pos, pt, lengths, np.zeros(B, np.int32)), od.logits(),
                         od.r0())
    finally:
        O.lib().orc_set_act_scale_plain(0)
        od.close()
    if hip_side:
        m = hip.Model(sess, cfg, seed=2)
        p = hip.Pool(m, ps, pages)
        d = hip.Decoder(m, p, B, pps, maxpos, split)
        try:
            def h_vset(layer):
                v = p.pages(1, layer).copy()
                v[0:4, :, 0, 0:32] = np.float16(v_big)
                p.upload(1, layer, 0, v[0:4])

            setup(lambda pg: p.fill_synthetic([pg], 5), h_vset, lambda: d.prime_lanes([0], [7]),
                  lambda: d.prime_rows([1], row1[None]))
            out["hip"] = (d.step_lanes(slots, rows, pos, pt, lengths, np.zeros(B, np.int32)), d.logits(), d.rows())
        finally:
            d.close(); p.close(); m.close()
    # the first normed row of lane 1 (the layer-0 qkv input) has the intended blocks
    g = om.norm(0, "attn_norm")
    h = O.rmsnorm(row1[None], g, float(cfg["gain_offset"]), float(cfg["eps"]))[0]
    om.close()
    assert np.abs(h[32:64]).max() < 2.0 ** -22 and 2.0 ** -22 < np.abs(h[64:96]).max() < 2.0 ** -19
    return out


def test_activation_scale_clamp_regimes_match_the_oracle(sess):
    """Activation blocks above 60960 saturate (q = +-127 at d = 480) and blocks
    below 2^-22 quantise to zero, on the GPU exactly as in the oracle: tokens,
    logits and next input rows bit for bit.  Saturation is shown end to end: V
    rows of 65504 and of 64512 give the same step (every value of the block
    clamps), while the plain amax/127 scale tells them apart."""
    print("case activation scale clamps", flush=True)
    a = _clamp_case(sess, 65504.0)
    b = _clamp_case(sess, 64512.0)
    for r in (a, b):
        for got, want in zip(r["hip"], r["oracle"]):
            assert np.array_equal(np.asarray(got).view(np.uint32), np.asarray(want).view(np.uint32))
    assert np.array_equal(a["hip"][1].view(np.uint32), b["hip"][1].view(np.uint32))
    pa = _clamp_case(sess, 65504.0, plain=True, hip_side=False)
    pb = _clamp_case(sess, 64512.0, plain=True, hip_side=False)
    assert not np.array_equal(pa["oracle"][1][0], pb["oracle"][1][0])


# ---------------------------------------------------------------------------
# every projection form at every row count and K-slice count
# ---------------------------------------------------------------------------
LINEAR_CFG = configs._desc(n_layers=1, d_model=4096, d_ff=14336, n_q=32, n_kv=8, head_dim=128, vocab=2048,
                           eps=1e-5, rope_global=500000.0, rope_local=500000.0)


@pytest.mark.parametrize("bits", [4, 8])
def test_projection_forms_rows_and_slices_match_the_oracle(sess, bits):
    """rstr_linear_run at Llama-3-8B widths (qkv 6144x4096, o 4096x4096, gate/up
    28672x4096, down 4096x14336): the MFMA tile at 1..4, 16, 64 and 128 rows, the
    one-wave weight-streaming GEMV and its workgroup form at 1..4 rows, each at 1, 2
    and 4 K slices where the form serves the shape, bit for bit against the
    oracle's canonical linear.  Includes the GEMV at two rows with all four K
    quarters in one wave (one slice), the instantiation once seen to lose a
    quarter's partial in a since-replaced chain."""
    cfg = configs.with_bits(LINEAR_CFG, bits)
    print(f"case projection forms q{bits}", flush=True)
    om = O.Model(cfg, seed=7)
    m = hip.Model(sess, cfg, seed=7)
    rng = np.random.default_rng(bits)
    ran = 0
    try:
        weights = {"q": [om.tensor(0, r) for r in ("q", "k", "v")], "o": [om.tensor(0, "o")],
                   "gate": [om.tensor(0, r) for r in ("gate", "up")], "down": [om.tensor(0, "down")]}
        for role, parts in weights.items():
            wq = np.concatenate([p[0] for p in parts])
            ws = np.concatenate([p[1] for p in parts])
            k = wq.shape[1] * 32
            for rows in (1, 2, 3, 4, 16, 64, 128):
                x = (rng.standard_normal((rows, k)) * rng.uniform(0.1, 3.0, (rows, 1))).astype(np.float32)
                xq, xs = O.quant_act(x)
                want = O.qlinear(bits, wq, ws, xq, xs)
                forms = ("tile",) if rows > 4 else ("tile", "wave_gemv", "wg_gemv")
                for form in forms:
                    for splits in (1, 2, 4):
                        try:
                            got = m.linear(0, role, xq, xs, splits, form)
                        except hip.RstrError as e:
                            assert "does not serve" in str(e), e
                            continue
                        ran += 1
                        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (role, rows, form, splits)
        assert ran > 120
    finally:
        m.close()
        om.close()
