"""The device-owning continuous-batching loop (``rstr.paged_runtime``): one test
per reference test in ``test/pretrained/continuation_paged_runtime_test.clj``,
with the same simulated decoder callbacks (tokens 100 + position, per-route
token counters) and the same expected schedules."""
import threading
import time
from concurrent.futures import CancelledError, ThreadPoolExecutor

import pytest

from rstr import paged_runtime as pr


class Dec:
    def __init__(self, batch, maxpos=64):
        self.batch_size, self.maxpos = batch, maxpos


def effect(aid, cid, tokens, max_new):
    """continuation_paged_runtime_test.clj:6-14."""
    return {"id": aid, "request": {"id": aid, "continuation_id": cid, "model_fingerprint": "fixture-model-v1",
                                   "tokens": list(tokens), "max_new_tokens": max_new}}


def await_value(timeout_s, fn):
    end = time.time() + timeout_s
    while True:
        v = fn()
        if v:
            return v
        if time.time() > end:
            raise AssertionError("Timed out waiting for paged runtime state")
        time.sleep(0.005)


POOL = ThreadPoolExecutor(8)


def test_prefill_and_decode_share_sparse_fixed_lanes():
    """:27-79."""
    counts = {"prefill": 0, "decode": 2}
    primes, subs = [], []
    first, release = threading.Event(), threading.Event()
    calls = [0]

    def step(_, work):
        subs.append(work)
        calls[0] += 1
        if calls[0] == 1:
            first.set()
            release.wait(5)
        out = []
        for it in work:
            counts[it["continuation_id"]] += 1
            out.append({**it, "token": 100 + it["position"]})
        return out

    rt = pr.open_runtime(Dec(3), prime_lanes=lambda _, v: primes.append(v), step_lanes=step,
                         route_token_count=lambda _, cid: counts[cid])
    try:
        pf = POOL.submit(rt.prefill, effect("prefill-assignment", "prefill", [1, 2, 3, 4, 5], 2))
        assert first.wait(1)
        deltas = []
        dc = POOL.submit(rt.decode, effect("decode-assignment", "decode", [7, 8, 9], 3),
                         lambda tok, i: deltas.append((tok, i)))
        time.sleep(0.05)
        release.set()
        assert pf.result(1) == {"ok?": True}
        assert dc.result(1) == {"ok?": True, "tokens": [102, 103, 104], "stop-reason": "length"}
        assert deltas == [(102, 0), (103, 1), (104, 2)]
        assert any({w["continuation_id"] for w in s} == {"prefill", "decode"} for s in subs)
        assert any(len(p) == 2 and 9 in {x["token"] for x in p} for p in primes), \
            "a prompt token and refilled decode token are primed together"
        assert counts["prefill"] == 4 and counts["decode"] == 5
        assert rt.state()["scheduled-tokens"] >= 7
    finally:
        release.set()
        rt.close()


def test_cancelled_assignment_leaves_after_the_current_step():
    """:81-121 (the reference interrupts the handler thread; here the
    assignment is cancelled, the path the interrupt takes)."""
    counts = {"decode": 2}
    entered, release = threading.Event(), threading.Event()

    def step(_, work):
        entered.set()
        release.wait(5)
        out = []
        for it in work:
            counts[it["continuation_id"]] += 1
            out.append({**it, "token": 100 + it["position"]})
        return out

    rt = pr.open_runtime(Dec(1), prime_lanes=lambda *a: None, step_lanes=step,
                         route_token_count=lambda _, cid: counts[cid])
    try:
        task = POOL.submit(rt.decode, effect("decode-assignment", "decode", [7, 8, 9], 20))
        assert entered.wait(1)
        assert rt.cancel_assignment("decode-assignment") == 1
        release.set()
        with pytest.raises(CancelledError):
            task.result(1)
        await_value(1, lambda: counts["decode"] >= 3 and all(l is None for l in rt.state()["lanes"]))
        after = counts["decode"]
        time.sleep(0.03)
        assert counts["decode"] == after and after <= 3
    finally:
        release.set()
        rt.close()


def test_background_restore_does_not_block_unrelated_decode_lanes():
    """:123-160."""
    counts = {"decode": 2}
    entered, release = threading.Event(), threading.Event()

    def step(_, work):
        out = []
        for it in work:
            counts[it["continuation_id"]] += 1
            out.append({**it, "token": 100 + it["position"]})
        return out

    rt = pr.open_runtime(Dec(1), prime_lanes=lambda *a: None, step_lanes=step,
                         route_token_count=lambda _, cid: counts[cid])
    try:
        def restore(_cancelled):
            entered.set()
            release.wait(5)
            return {"ok?": True}
        rs = POOL.submit(rt.run_background_operation, "restore-assignment", restore)
        assert entered.wait(1)
        dc = POOL.submit(rt.decode, effect("decode-assignment", "decode", [7, 8, 9], 2))
        assert dc.result(1) == {"ok?": True, "tokens": [102, 103], "stop-reason": "length"}
        assert not rs.done(), "decode completes while the independent restore boundary is pending"
        release.set()
        assert rs.result(1) == {"ok?": True}
    finally:
        release.set()
        rt.close()


def test_decode_rejects_an_incomplete_prompt_without_poisoning_the_runtime():
    """:162-177."""
    rt = pr.open_runtime(Dec(2), prime_lanes=lambda *a: None, step_lanes=lambda *a: [],
                         route_token_count=lambda *a: 1)
    try:
        with pytest.raises(pr.RuntimeError_, match="completely primed"):
            rt.decode(effect("decode-assignment", "decode", [7, 8, 9], 2))
        assert rt.state()["iterations"] == 0
    finally:
        rt.close()


def test_single_lane_prefill_uses_exact_bulk_tiles_and_a_scalar_tail():
    """:179-221."""
    counts = {"prefill": 0}
    bulk, scalar = [], []

    def prefill_range(_, cid, tokens, position):
        bulk.append((cid, list(tokens), position))
        counts[cid] += len(tokens)

    def step(_, work):
        out = []
        for it in work:
            scalar.append((it["continuation_id"], it["position"]))
            counts[it["continuation_id"]] += 1
            out.append({**it, "token": 100 + it["position"]})
        return out

    rt = pr.open_runtime(Dec(1), prefill_tile_size=3, prefill_range=prefill_range, prime_lanes=lambda *a: None,
                         step_lanes=step, route_token_count=lambda _, cid: counts[cid])
    try:
        assert rt.prefill(effect("prefill-assignment", "prefill", [10, 11, 12, 13, 14, 15, 16, 17], 1)) == \
            {"ok?": True}
        assert bulk == [("prefill", [10, 11, 12], 0), ("prefill", [13, 14, 15], 3)]
        assert scalar == [("prefill", 6)]
        assert counts["prefill"] == 7
        st = rt.state()
        assert st["bulk-prefill-tiles"] == 2 and st["bulk-prefill-tokens"] == 6
        assert st["prefill-tile-size"] == 3
        assert isinstance(st["bulk-prefill-ms-per-token"], float)
        assert st["calibration"]["prefill-ms-per-token"]["count"] == 3
        assert isinstance(st["calibration"]["prefill-ms-per-token"]["ewma"], float)
        assert st["scheduled-tokens"] == 7
    finally:
        rt.close()


def test_decode_preempts_prefill_at_the_next_bulk_tile_boundary():
    """:223-270."""
    counts = {"prefill": 0, "decode": 2}
    calls = []
    entered, release = threading.Event(), threading.Event()

    def prefill_range(_, cid, tokens, position):
        calls.append(("bulk", cid, position))
        if position == 0:
            entered.set()
            release.wait(5)
        counts[cid] += len(tokens)

    def step(_, work):
        out = []
        for it in work:
            calls.append(("step", it["continuation_id"], it["position"]))
            counts[it["continuation_id"]] += 1
            out.append({**it, "token": 100 + it["position"]})
        return out

    rt = pr.open_runtime(Dec(1), prefill_tile_size=3, prefill_range=prefill_range, prime_lanes=lambda *a: None,
                         step_lanes=step, route_token_count=lambda _, cid: counts[cid])
    try:
        pf = POOL.submit(rt.prefill, effect("prefill-assignment", "prefill", [10, 11, 12, 13, 14, 15, 16, 17], 1))
        assert entered.wait(1)
        dc = POOL.submit(rt.decode, effect("decode-assignment", "decode", [7, 8, 9], 1))
        await_value(1, lambda: rt.state()["active-job-count"] == 2)
        release.set()
        assert dc.result(1) == {"ok?": True, "tokens": [102], "stop-reason": "length"}
        assert pf.result(1) == {"ok?": True}
        assert calls == [("bulk", "prefill", 0), ("step", "decode", 2), ("bulk", "prefill", 3),
                         ("step", "prefill", 6)]
    finally:
        release.set()
        rt.close()


def test_runtime_options_are_validated():
    """open-runtime's checks (paged_runtime.clj:362-405)."""
    with pytest.raises(pr.RuntimeError_, match="exceeds the decoder"):
        pr.open_runtime(Dec(1), capacity=2)
    with pytest.raises(pr.RuntimeError_, match="one runtime lane"):
        pr.open_runtime(Dec(2), prefill_tile_size=3, prefill_range=lambda *a: None)
    with pytest.raises(pr.RuntimeError_, match="alpha"):
        pr.open_runtime(Dec(1), calibration_alpha=0.0)
    rt = pr.open_runtime(Dec(1))
    rt.close()
    with pytest.raises(pr.RuntimeError_, match="closed"):
        rt.run_operation(lambda: 1)


def _runtime_vs_generate(make_device, pool_device, cfg):
    from rstr.page_pool import PagePool
    from rstr.paged_decoder import PagedDecoder
    from test_prefill import MAXPOS, PAGES, PPS, PS, T, _prompt
    prompt = _prompt(cfg)
    pool = PagePool(PS, PAGES, cfg["n_layers"], cfg["n_kv"], cfg["head_dim"], device=pool_device)
    dec = PagedDecoder(pool, make_device(), batch_size=1, maxpos=MAXPOS, pages_per_sequence=PPS, prefill_T=T)
    want = dec.generate("ref", prompt, 5)
    dec.allocate_continuation("rt")
    with pr.open_runtime(dec) as rt:
        assert rt.prefill(effect("a", "rt", prompt, 5)) == {"ok?": True}
        got = rt.decode(effect("a", "rt", prompt, 5))
        st = rt.state()
    assert got == {"ok?": True, "tokens": want, "stop-reason": "length"}
    assert st["bulk-prefill-tiles"] == (len(prompt) - 1) // T
    return got


def test_runtime_over_the_oracle_decoder_equals_direct_generation():
    """The runtime driving a real paged decoder (the oracle device, bulk tiles
    and a scalar tail) produces the tokens direct generation does."""
    import oracle as O
    from rstr import configs
    from test_prefill import MAXPOS, PAGES, PPS, PS, SEED, SPLIT, T, OracleDevice
    cfg = configs.MODELS["tiny_llama"]
    om = O.Model(cfg, seed=SEED)
    od = O.Decoder(om, T, PS, PAGES, PPS, MAXPOS, kv_f16=True, split=SPLIT)
    try:
        _runtime_vs_generate(lambda: OracleDevice(od), od, cfg)
    finally:
        od.close()
        om.close()


@pytest.mark.gpu
def test_runtime_over_the_hip_decoder_equals_direct_generation():
    print("case runtime hip", flush=True)
    from rstr import configs, hip
    from rstr.paged_decoder import HipStepDevice
    from test_prefill import MAXPOS, PAGES, PPS, PS, SEED, SPLIT, T
    cfg = configs.MODELS["tiny_llama"]
    with hip.Session(0) as sess:
        m = hip.Model(sess, cfg, seed=SEED)
        p = hip.Pool(m, PS, PAGES)
        d = hip.Decoder(m, p, 1, PPS, MAXPOS, SPLIT)
        pf = hip.Prefill(m, p, T, PPS, MAXPOS, SPLIT)
        _runtime_vs_generate(lambda: HipStepDevice(d, pf), p, cfg)
