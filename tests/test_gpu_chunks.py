"""Durable chunk export/restore on the GPU (``rstr_chunk_export_submit`` /
``rstr_chunk_restore_submit`` through the page-pool mirror) against the CPU
gather/scatter of ``oracle/chunk_oracle.py`` on the same slabs, bit for bit:
ranges that start and end inside pages, fragmented and contiguous page lists,
fp16 and f32 payloads, overlapping asynchronous transfers, a Llama-shaped pool,
and the error paths."""
import numpy as np
import pytest

import chunk_oracle as OC
from rstr import chunks, configs, hip
from rstr.page_pool import PagePool, Route

pytestmark = pytest.mark.gpu

CFG = configs.MODELS["tiny_llama"]


def _slabs(p, L):
    """Host copies of the pool's 2L slabs as [physical token][ept] uint16."""
    ept = p.model.cfg["n_kv"] * p.model.cfg["head_dim"]
    return [p.pages(s, l).view(np.uint16).reshape(-1, ept).copy() for s in (0, 1) for l in range(L)]


def _mirror(p, ps, P, cfg):
    return PagePool(ps, P, cfg["n_layers"], cfg["n_kv"], cfg["head_dim"], "half", device=p)


def _desc(pool, start, count, dtype="float16"):
    lay = chunks.pool_layout(pool)
    return {"chunk/start": start, "chunk/token-count": count,
            "chunk/layout": {"dtype": dtype, "attention-state": dict(lay, dtype=dtype)}}


@pytest.mark.parametrize("ps,case", [(16, "mid-page"), (16, "single"), (16, "whole"), (4, "fragmented"),
                                     (16, "contiguous")])
def test_export_and_restore_match_the_oracle(ps, case):
    print("case chunk", ps, case, flush=True)
    P, L = 48, CFG["n_layers"]
    rng = np.random.default_rng(ps * 7 + len(case))
    with hip.Session(0) as sess:
        m = hip.Model(sess, CFG, seed=2)
        p = hip.Pool(m, ps, P)
        p.fill_synthetic(np.arange(P, dtype=np.int32), 11)
        pool = _mirror(p, ps, P, CFG)
        n = 9
        pages = list(range(3, 3 + n)) if case == "contiguous" else [int(x) for x in rng.permutation(P)[:n]]
        tokens = n * ps - 3
        start, count = {"mid-page": (5, 2 * ps + 3), "single": (ps + 2, 1), "whole": (0, tokens),
                        "fragmented": (1, tokens - 2), "contiguous": (3, 5 * ps)}[case]
        pool.routes = {"a": Route("a", tuple(pages), tokens, 0)}
        before = _slabs(p, L)
        chunk = chunks.export_chunk(pool, "a", "fp", {"chunk/start": start, "chunk/token-count": count})
        want = OC.gather(before, pages, ps, start, count)
        assert chunk["chunk/payload"].dtype == np.uint16
        assert np.array_equal(chunk["chunk/payload"], want)
        # restore a different payload into another route of other pages
        others = [x for x in range(P) if x not in pages][:n]
        pool.routes["b"] = Route("b", tuple(others), tokens, 0)
        payload = rng.integers(0, 2**15, want.size).astype(np.uint16)
        chunks.restore_chunk(pool, "b", _desc(pool, start, count), payload)
        expect = [s.copy() for s in before]
        OC.scatter(expect, others, ps, start, count, payload)
        after = _slabs(p, L)
        for i in range(2 * L):
            assert np.array_equal(after[i], expect[i]), i
        st = chunks.transfer_stats(pool)["counters"]
        assert st[("download", "device-event", True)]["bytes"] == want.nbytes
        assert st[("upload", "device-event", True)]["bytes"] == payload.nbytes


def test_f32_payload_rounds_like_the_oracle():
    print("case chunk f32", flush=True)
    ps, P, L = 16, 16, CFG["n_layers"]
    with hip.Session(0) as sess:
        m = hip.Model(sess, CFG, seed=2)
        p = hip.Pool(m, ps, P)
        pool = _mirror(p, ps, P, CFG)
        pool.routes = {"a": Route("a", (7, 2, 9), 40, 0)}
        count = 33
        rng = np.random.default_rng(5)
        vals = (rng.standard_normal(p.chunk_elements(count)) * 300).astype(np.float32)
        vals[:4] = [1 + 2**-11, 1 + 3 * 2**-11, 70000.0, -1e-9]
        before = _slabs(p, L)
        chunks.restore_chunk(pool, "a", _desc(pool, 4, count, "float32"), vals)
        expect = [s.copy() for s in before]
        OC.scatter(expect, [7, 2, 9], ps, 4, count, vals)
        after = _slabs(p, L)
        for i in range(2 * L):
            assert np.array_equal(after[i], expect[i]), i


def test_overlapping_transfers_complete_in_any_order():
    print("case chunk async", flush=True)
    ps, P, L = 16, 32, CFG["n_layers"]
    with hip.Session(0) as sess:
        m = hip.Model(sess, CFG, seed=2)
        p = hip.Pool(m, ps, P)
        p.fill_synthetic(np.arange(P, dtype=np.int32), 3)
        pool = _mirror(p, ps, P, CFG)
        pool.routes = {"a": Route("a", (4, 1, 8, 3), 60, 0), "b": Route("b", (10, 11, 12), 40, 0)}
        before = _slabs(p, L)
        e1 = chunks.submit_export_chunk(pool, "a", "fp", {"chunk/start": 0, "chunk/token-count": 60})
        payload = np.arange(p.chunk_elements(40), dtype=np.uint16)
        res = chunks.submit_restore_chunk(pool, "b", _desc(pool, 0, 40), payload)
        e2 = chunks.submit_export_chunk(pool, "b", "fp", {"chunk/start": 0, "chunk/token-count": 40})
        assert pool.stats()["active-leases"] == 2
        with pytest.raises(hip.RstrError, match="in flight"):
            p.close()
        c2 = chunks.complete_export_chunk(pool, e2)     # stream order: after the restore
        assert np.array_equal(c2["chunk/payload"], payload)
        chunks.complete_restore_chunk(pool, res)
        c1 = chunks.complete_export_chunk(pool, e1)
        assert np.array_equal(c1["chunk/payload"], OC.gather(before, [4, 1, 8, 3], ps, 0, 60))
        assert pool.stats()["active-leases"] == 0
        assert chunks.chunk_transfer_complete(pool, res) is True


def test_llama_shaped_pool_round_trip():
    print("case chunk llama", flush=True)
    cfg = dict(configs.MODELS["llama3_8b"], n_layers=4)
    ps, P, L = 16, 300, 4
    rng = np.random.default_rng(9)
    with hip.Session(0) as sess:
        m = hip.Model(sess, cfg, seed=1)
        p = hip.Pool(m, ps, P)
        p.fill_synthetic(np.arange(P, dtype=np.int32), 8)
        pool = _mirror(p, ps, P, cfg)
        pages = [int(x) for x in rng.permutation(P)[:140]]
        pool.routes = {"a": Route("a", tuple(pages), 140 * ps, 0)}
        before = _slabs(p, L)
        chunk = chunks.export_chunk(pool, "a", "fp", {"chunk/start": 7, "chunk/token-count": 2000})
        assert np.array_equal(chunk["chunk/payload"], OC.gather(before, pages, ps, 7, 2000))
        others = [x for x in range(P) if x not in pages][:140]
        pool.routes["b"] = Route("b", tuple(others), 140 * ps, 0)
        chunks.restore_chunk(pool, "b", _desc(pool, 7, 2000), chunk["chunk/payload"])
        back = chunks.export_chunk(pool, "b", "fp", {"chunk/start": 7, "chunk/token-count": 2000})
        assert np.array_equal(back["chunk/payload"], chunk["chunk/payload"])


def test_device_rejects_bad_ranges_and_dtypes():
    print("case chunk errors", flush=True)
    with hip.Session(0) as sess:
        m = hip.Model(sess, CFG, seed=2)
        p = hip.Pool(m, 16, 8)
        with pytest.raises(hip.RstrError, match="outside"):
            p.export_submit([1, 2], 20, 13)
        with pytest.raises(hip.RstrError, match="page id"):
            p.export_submit([1, 99], 10, 10)
        with pytest.raises(hip.RstrError, match="outside"):
            p.export_submit([1, 2], 0, 0)
        with pytest.raises(ValueError, match="cannot be restored"):
            p.restore_submit([1], 0, 2, np.zeros(p.chunk_elements(2), np.int32))
        t = p.restore_submit([1], 0, 2, np.zeros(p.chunk_elements(2), np.uint16))
        st = t.complete()
        assert st["bytes"] == p.chunk_elements(2) * 2 and st["direction"] == "upload"
        with pytest.raises(hip.RstrError, match="already completed"):
            t.complete()


def test_restored_prefix_continues_exactly_like_the_original_route():
    """Export a route's first 48 tokens (computed through bulk prefill tiles),
    restore them into a fresh route, and generate from the same prompt: only the
    uncached suffix is computed (paged_decoder.clj:774-813) and the tokens equal
    the original route's."""
    print("case chunk restore then decode", flush=True)
    from rstr.paged_decoder import HipStepDevice, PagedDecoder
    ps, P, maxpos, T = 16, 40, 128, 24
    pps = maxpos // ps
    prompt = [int(x) for x in np.random.default_rng(4).integers(0, CFG["vocab"], 61)]
    with hip.Session(0) as sess:
        m = hip.Model(sess, CFG, seed=6)
        p = hip.Pool(m, ps, P)
        d = hip.Decoder(m, p, 1, pps, maxpos, 16)
        pf = hip.Prefill(m, p, T, pps, maxpos, 16)
        pool = _mirror(p, ps, P, CFG)
        dev = HipStepDevice(d, pf)
        dec = PagedDecoder(pool, dev, batch_size=1, maxpos=maxpos, pages_per_sequence=pps, prefill_T=T)
        want = dec.generate("a", prompt, 6)
        chunk = chunks.export_chunk(pool, "a", "fp", {"chunk/start": 0, "chunk/token-count": 48})
        pool.allocate_route("b", 48)
        chunks.restore_chunk(pool, "b", _desc(pool, 0, 48), chunk["chunk/payload"])
        ran = []
        orig = dev.run_prefill
        dev.run_prefill = lambda: (ran.append(1), orig())
        got = dec.generate("b", prompt, 6)
        assert got == want
        assert ran == []  # the restored 48 tokens are not recomputed; 12 suffix tokens decode singly
        # the restored route's pages hold the same K/V as the original's over the prefix
        ra, rb = pool.route("a"), pool.route("b")
        slabs = _slabs(p, CFG["n_layers"])
        assert np.array_equal(OC.gather(slabs, ra.pages, ps, 0, 60), OC.gather(slabs, rb.pages, ps, 0, 60))
