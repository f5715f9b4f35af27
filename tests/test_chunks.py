"""Durable KV chunk export/restore: the host mirror (``rstr.chunks``) against the
reference's known answers in ``test/pretrained/continuation_page_pool_test.clj``
(fixture: 2 layers, one kv head of width 2, 4-token pages, 8 pages, fp16 --
:10-23), and the CPU restatement of the device gather/scatter
(``oracle/chunk_oracle.py``) pinned against the reference's ranged-copy plan.

The reference tests check the ranged copies its pool submits (pool offsets,
payload offsets, lengths per slab/layer/run).  Here the same plan comes from
``transfer_runs`` / ``payload_plan`` / ``direct_entries``; the device moves the
whole chunk in one kernel, so the oracle gather -- what the GPU tests compare
the kernel with -- is checked to equal applying that plan slice by slice.
"""
import numpy as np
import pytest

import chunk_oracle as OC
from rstr import chunks
from rstr.page_pool import PagePoolError
from test_page_pool import HEAD_DIM, N_KV, N_LAYERS, PAGE_SIZE, PAGES, fixture_pool

EPT = N_KV * HEAD_DIM
F16 = lambda xs: np.asarray(xs, np.float32).astype(np.float16).view(np.uint16)  # Float/floatToFloat16


class FakeTransfer:
    def __init__(self, payload, nbytes, ready=True):
        self.payload, self.nbytes, self.ready, self.completed = payload, nbytes, ready, False

    def done(self):
        return self.ready

    def complete(self):
        self.completed = True
        return {"bytes": self.nbytes, "device_ms": 0.004, "direction": None, "payload": self.payload}


class NumpyPoolDevice:
    """Pool device over host slabs [K layers, V layers][physical token][ept],
    moving chunks with the oracle gather/scatter."""

    def __init__(self, pages=PAGES, page_size=PAGE_SIZE, layers=N_LAYERS, ept=EPT, ready=True, seed=0):
        rng = np.random.default_rng(seed)
        self.page_size, self.ready = page_size, ready
        self.slabs = [rng.integers(0, 2**15, (pages * page_size, ept)).astype(np.uint16) for _ in range(2 * layers)]
        self.submitted = []

    def copy_page(self, src, dst):
        ps = self.page_size
        for s in self.slabs:
            s[dst * ps:(dst + 1) * ps] = s[src * ps:(src + 1) * ps]

    def export_submit(self, pages, start, count):
        out = OC.gather(self.slabs, pages, self.page_size, start, count)
        t = FakeTransfer(out, out.nbytes, self.ready)
        self.submitted.append(("export", tuple(pages), start, count, t))
        return t

    def restore_submit(self, pages, start, count, payload):
        OC.scatter(self.slabs, pages, self.page_size, start, count, payload)
        t = FakeTransfer(None, np.asarray(payload).nbytes, self.ready)
        self.submitted.append(("restore", tuple(pages), start, count, t))
        return t


def fp16_descriptor(start, count):
    pool = fixture_pool()
    return {"chunk/start": start, "chunk/token-count": count,
            "chunk/layout": {"dtype": "float16", "attention-state": dict(chunks.pool_layout(pool), dtype="float16")}}


def _pool(device, free, refcounts, pages, token_count, start_position=0):
    return fixture_pool(device=device, free=free, refcounts=refcounts,
                        routes={"continuation": {"pages": pages, "token_count": token_count,
                                                 "start_position": start_position}})


def _entries(pool, start, count):
    r = pool.route("continuation")
    layout = chunks.pool_layout(pool)
    return chunks.direct_entries(layout, chunks.payload_plan(layout, count),
                                 chunks.transfer_runs(r, start, count, pool.page_size))


# ---- reference known answers ---------------------------------------------------------
def test_durable_chunk_scatters_across_noncontiguous_physical_pages():
    """continuation_page_pool_test.clj:208-254."""
    dev = NumpyPoolDevice()
    pool = _pool(dev, [0, 2, 4, 6], {1: 1, 3: 1, 5: 1, 7: 1}, [5, 1], 7)
    payload = F16(range(32))  # 2 slabs x 2 layers x 4 tokens x 2 elements/token
    ent = _entries(pool, 2, 4)
    # each slab/layer splits at the logical page boundary
    assert len(ent) == 8
    assert [(e["slab"], e["layer"]) for e in ent] == [("key", 0), ("key", 0), ("key", 1), ("key", 1),
                                                       ("value", 0), ("value", 0), ("value", 1), ("value", 1)]
    # logical tokens 2-3 target physical page 5; 4-5 target page 1
    assert [e["pool-element"] for e in ent] == [44, 8, 44, 8, 44, 8, 44, 8]
    # source slices follow slab/layer payload order
    assert [e["payload-element"] for e in ent] == [0, 4, 8, 12, 16, 20, 24, 28]
    assert all(e["elements"] == 4 for e in ent)
    route = chunks.restore_chunk(pool, "continuation", fp16_descriptor(2, 4), payload)
    assert route.continuation_id == "continuation"
    # the scattered values sit where the plan says
    for i, e in enumerate(ent):
        sl = (0 if e["slab"] == "key" else N_LAYERS) + e["layer"]
        flat = dev.slabs[sl].ravel()
        assert np.array_equal(flat[e["pool-element"]:e["pool-element"] + 4], payload[4 * i:4 * i + 4])
    st = chunks.transfer_stats(pool)
    c = st["counters"][("upload", "device-event", True)]
    assert c["bytes"] == 64 and c["submissions"] == 1
    assert st["calibration"]["gpu-upload-bytes-per-ms"]["count"] == 1
    assert st["calibration"]["gpu-upload-bytes-per-ms"]["ewma"] > 0


def test_durable_chunk_coalesces_contiguous_physical_pages():
    """continuation_page_pool_test.clj:256-287."""
    pool = _pool(NumpyPoolDevice(), [0, 3, 4, 5, 6, 7], {1: 1, 2: 1}, [1, 2], 8)
    ent = _entries(pool, 2, 4)
    assert len(ent) == 4, "one contiguous run is submitted for each slab/layer"
    assert [e["pool-element"] for e in ent] == [12, 12, 12, 12]
    assert [e["payload-element"] for e in ent] == [0, 8, 16, 24]
    assert all(e["elements"] == 8 for e in ent)
    chunks.restore_chunk(pool, "continuation", fp16_descriptor(2, 4), np.zeros(32, np.uint16))


class Retained:
    def __init__(self):
        self.closed = False

    def close(self):
        self.closed = True


def test_submitted_restore_retains_its_resource_through_device_completion():
    """continuation_page_pool_test.clj:289-340."""
    dev = NumpyPoolDevice(ready=False)
    pool = _pool(dev, [0, 3, 4, 5, 6, 7], {1: 1, 2: 1}, [1, 2], 8)
    res = Retained()
    tr = chunks.submit_restore_chunk(pool, "continuation", fp16_descriptor(2, 4), np.zeros(32, np.uint16), [res])
    assert isinstance(tr, chunks.ChunkTransfer)
    assert tr.retained == [res]
    assert chunks.chunk_transfer_complete(pool, tr) is False
    assert not res.closed
    tr.transfer.ready = True
    assert chunks.chunk_transfer_complete(pool, tr) is True
    assert chunks.complete_restore_chunk(pool, tr).continuation_id == "continuation"
    assert res.closed
    assert chunks.transfer_stats(pool)["counters"][("upload", "device-event", True)]["bytes"] == 64


def test_submitted_export_retains_its_route_through_device_completion():
    """continuation_page_pool_test.clj:342-395."""
    dev = NumpyPoolDevice(ready=False)
    pool = _pool(dev, [0, 3, 4, 5, 6, 7], {1: 1, 2: 1}, [1, 2], 8)
    ex = chunks.submit_export_chunk(pool, "continuation", "fixture-paged-v1",
                                    {"chunk/start": 2, "chunk/token-count": 4})
    assert isinstance(ex, chunks.ChunkExport)
    assert len(_entries(pool, 2, 4)) == 4
    assert pool.stats()["active-leases"] == 1
    assert chunks.chunk_export_complete(pool, ex) is False
    ex.transfer.ready = True
    assert chunks.chunk_export_complete(pool, ex) is True
    chunk = chunks.complete_export_chunk(pool, ex)
    want = OC.gather(dev.slabs, [1, 2], PAGE_SIZE, 2, 4)
    assert np.array_equal(chunk["chunk/payload"], want)
    assert pool.stats()["active-leases"] == 0
    assert chunks.transfer_stats(pool)["counters"][("download", "device-event", True)]["bytes"] == 64


def test_rejected_export_submission_releases_its_route_lease():
    """continuation_page_pool_test.clj:397-414."""
    class Rejecting(NumpyPoolDevice):
        def export_submit(self, *a):
            raise RuntimeError("rejected")
    pool = _pool(Rejecting(), [0, 3, 4, 5, 6, 7], {1: 1, 2: 1}, [1, 2], 8)
    with pytest.raises(RuntimeError):
        chunks.submit_export_chunk(pool, "continuation", "fixture-paged-v1",
                                   {"chunk/start": 0, "chunk/token-count": 4})
    assert pool.stats()["active-leases"] == 0


def test_resident_pages_gather_into_the_portable_durable_chunk_layout():
    """continuation_page_pool_test.clj:482-522: the export entries cover the
    payload exactly once (the reference's mock writes dst-element + index + 1
    and expects 1..32), and the durable map is version 3 / fp16."""
    dev = NumpyPoolDevice()
    pool = _pool(dev, [0, 2, 4, 6], {1: 1, 3: 1, 5: 1, 7: 1}, [5, 1], 7)
    ent = _entries(pool, 2, 4)
    assert len(ent) == 8, "every slab/layer splits at the physical page boundary"
    covered = np.zeros(32, np.int32)
    for e in ent:
        covered[e["payload-element"]:e["payload-element"] + e["elements"]] += 1
    assert covered.tolist() == [1] * 32
    chunk = chunks.export_chunk(pool, "continuation", "fixture-paged-v1", {"chunk/start": 2, "chunk/token-count": 4})
    assert chunk["chunk/version"] == 3
    assert chunk["chunk/model-fingerprint"] == "fixture-paged-v1"
    assert chunk["chunk/layout"]["dtype"] == "float16"
    assert chunk["chunk/layout"]["attention-state"]["byte-order"] == "little-endian"
    assert chunk["chunk/elements-per-slab"] == 8
    assert [e["element-offset"] for e in chunk["chunk/slabs"]] == [0, 8, 16, 24]
    assert chunk["chunk/payload"].size == 32
    assert pool.stats()["active-leases"] == 0


# ---- validation ---------------------------------------------------------------------
def test_restore_and_export_validation():
    dev = NumpyPoolDevice()
    pool = _pool(dev, [0, 2, 4, 6], {1: 1, 3: 1, 5: 1, 7: 1}, [5, 1], 7)
    z = np.zeros(32, np.uint16)
    with pytest.raises(PagePoolError, match="nonresident"):
        chunks.restore_chunk(pool, "other", fp16_descriptor(0, 4), z)
    with pytest.raises(PagePoolError, match="outside the resident"):
        chunks.restore_chunk(pool, "continuation", fp16_descriptor(4, 4), z)
    with pytest.raises(PagePoolError, match="outside the resident"):
        chunks.restore_chunk(pool, "continuation", fp16_descriptor(0, 0), np.zeros(0, np.uint16))
    bad = fp16_descriptor(0, 4)
    bad["chunk/layout"]["attention-state"] = dict(bad["chunk/layout"]["attention-state"], kind="mla")
    with pytest.raises(PagePoolError, match="layout differs"):
        chunks.restore_chunk(pool, "continuation", bad, z)
    with pytest.raises(PagePoolError, match="FP16 payload length"):
        chunks.restore_chunk(pool, "continuation", fp16_descriptor(0, 4), np.zeros(31, np.uint16))
    with pytest.raises(PagePoolError, match="cannot be restored"):
        chunks.restore_chunk(pool, "continuation", fp16_descriptor(0, 4), np.zeros(32, np.float64))
    f32 = fp16_descriptor(0, 4)
    f32["chunk/layout"]["attention-state"] = dict(f32["chunk/layout"]["attention-state"], dtype="float32")
    with pytest.raises(PagePoolError, match="FP32 payload length"):
        chunks.restore_chunk(pool, "continuation", f32, np.zeros(30, np.float32))
    res = pool.reserve_append("continuation")
    with pytest.raises(PagePoolError, match="append is pending"):
        chunks.restore_chunk(pool, "continuation", fp16_descriptor(0, 4), z)
    pool.abort_append("continuation", res)
    shifted = _pool(NumpyPoolDevice(), [0, 2, 4, 6], {1: 1, 3: 1, 5: 1, 7: 1}, [5, 1], 7, start_position=3)
    with pytest.raises(PagePoolError, match="zero absolute start"):
        chunks.export_chunk(shifted, "continuation", "fp", {"chunk/start": 0, "chunk/token-count": 2})
    assert shifted.stats()["active-leases"] == 0
    other = chunks.submit_export_chunk(pool, "continuation", "fp", {"chunk/start": 0, "chunk/token-count": 2})
    with pytest.raises(PagePoolError, match="different page pool"):
        chunks.complete_export_chunk(shifted, other)
    chunks.complete_export_chunk(pool, other)


def test_f32_restore_rounds_to_nearest_even():
    """half-payload (page_pool.clj:1084-1109) with Float/floatToFloat16: ties
    between fp16 neighbours go to the even one."""
    dev = NumpyPoolDevice()
    pool = _pool(dev, [0, 2, 4, 6], {1: 1, 3: 1, 5: 1, 7: 1}, [5, 1], 7)
    # 1 + 2^-11 is half-way between 1 and 1 + 2^-10 -> 1; 1 + 3*2^-11 -> 1 + 2^-9
    vals = np.array([1 + 2**-11, 1 + 3 * 2**-11, -2.5, 65504.0, 1e-8, 0.1] + [0.5] * 26, np.float32)
    desc = fp16_descriptor(0, 4)
    desc["chunk/layout"]["attention-state"] = dict(desc["chunk/layout"]["attention-state"], dtype="float32")
    chunks.restore_chunk(pool, "continuation", desc, vals)
    got = OC.gather(dev.slabs, [5, 1], PAGE_SIZE, 0, 4).view(np.float16)
    assert got[0] == np.float16(1.0) and got[1] == np.float16(1 + 2**-9)
    assert got[:6].tolist() == [1.0, 1.0 + 2**-9, -2.5, 65504.0, 0.0, float(np.float16(0.1))]


# ---- the oracle gather against the reference's ranged-copy plan ------------------------------
@pytest.mark.parametrize("seed", range(6))
def test_oracle_gather_equals_the_reference_ranged_copies(seed):
    rng = np.random.default_rng(seed)
    ps, P, L, ept = int(rng.choice([4, 16])), 24, 3, 8
    dev = NumpyPoolDevice(P, ps, L, ept, seed=seed)
    n_pages = int(rng.integers(1, 8))
    pages = [int(p) for p in rng.permutation(P)[:n_pages]]
    if seed % 2:  # force some physically adjacent pages (coalesced runs)
        pages = sorted(pages)
    tokens = n_pages * ps - int(rng.integers(0, ps))
    start = int(rng.integers(0, tokens))
    count = int(rng.integers(1, tokens - start + 1))
    from rstr.page_pool import PagePool, Route
    pool = PagePool(ps, P, L, 1, ept, "half", device=dev)
    pool.routes = {"c": Route("c", tuple(pages), tokens, 0)}
    layout = chunks.pool_layout(pool)
    plan = chunks.payload_plan(layout, count)
    ent = chunks.direct_entries(layout, plan, chunks.transfer_runs(pool.route("c"), start, count, ps))
    want = np.zeros(2 * L * count * ept, np.uint16)
    for e in ent:
        sl = (0 if e["slab"] == "key" else L) + e["layer"]
        flat = dev.slabs[sl].ravel()
        want[e["payload-element"]:e["payload-element"] + e["elements"]] = \
            flat[e["pool-element"]:e["pool-element"] + e["elements"]]
    got = chunks.export_chunk(pool, "c", "fp", {"chunk/start": start, "chunk/token-count": count})["chunk/payload"]
    assert np.array_equal(got, want)
    # round trip into a fresh route of other pages
    free = [p for p in range(P) if p not in pages][:n_pages]
    pool.routes["d"] = Route("d", tuple(free), tokens, 0)
    chunks.restore_chunk(pool, "d", dict(fp16_descriptor(start, count), **{
        "chunk/layout": {"dtype": "float16", "attention-state": dict(layout, dtype="float16")}}), got)
    back = chunks.export_chunk(pool, "d", "fp", {"chunk/start": start, "chunk/token-count": count})["chunk/payload"]
    assert np.array_equal(back, got)


def test_calibration_is_an_ewma_with_alpha_one_fifth():
    """telemetry.clj:4-52."""
    pool = fixture_pool()
    for b, wall in ((1000, 2_000_000), (3000, 1_000_000)):
        chunks.record_transfer(pool, {"direction": "download", "timing-source": "device-event", "asynchronous?": True,
                                      "bytes": b, "commands": 1, "elapsed-ns": 10, "submit-host-ns": 1,
                                      "host-wall-ns": wall})
    cal = chunks.transfer_stats(pool)["calibration"]["gpu-download-bytes-per-ms"]
    assert cal["count"] == 2 and cal["minimum"] == 500.0 and cal["maximum"] == 3000.0
    assert cal["ewma"] == pytest.approx(0.2 * 3000.0 + 0.8 * 500.0)
    c = chunks.transfer_stats(pool)["counters"][("download", "device-event", True)]
    assert (c["submissions"], c["bytes"], c["host-wall-ns"]) == (2, 4000, 3_000_000)
