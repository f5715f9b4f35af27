"""Known-answer tests of the page-pool mirror, one per reference test in
``test/pretrained/continuation_page_pool_test.clj`` that exercises the decode
path's bookkeeping (capacity, routes, copy-on-write, ranges, leases, dense
tables, forks).  The fixture matches the reference's: a 2-layer model with one
kv head of width 2, 4-token pages, 8 physical pages, fp16 storage
(continuation_page_pool_test.clj:10-23).  The device is a recorder: one
``copy_page`` call stands for the reference's per-(slab, layer) copy-range!
calls, so it is expanded here into (slab, layer, elements) copies.
"""
import pytest
from sortedcontainers import SortedSet

from rstr.page_pool import PagePool, PagePoolError, Route, dense_values

N_LAYERS, N_KV, HEAD_DIM, PAGE_SIZE, PAGES = 2, 1, 2, 4, 8


class CopyRecorder:
    def __init__(self):
        self.pages = []

    def copy_page(self, src, dst):
        self.pages.append((src, dst))

    def range_copies(self):
        """The reference's copy-range! calls: every slab and layer of the page."""
        elems = PAGE_SIZE * N_KV * HEAD_DIM
        return [(slab, layer, src, dst, elems) for (src, dst) in self.pages
                for slab in ("key", "value") for layer in range(N_LAYERS)]


def fixture_pool(device=None, free=None, refcounts=None, routes=None):
    pool = PagePool(PAGE_SIZE, PAGES, N_LAYERS, N_KV, HEAD_DIM, "half", device=device or CopyRecorder())
    if free is not None:
        pool.free = SortedSet(free)
    if refcounts is not None:
        pool.refcounts = dict(refcounts)
    if routes is not None:
        pool.routes = {cid: Route(cid, tuple(r["pages"]), r["token_count"], r.get("start_position", 0))
                       for cid, r in routes.items()}
    return pool


def test_projected_capacity_is_held_through_restore_and_growth():
    """continuation_page_pool_test.clj:26-48."""
    pool = fixture_pool()
    cap = pool.reserve_capacity("request", 10)
    assert pool.free_page_count() == 5
    st = pool.stats()
    assert (st["capacity-reservations"], st["reserved-pages"]) == (1, 3)
    pool.allocate_route("request", 4, capacity_reservation=cap)
    assert pool.stats()["reserved-pages"] == 2
    for _ in range(6):
        pool.commit_append("request", pool.reserve_append("request"))
    assert pool.route("request").token_count == 10
    assert pool.stats()["reserved-pages"] == 0
    assert pool.release_capacity(cap) is True
    assert pool.release_capacity(cap) is False
    assert pool.free_page_count() == 5
    assert pool.release_route("request") is True
    assert pool.free_page_count() == 8


def test_resident_route_reports_logical_tensor_bytes():
    """continuation_page_pool_test.clj:50-59."""
    pool = fixture_pool()
    assert pool.route_bytes("missing") is None
    assert pool.chunk_payload_bytes(4) == 64
    assert pool.chunk_payload_bytes(0) == 0
    pool.allocate_route("request", 3)
    assert pool.route_bytes("request") == 48


def test_unused_capacity_is_recoverable_and_unavailable_to_other_routes():
    """continuation_page_pool_test.clj:61-71."""
    pool = fixture_pool()
    cap = pool.reserve_capacity("reserved", 32)
    assert pool.free_page_count() == 0
    with pytest.raises(PagePoolError, match="insufficient"):
        pool.allocate_route("other", 1)
    assert pool.release_capacity(cap)
    assert pool.free_page_count() == 8


def test_projected_capacity_includes_shared_tail_copy_on_write():
    """continuation_page_pool_test.clj:73-89."""
    pool = fixture_pool()
    pool.allocate_route("root", 3)
    pool.fork_route("root", "fork")
    cap = pool.reserve_capacity("fork", 4)
    assert pool.stats()["reserved-pages"] == 1
    res = pool.reserve_append("fork")
    assert res.replaced_page == 0
    pool.commit_append("fork", res)
    assert pool.stats()["reserved-pages"] == 0
    assert pool.release_capacity(cap)


def test_routes_share_full_pages_and_copy_on_write_the_tail():
    """continuation_page_pool_test.clj:91-125: COW of the shared partial tail."""
    dev = CopyRecorder()
    pool = fixture_pool(dev)
    root = pool.allocate_route("root", 6)
    fork = pool.fork_route("root", "fork")
    assert list(root.pages) == [0, 1] == list(fork.pages)
    assert pool.free_page_count() == 6
    res = pool.reserve_append("fork")
    assert res.replaced_page == 1
    assert res.physical_page == 2
    assert res.page_offset == 2
    copies = dev.range_copies()
    assert len(copies) == 4
    assert all(c[4] == 8 for c in copies)
    assert dev.pages == [(1, 2)]
    committed = pool.commit_append("fork", res)
    assert list(committed.pages) == [0, 2]
    assert committed.token_count == 7
    assert list(pool.route("root").pages) == [0, 1]
    assert pool.release_route("fork")
    assert pool.free_page_count() == 6
    assert pool.release_route("root")
    assert pool.free_page_count() == 8


def test_aborted_append_restores_the_shared_route():
    """continuation_page_pool_test.clj:127-141."""
    pool = fixture_pool()
    pool.allocate_route("root", 3)
    pool.fork_route("root", "fork")
    res = pool.reserve_append("fork")
    restored = pool.abort_append("fork", res)
    assert list(restored.pages) == [0]
    assert restored.token_count == 3
    assert pool.refcounts[0] == 2
    assert pool.free_page_count() == 7


def test_append_ranges_reserve_consecutive_slots_and_publish_once():
    """continuation_page_pool_test.clj:143-161."""
    pool = fixture_pool()
    pool.allocate_route("request", 3)
    res = pool.reserve_append_range("request", 6)
    lease = pool.acquire_prospective_lease([{"continuation_id": "request", "reservation": res}])
    assert [(s.physical_page, s.page_offset) for s in res.slots] == [(0, 3), (1, 0), (1, 1), (1, 2), (1, 3), (2, 0)]
    assert list(lease.routes[0].pages) == [0, 1, 2]
    assert lease.routes[0].token_count == 9
    assert pool.route("request").token_count == 3, "the prospective range stays invisible before publication"
    assert pool.commit_append("request", res).token_count == 9
    assert pool.release_lease(lease)


def test_aborted_append_range_restores_copy_on_write_tail_and_all_pages():
    """continuation_page_pool_test.clj:163-183."""
    dev = CopyRecorder()
    pool = fixture_pool(dev)
    pool.allocate_route("root", 3)
    pool.fork_route("root", "fork")
    res = pool.reserve_append_range("fork", 6)
    assert list(pool.route("fork").pages) == [1, 2, 3]
    assert len(dev.range_copies()) == 4
    assert list(pool.abort_append("fork", res).pages) == [0]
    assert pool.route("fork").token_count == 3
    assert pool.refcounts[0] == 2
    assert pool.free_page_count() == 7


def test_dense_routes_compose_unrelated_continuations_into_a_batch():
    """continuation_page_pool_test.clj:525-537."""
    pool = fixture_pool(free=[6, 7], refcounts={0: 1, 1: 1, 2: 1, 3: 1, 4: 1, 5: 1},
                        routes={"a": {"pages": [4, 2], "token_count": 6},
                                "b": {"pages": [5, 0, 3, 1], "token_count": 13, "start_position": 8}})
    v = pool.dense_route_values(["a", "b"])
    assert list(v["page-table"]) == [4, 2, -1, -1, 5, 0, 3, 1]
    assert list(v["lengths"]) == [6, 13]
    assert list(v["start-positions"]) == [0, 8]
    assert v["pages-per-sequence"] == 4


def test_leases_pin_an_immutable_route_snapshot_through_copy_on_write():
    """continuation_page_pool_test.clj:564-587."""
    pool = fixture_pool()
    pool.allocate_route("request", 3)
    lease = pool.acquire_lease(["request"])
    res = pool.reserve_append("request")
    assert res.replaced_page == 0, "the lease makes the live partial tail copy-on-write"
    pool.commit_append("request", res)
    assert list(pool.route("request").pages) == [1]
    assert list(lease.routes[0].pages) == [0], "the scheduled page-table snapshot remains immutable"
    assert pool.release_route("request")
    assert pool.free_page_count() == 7, "the old page remains pinned after logical eviction"
    assert list(pool.leased_dense_route_values(lease)["page-table"]) == [0]
    assert pool.release_lease(lease)
    assert pool.free_page_count() == 8


def test_prospective_leases_see_a_whole_batch_only_after_exact_reservation():
    """continuation_page_pool_test.clj:589-615."""
    pool = fixture_pool()
    pool.allocate_route("a", 3)
    pool.allocate_route("b", 4)
    entries = [{"continuation_id": c, "reservation": pool.reserve_append(c)} for c in ("a", "b")]
    lease = pool.acquire_prospective_lease(entries)
    v = pool.leased_dense_route_values(lease, pages_per_sequence=2)
    assert list(v["lengths"]) == [4, 5]
    assert list(v["page-table"]) == [0, -1, 1, 2]
    assert [pool.route(c).token_count for c in ("a", "b")] == [3, 4], "the live routes stay uncommitted"
    with pytest.raises(PagePoolError, match="stale"):
        pool.acquire_prospective_lease([dict(entries[0], reservation={})])
    assert [r.token_count for r in pool.commit_appends(entries)] == [4, 5]
    assert pool.release_lease(lease)


def test_batched_abort_validates_every_reservation_before_changing_routes():
    """continuation_page_pool_test.clj:617-637."""
    pool = fixture_pool()
    pool.allocate_route("a", 0)
    pool.allocate_route("b", 0)
    entries = [{"continuation_id": c, "reservation": pool.reserve_append(c)} for c in ("a", "b")]
    bad = [entries[0], dict(entries[1], reservation={})]
    with pytest.raises(PagePoolError, match="stale"):
        pool.abort_appends(bad)
    assert all(pool.route(c).pending is not None for c in ("a", "b"))
    assert [r.token_count for r in pool.abort_appends(entries)] == [0, 0]
    assert pool.free_page_count() == 8


def test_fork_at_a_shorter_boundary_shares_only_the_covering_pages():
    """continuation_page_pool_test.clj:639-658."""
    pool = fixture_pool()
    pool.allocate_route("root", 7)
    root_pages = list(pool.route("root").pages)
    aligned = pool.fork_route("root", "aligned", 4)
    partial = pool.fork_route("root", "partial", 5)
    assert len(root_pages) == 2
    assert list(aligned.pages) == [root_pages[0]]
    assert aligned.token_count == 4
    assert list(partial.pages) == root_pages
    assert partial.token_count == 5
    assert pool.refcounts[root_pages[0]] == 3
    assert pool.refcounts[root_pages[1]] == 2
    assert pool.route("root").token_count == 7, "the source route is unchanged"
    with pytest.raises(PagePoolError, match="exceeds"):
        pool.fork_route("root", "too-long", 8)


def test_lowest_free_page_is_taken_first_and_cow_replacement_first():
    """page_pool.clj:513-524 (sorted free set): allocation order is ascending."""
    pool = fixture_pool(free=[5, 1, 6, 2])
    r = pool.allocate_route("x", 9)
    assert list(r.pages) == [1, 2, 5]


def test_dense_values_pads_with_minus_one():
    """page_pool.clj:1423-1446."""
    routes = [Route("a", (3,), 2), Route("b", (), 0)]
    v = dense_values(routes, pages_per_sequence=3)
    assert list(v["page-table"]) == [3, -1, -1, -1, -1, -1]
    assert list(v["lengths"]) == [2, 0]
