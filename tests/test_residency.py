"""Known-answer tests of the admission/eviction mirror, one per reference test in
``test/pretrained/continuation_residency_test.clj`` (fixture pool: 4-token
pages, 4 physical pages, one layer with one kv head of width 2, fp16).
"""
import pytest
from sortedcontainers import SortedSet

from rstr import residency
from rstr.page_pool import CapacityReservation, PagePool, PagePoolError, Route


def _route(cid, pages, token_count=0, policy=None, pending=None):
    pol = tuple(sorted((policy or {}).items(), key=lambda kv: repr(kv[0])))
    return Route(cid, tuple(pages), token_count, 0, pending=pending, policy=pol)


def fixture_pool(free, refcounts, routes, leases=None):
    """continuation_residency_test.clj:10-15."""
    pool = PagePool(4, 4, 1, 1, 2, "half")
    pool.free = SortedSet(free)
    pool.refcounts = dict(refcounts)
    pool.routes = {r.continuation_id: r for r in routes}
    pool.leases = dict(leases or {})
    return pool


def snapshot(physical_pages, free, refcounts, routes, leases=None):
    return {"physical-pages": physical_pages, "page-size": 4, "free-pages": frozenset(free),
            "refcounts": dict(refcounts), "routes": {r.continuation_id: r for r in routes},
            "leases": dict(leases or {}), "capacity-reservations": {}}


def test_admission_prefers_low_value_durable_routes():
    """continuation_residency_test.clj:17-42."""
    pool = fixture_pool([], {0: 1, 1: 1, 2: 1, 3: 1}, [
        _route("cold", [0, 1], 8, {"durable?": True, "last-access": 1, "reuse-probability": 0.1,
                                   "recompute-ms": 10.0, "reload-ms": 5.0}),
        _route("hot", [2, 3], 8, {"durable?": True, "last-access": 2, "reuse-probability": 0.9,
                                  "recompute-ms": 20.0, "reload-ms": 2.0})])
    result = residency.admit_route(pool, "incoming", 8, policy={"durable?": False, "last-access": 3})
    assert result["admissible?"]
    assert result["evictions"] == ["cold"]
    assert pool.route("cold") is None
    assert pool.route("incoming").pages == (0, 1)
    assert pool.route("hot").pages == (2, 3)


def test_admission_never_evicts_pinned_dirty_or_leased_routes():
    """continuation_residency_test.clj:44-65."""
    pool = fixture_pool([], {0: 1, 1: 2, 2: 1, 3: 1}, [
        _route("dirty", [0], 4, {"durable?": False}),
        _route("leased", [1], 4, {"durable?": True}),
        _route("pinned", [2, 3], 8, {"durable?": True, "pinned?": True})],
        leases={7: {"pages": [1], "continuation_ids": ["leased"], "prospective": False}})
    before = pool.residency_snapshot()
    result = residency.admit_route(pool, "incoming", 4)
    assert result["admissible?"] is False
    assert result["shortfall-pages"] == 1
    assert pool.residency_snapshot() == before


def test_shared_pages_are_accounted_for_as_a_set_of_evictions():
    """continuation_residency_test.clj:67-81: both low-value sharing routes may
    be removed before a page is free."""
    snap = snapshot(2, [], {0: 2, 1: 1}, [
        _route("fork-a", [0], 0, {"durable?": True, "last-access": 0}),
        _route("fork-b", [0], 0, {"durable?": True, "last-access": 1}),
        _route("other", [1], 0, {"durable?": True, "last-access": 2})])
    plan = residency.plan_admission(snap, 4)
    assert plan["admissible?"]
    assert plan["evictions"] == ["fork-a", "fork-b"]


def test_capacity_admission_uses_incremental_route_growth():
    """continuation_residency_test.clj:83-99."""
    snap = snapshot(4, [2, 3], {0: 1, 1: 1}, [
        _route("running", [0], 3, {"durable?": False}),
        _route("cold", [1], 4, {"durable?": True})])
    plan = residency.plan_capacity_admission(snap, "running", 16)
    assert plan["admissible?"]
    assert plan["required-pages"] == 3
    assert plan["evictions"] == ["cold"]
    assert "running" not in plan["evictions"]


def test_capacity_admission_reserves_after_eviction():
    """continuation_residency_test.clj:101-121."""
    pool = fixture_pool([2, 3], {0: 1, 1: 1}, [
        _route("running", [0], 3, {"durable?": False}),
        _route("cold", [1], 4, {"durable?": True})])
    result = residency.reserve_admission(pool, "running", 16)
    assert result["admissible?"]
    assert result["evictions"] == ["cold"]
    assert isinstance(result["capacity-reservation"], CapacityReservation)
    assert pool.stats()["reserved-pages"] == 3
    assert pool.route("running") is not None
    assert pool.route("cold") is None
    assert pool.release_capacity(result["capacity-reservation"])


def test_evictable_capacity_observes_protection_and_shared_refcounts():
    """continuation_residency_test.clj:123-131."""
    snap = snapshot(1, [], {0: 2}, [
        _route("fork-a", [0], 4, {"durable?": True}),
        _route("fork-b", [0], 4, {"durable?": True})])
    assert residency.evictable_page_count(snap) == 1
    assert residency.evictable_page_count(snap, {"fork-a"}) == 0


# ---- the value formula and its validation (residency.clj:9-39) --------------
def test_cache_value_closed_form_and_defaults():
    r = _route("r", [0, 1], 8, {"reuse-probability": 0.5, "recompute-ms": 30.0, "reload-ms": 10.0,
                                "sharing-bonus": 2.0, "slo-bonus": 1.0})
    assert residency.cache_value(r) == 0.5 * 20.0 + 2.0 + 1.0
    # reload slower than recompute contributes nothing; missing fields are zero
    assert residency.cache_value(_route("s", [0], 4, {"reuse-probability": 1.0, "recompute-ms": 1.0,
                                                       "reload-ms": 5.0})) == 0.0
    assert residency.cache_value(_route("t", [0], 4)) == 0.0


@pytest.mark.parametrize("policy,msg", [
    ({"recompute-ms": -1.0}, "non-negative numbers"),
    ({"slo-bonus": "x"}, "non-negative numbers"),
    ({"reuse-probability": 1.5}, r"\[0,1\]"),
])
def test_cache_value_rejects_invalid_policies(policy, msg):
    with pytest.raises(PagePoolError, match=msg):
        residency.cache_value(_route("r", [0], 4, policy))


def test_eviction_order_is_density_then_last_access_then_identity():
    """Equal value densities fall back to the oldest last-access, then the id."""
    routes = [_route("b", [0], 4, {"durable?": True, "last-access": 5}),
              _route("a", [1], 4, {"durable?": True, "last-access": 5}),
              _route("c", [2], 4, {"durable?": True, "last-access": 1}),
              _route("big", [3], 4, {"durable?": True, "sharing-bonus": 1.0})]
    snap = snapshot(4, [], {0: 1, 1: 1, 2: 1, 3: 1}, routes)
    assert residency.plan_admission(snap, 16)["evictions"] == ["c", "a", "b", "big"]
    assert residency.plan_admission(snap, 4)["evictions"] == ["c"]
    with pytest.raises(PagePoolError, match="non-negative integer"):
        residency.plan_admission(snap, -1)
