"""Cost-aware admission and eviction of resident continuation routes: the host
mirror of ``src/pretrained/continuation/residency.clj``.

Planning reads an immutable ``PagePool.residency_snapshot()`` and simulates
shared-page reference counts, so a plan accounts for evictions that free no
page until every route sharing it is gone.  Applying a plan (``admit_route``,
``reserve_admission``) releases the victims and then allocates or reserves on
the same pool, mirroring the reference's ``locking pool`` sections (the host
control plane here is single-threaded per pool).
"""
from __future__ import annotations

import math
import numbers

from .page_pool import PagePool, PagePoolError, capacity_page_requirement, page_count

_COST_FIELDS = ("reuse-probability", "recompute-ms", "reload-ms", "sharing-bonus", "slo-bonus")


def _policy(route) -> dict:
    p = getattr(route, "policy", None)
    if p is None:
        return {}
    return dict(p) if not isinstance(p, dict) else p


def _cid(route):
    return route.continuation_id


def cache_value(route) -> float:
    """Retained value of one resident route in utility milliseconds
    (residency.clj:9-39): p_reuse * max(0, recompute - reload) + sharing + slo.
    Missing policy fields are zero; negative or non-numeric costs and a reuse
    probability outside [0, 1] are rejected."""
    pol = _policy(route)
    values = {f: (pol.get(f) if pol.get(f) is not None else 0.0) for f in _COST_FIELDS}
    for field in _COST_FIELDS:
        v = values[field]
        if isinstance(v, bool) or not isinstance(v, numbers.Real) or float(v) < 0.0 or math.isnan(float(v)):
            raise PagePoolError("Route policy costs must be non-negative numbers",
                                continuation_id=_cid(route), field=field, value=v)
    prob = float(values["reuse-probability"])
    if not 0.0 <= prob <= 1.0:
        raise PagePoolError("Route reuse probability must be in [0,1]",
                            continuation_id=_cid(route), reuse_probability=prob)
    return (prob * max(0.0, float(values["recompute-ms"]) - float(values["reload-ms"]))
            + float(values["sharing-bonus"]) + float(values["slo-bonus"]))


def _value_density(route) -> float:
    """residency.clj:41-44: value per resident page."""
    return cache_value(route) / float(max(1, len(route.pages)))


def _leased_continuations(snapshot) -> set:
    """residency.clj:46-48."""
    out = set()
    for lease in snapshot["leases"].values():
        out.update(lease.get("continuation_ids", ()))
    return out


def _eligible(leased, protected, route) -> bool:
    """residency.clj:50-57: durable, unpinned, not mid-append, unleased, unprotected."""
    pol = _policy(route)
    return (pol.get("durable?") is True and not pol.get("pinned?")
            and route.pending is None and _cid(route) not in leased and _cid(route) not in protected)


def _release_simulated(sim, route):
    """residency.clj:59-69: drop one reference per page; a last reference frees it."""
    refcounts, free = sim
    for p in route.pages:
        refs = refcounts.get(p, 0)
        if refs == 1:
            del refcounts[p]
            free.add(p)
        else:
            refcounts[p] = refs - 1
    return sim


def _sort_key(route):
    """residency.clj:76-78: value density, then oldest last-access, then identity."""
    pol = _policy(route)
    last = pol.get("last-access")
    return (_value_density(route), int(last) if last is not None else 0, str(_cid(route)))


def _plan_pages(snapshot, required: int, protected) -> dict:
    """residency.clj:71-104."""
    available = len(snapshot["free-pages"])
    leased = _leased_continuations(snapshot)
    candidates = sorted((r for r in snapshot["routes"].values() if _eligible(leased, protected, r)),
                        key=_sort_key)
    sim = (dict(snapshot["refcounts"]), set(snapshot["free-pages"]))
    evictions = []
    remaining = list(candidates)
    while True:
        free = len(sim[1])
        if free >= required:
            return {"admissible?": True, "required-pages": required, "available-pages": available,
                    "evictions": evictions, "free-pages-after-eviction": free}
        if not remaining:
            return {"admissible?": False, "required-pages": required, "available-pages": available,
                    "evictions": [], "shortfall-pages": required - free}
        victim = remaining.pop(0)
        _release_simulated(sim, victim)
        evictions.append(_cid(victim))


def plan_admission(snapshot: dict, token_count, protected_continuation_ids=()) -> dict:
    """Evictions needed to admit a new route of ``token_count`` tokens
    (residency.clj:106-121).  Lowest value density goes first, then the oldest
    last-access, then the continuation identity."""
    if isinstance(token_count, bool) or not isinstance(token_count, numbers.Integral) or token_count < 0:
        raise PagePoolError("Admission token count must be a non-negative integer", token_count=token_count)
    return _plan_pages(snapshot, page_count(int(token_count), snapshot["page-size"]),
                       set(protected_continuation_ids))


def plan_capacity_admission(snapshot: dict, cid, token_capacity, protected_continuation_ids=()) -> dict:
    """Evictions for a continuation's incremental projected capacity
    (residency.clj:123-140): resident pages are credited, a shared partial tail
    adds its copy-on-write page, and the target is never a victim."""
    return _plan_pages(snapshot, capacity_page_requirement(snapshot, cid, token_capacity),
                       set(protected_continuation_ids) | {cid})


def evictable_page_count(snapshot: dict, protected_continuation_ids=()) -> int:
    """Unique physical pages recoverable by evicting every eligible route
    (residency.clj:142-159), shared reference counts simulated."""
    leased = _leased_continuations(snapshot)
    protected = set(protected_continuation_ids)
    sim = (dict(snapshot["refcounts"]), set(snapshot["free-pages"]))
    for r in snapshot["routes"].values():
        if _eligible(leased, protected, r):
            _release_simulated(sim, r)
    return len(sim[1]) - len(snapshot["free-pages"])


def reserve_admission(pool: PagePool, cid, token_capacity, protected_continuation_ids=()) -> dict:
    """Evict eligible routes, then reserve projected capacity (residency.clj:161-181).
    Returns the plan with ``capacity-reservation`` when admissible, otherwise the
    unchanged non-admissible plan (the pool is not modified)."""
    plan = plan_capacity_admission(pool.residency_snapshot(), cid, token_capacity, protected_continuation_ids)
    if not plan["admissible?"]:
        return plan
    for victim in plan["evictions"]:
        pool.release_route(victim)
    plan = dict(plan)
    plan["capacity-reservation"] = pool.reserve_capacity(cid, token_capacity)
    return plan


def admit_route(pool: PagePool, cid, token_count, start_position: int = 0, policy=None,
                protected_continuation_ids=()) -> dict:
    """Evict durable routes as planned and allocate a new resident route
    (residency.clj:183-202).  Returns the plan with ``resident-route``, or the
    unchanged non-admissible plan."""
    plan = plan_admission(pool.residency_snapshot(), token_count, protected_continuation_ids)
    if not plan["admissible?"]:
        return plan
    for victim in plan["evictions"]:
        pool.release_route(victim)
    plan = dict(plan)
    plan["resident-route"] = pool.allocate_route(cid, int(token_count), start_position=start_position,
                                                 policy=policy)
    return plan
