"""Worker-local paged attention state: the bookkeeping half of
``src/pretrained/continuation/page_pool.clj`` (physical pages, reference counts,
routes, leases, capacity reservations, copy-on-write appends, dense page tables).

The reference keeps this control plane in Clojure; this is the host-side mirror
the harness and tests drive.  Semantics follow the reference function by
function (citations per method); the device half (slab allocation and the
copy-on-write page copy) is delegated to ``device`` -- a ``rstr.hip.Pool`` or a
recording fake -- exactly where the reference calls Raster.

Every mutation validates first and changes state only on success, matching the
reference's compute-new-state-then-``reset!`` pattern.
"""
from __future__ import annotations

import itertools
from dataclasses import dataclass, replace

import numpy as np
from sortedcontainers import SortedSet


class PagePoolError(ValueError):
    """ex-info equivalent: a message plus a data map."""

    def __init__(self, msg: str, **data):
        super().__init__(msg)
        self.data = data


def page_count(token_count: int, page_size: int) -> int:
    """page_pool.clj:74-78."""
    return 0 if token_count == 0 else (token_count - 1) // page_size + 1


@dataclass(frozen=True)
class Route:
    continuation_id: object
    pages: tuple
    token_count: int
    start_position: int = 0
    pending: object = None
    policy: tuple = ()


@dataclass(frozen=True)
class Slot:
    logical_page: int
    physical_page: int
    page_offset: int


@dataclass(frozen=True)
class Reservation:
    """The :pending map of reserve-append-range! (page_pool.clj:947-958)."""
    expected_token_count: int
    token_count: int
    logical_page: int
    physical_page: int
    page_offset: int
    slots: tuple
    allocated_pages: tuple
    added_pages: tuple
    added_page: bool
    replaced_page: object


@dataclass(frozen=True)
class PageLease:
    pool: object
    id: int
    routes: tuple


@dataclass(frozen=True)
class CapacityReservation:
    pool: object
    id: int
    continuation_id: object


_ids = itertools.count(1)


class PagePool:
    """DevicePagePool record (page_pool.clj:15): layout, page size, pages, dtype."""

    def __init__(self, page_size: int, physical_pages: int, n_layers: int = 1, n_kv: int = 1,
                 head_dim: int = 1, dtype: str = "half", device=None):
        """open-pool! (page_pool.clj:235-303) minus the Raster allocation."""
        for name, v in (("page-size", page_size), ("physical-pages", physical_pages)):
            if not isinstance(v, (int, np.integer)) or v <= 0:
                raise PagePoolError("Page-pool extent must be a positive integer", field=name, value=v)
        if page_size > 2**31 - 1 or physical_pages > 2**31 - 1:
            raise PagePoolError("Raster page routing uses int32 page coordinates")
        if dtype not in ("half", "float"):
            raise PagePoolError("Page pool currently supports FP16 or FP32 storage", dtype=dtype)
        self.page_size = int(page_size)
        self.physical_pages = int(physical_pages)
        self.n_layers, self.n_kv, self.head_dim, self.dtype = n_layers, n_kv, head_dim, dtype
        self.device = device
        self.free = SortedSet(range(self.physical_pages))
        self.refcounts: dict[int, int] = {}
        self.routes: dict = {}
        self.leases: dict[int, dict] = {}
        self.capacity_reservations: dict[int, dict] = {}

    # ---- queries ----------------------------------------------------------
    def route(self, cid):
        """page_pool.clj:310-313."""
        return self.routes.get(cid)

    def elements_per_token(self) -> int:
        return 2 * self.n_layers * self.n_kv * self.head_dim

    def route_bytes(self, cid):
        """page_pool.clj:315-331 (shared pages counted per logical route)."""
        r = self.routes.get(cid)
        if r is None:
            return None
        return r.token_count * self.elements_per_token() * (2 if self.dtype == "half" else 4)

    def chunk_payload_bytes(self, token_count: int) -> int:
        """page_pool.clj:333-350."""
        if not isinstance(token_count, (int, np.integer)) or token_count < 0:
            raise PagePoolError("Chunk token count must be a non-negative integer")
        return token_count * self.elements_per_token() * (2 if self.dtype == "half" else 4)

    def free_page_count(self) -> int:
        """page_pool.clj:418-421."""
        return len(self.free)

    def stats(self) -> dict:
        """page_pool.clj:423-435."""
        return {"physical-pages": self.physical_pages, "free-pages": len(self.free),
                "resident-pages": len(self.refcounts),
                "shared-pages": sum(1 for v in self.refcounts.values() if v > 1),
                "resident-routes": len(self.routes), "active-leases": len(self.leases),
                "capacity-reservations": len(self.capacity_reservations),
                "reserved-pages": sum(len(e["pages"]) for e in self.capacity_reservations.values())}

    def residency_snapshot(self) -> dict:
        """page_pool.clj:352-367: immutable data for admission/eviction planners."""
        return {"physical-pages": self.physical_pages, "page-size": self.page_size,
                "free-pages": frozenset(self.free), "refcounts": dict(self.refcounts),
                "routes": dict(self.routes),
                "leases": {k: dict(v) for k, v in self.leases.items()},
                "capacity-reservations": {k: dict(v) for k, v in self.capacity_reservations.items()}}

    def capacity_page_requirement(self, snapshot: dict, cid, token_capacity: int) -> int:
        return capacity_page_requirement(snapshot, cid, token_capacity)

    def touch_route(self, cid, observations: dict):
        """page_pool.clj:396-416."""
        if not isinstance(observations, dict):
            raise PagePoolError("Route policy observations must be a map")
        r = self.routes.get(cid)
        if r is None:
            raise PagePoolError("Cannot touch a nonresident continuation", continuation_id=cid)
        pol = dict(r.policy)
        pol.update(observations)
        nr = replace(r, policy=tuple(sorted(pol.items(), key=lambda kv: repr(kv[0]))))
        self.routes[cid] = nr
        return nr

    # ---- page ownership -----------------------------------------------------
    def _take_free(self, n: int, cid):
        """page_pool.clj:513-524: the lowest free pages."""
        if n > len(self.free):
            raise PagePoolError("Device page pool has insufficient free capacity",
                                continuation_id=cid, required=n, available=len(self.free))
        return list(itertools.islice(self.free, n))

    def _commit_take(self, pages):
        for p in pages:
            self.free.remove(p)
            self.refcounts[p] = 1

    def _route_reservation(self, cid):
        """page_pool.clj:554-565."""
        matches = [rid for rid, e in self.capacity_reservations.items() if e["continuation_id"] == cid]
        if len(matches) > 1:
            raise PagePoolError("Continuation has multiple capacity reservations", continuation_id=cid)
        return CapacityReservation(self, matches[0], cid) if matches else None

    def _reservation_entry(self, res, cid):
        """page_pool.clj:526-536."""
        if not isinstance(res, CapacityReservation) or res.continuation_id != cid:
            raise PagePoolError("Capacity reservation belongs to another continuation",
                                continuation_id=cid)
        e = self.capacity_reservations.get(res.id)
        if e is None:
            raise PagePoolError("Capacity reservation is stale or released", continuation_id=cid)
        return e

    def _claim_reserved(self, res, cid, n: int):
        """page_pool.clj:538-552 (validation half)."""
        e = self._reservation_entry(res, cid)
        if n > len(e["pages"]):
            raise PagePoolError("Capacity reservation has insufficient remaining pages",
                                continuation_id=cid, required=n, available=len(e["pages"]))
        return list(e["pages"][:n])

    def _commit_claim(self, res, pages):
        e = self.capacity_reservations[res.id]
        e["pages"] = e["pages"][len(pages):]
        for p in pages:
            self.refcounts[p] = 1

    def _release_page(self, page: int):
        """page_pool.clj:726-736."""
        refs = self.refcounts.get(page, 0)
        if refs <= 0:
            raise PagePoolError("Resident page reference count is corrupt", page=page, refcount=refs)
        if refs == 1:
            del self.refcounts[page]
            self.free.add(page)
        else:
            self.refcounts[page] = refs - 1

    # ---- capacity -----------------------------------------------------------
    def reserve_capacity(self, cid, token_capacity: int) -> CapacityReservation:
        """page_pool.clj:567-611."""
        if cid is None or not isinstance(token_capacity, (int, np.integer)) or token_capacity < 0:
            raise PagePoolError("Capacity reservation identity and extent are invalid",
                                continuation_id=cid, token_capacity=token_capacity)
        r = self.routes.get(cid)
        if r is not None and r.pending is not None:
            raise PagePoolError("Cannot reserve capacity during a pending append", continuation_id=cid)
        if self._route_reservation(cid) is not None:
            raise PagePoolError("Continuation already has a capacity reservation", continuation_id=cid)
        required = capacity_page_requirement(self._snapshot_light(), cid, int(token_capacity))
        if required > len(self.free):
            raise PagePoolError("Device page pool cannot reserve projected capacity",
                                continuation_id=cid, token_capacity=token_capacity,
                                required_pages=required, available_pages=len(self.free))
        pages = list(itertools.islice(self.free, required))
        for p in pages:
            self.free.remove(p)
        rid = next(_ids)
        self.capacity_reservations[rid] = {"continuation_id": cid, "token_capacity": int(token_capacity),
                                           "pages": pages}
        return CapacityReservation(self, rid, cid)

    def _snapshot_light(self):
        return {"page-size": self.page_size, "routes": self.routes, "refcounts": self.refcounts}

    def release_capacity(self, res: CapacityReservation) -> bool:
        """page_pool.clj:613-633."""
        if not isinstance(res, CapacityReservation) or res.pool is not self:
            raise PagePoolError("Capacity reservation belongs to a different pool")
        e = self.capacity_reservations.pop(res.id, None)
        if e is None:
            return False
        for p in e["pages"]:
            self.free.add(p)
        return True

    # ---- routes -------------------------------------------------------------
    def allocate_route(self, cid, token_count: int, start_position: int = 0, policy=None,
                       capacity_reservation: CapacityReservation | None = None) -> Route:
        """page_pool.clj:635-677."""
        policy = {} if policy is None else policy
        if cid is None or token_count < 0 or start_position < 0:
            raise PagePoolError("Resident route identity and extents are invalid", continuation_id=cid)
        if not isinstance(policy, dict):
            raise PagePoolError("Resident route policy must be a map", continuation_id=cid)
        if cid in self.routes:
            raise PagePoolError("Continuation already has a resident route", continuation_id=cid)
        required = page_count(int(token_count), self.page_size)
        if capacity_reservation is not None and capacity_reservation.pool is not self:
            raise PagePoolError("Capacity reservation belongs to a different pool", continuation_id=cid)
        if capacity_reservation is not None:
            pages = self._claim_reserved(capacity_reservation, cid, required)
            self._commit_claim(capacity_reservation, pages)
        else:
            pages = self._take_free(required, cid)
            self._commit_take(pages)
        r = Route(cid, tuple(pages), int(token_count), int(start_position),
                  policy=tuple(sorted(policy.items(), key=lambda kv: repr(kv[0]))))
        self.routes[cid] = r
        return r

    def fork_route(self, source_id, target_id, token_count: int | None = None) -> Route:
        """page_pool.clj:679-724: share the covering pages of the first token_count tokens."""
        src = self.routes.get(source_id)
        if target_id is None:
            raise PagePoolError("Target continuation requires an identity")
        if src is None:
            raise PagePoolError("Source continuation is not resident", continuation_id=source_id)
        if target_id in self.routes:
            raise PagePoolError("Target continuation already has a resident route", continuation_id=target_id)
        if src.pending is not None:
            raise PagePoolError("Cannot fork a continuation with an uncommitted append",
                                continuation_id=source_id)
        n = src.token_count if token_count is None else int(token_count)
        if n < 0 or n > src.token_count:
            raise PagePoolError("Fork token count exceeds the source route", continuation_id=source_id,
                                token_count=n, source_token_count=src.token_count)
        pages = src.pages[:page_count(n, self.page_size)]
        for p in pages:
            self.refcounts[p] = self.refcounts.get(p, 0) + 1
        t = replace(src, continuation_id=target_id, pages=tuple(pages), token_count=n)
        self.routes[target_id] = t
        return t

    def release_route(self, cid) -> bool:
        """page_pool.clj:738-754."""
        r = self.routes.get(cid)
        if r is None:
            return False
        if r.pending is not None:
            raise PagePoolError("Cannot release a route with an uncommitted append", continuation_id=cid)
        del self.routes[cid]
        for p in r.pages:
            self._release_page(p)
        return True

    # ---- leases -------------------------------------------------------------
    def acquire_lease(self, cids) -> PageLease:
        """page_pool.clj:756-788: pin route snapshots, one reference per occurrence."""
        cids = list(cids)
        if not cids:
            raise PagePoolError("A page lease requires at least one continuation")
        routes = []
        for c in cids:
            r = self.routes.get(c)
            if r is None:
                raise PagePoolError("Cannot lease a nonresident continuation", continuation_id=c)
            routes.append(r)
        for r in routes:
            if r.pending is not None:
                raise PagePoolError("Cannot lease a route with an uncommitted append",
                                    continuation_id=r.continuation_id)
        return self._pin(routes, cids, False)

    def _pin(self, routes, cids, prospective):
        lid = next(_ids)
        pages = [p for r in routes for p in r.pages]
        for p in pages:
            self.refcounts[p] = self.refcounts.get(p, 0) + 1
        self.leases[lid] = {"pages": pages, "continuation_ids": cids, "prospective": prospective}
        return PageLease(self, lid, tuple(routes))

    def acquire_prospective_lease(self, entries) -> PageLease:
        """page_pool.clj:790-839: pin the post-append snapshots of exact pending reservations."""
        entries = list(entries)
        cids = [e["continuation_id"] for e in entries]
        if not entries:
            raise PagePoolError("A prospective page lease requires append reservations")
        if len(cids) != len(set(cids)):
            raise PagePoolError("Prospective lease continuation identities must be unique")
        routes = []
        for e in entries:
            r = self.routes.get(e["continuation_id"])
            if r is None:
                raise PagePoolError("Cannot lease a nonresident continuation",
                                    continuation_id=e["continuation_id"])
            res = e.get("reservation")
            if res is None or res != r.pending:
                raise PagePoolError("Prospective lease reservation is stale",
                                    continuation_id=e["continuation_id"])
            routes.append(replace(r, pending=None, token_count=r.token_count + res.token_count))
        return self._pin(routes, cids, True)

    def release_lease(self, lease: PageLease) -> bool:
        """page_pool.clj:841-857."""
        if not isinstance(lease, PageLease) or lease.pool is not self:
            raise PagePoolError("Page lease belongs to a different pool")
        e = self.leases.pop(lease.id, None)
        if e is None:
            return False
        for p in e["pages"]:
            self._release_page(p)
        return True

    # ---- appends ------------------------------------------------------------
    def reserve_append_range(self, cid, token_count: int) -> Reservation:
        """page_pool.clj:902-973: consecutive slots; a shared partial tail is copied first."""
        if not isinstance(token_count, (int, np.integer)) or token_count <= 0:
            raise PagePoolError("Append range token count must be a positive integer", continuation_id=cid)
        r = self.routes.get(cid)
        if r is None:
            raise PagePoolError("Continuation is not resident", continuation_id=cid)
        if r.pending is not None:
            raise PagePoolError("Continuation already has a pending append", continuation_id=cid)
        ps = self.page_size
        expected = r.token_count
        nxt = expected + int(token_count)
        logical_page = expected // ps
        page_offset = expected % ps
        existing = r.pages[logical_page] if logical_page < len(r.pages) else None
        shared = existing is not None and self.refcounts.get(existing, 0) > 1
        target_pages = page_count(nxt, ps)
        added_count = target_pages - len(r.pages)
        allocation = added_count + (1 if shared else 0)
        cap = self._route_reservation(cid)
        if allocation > 0:
            allocated = (self._claim_reserved(cap, cid, allocation) if cap is not None
                         else self._take_free(allocation, cid))
        else:
            allocated = []
        replacement = allocated[0] if shared else None
        added = allocated[1:] if shared else list(allocated)
        if replacement is not None and self.device is not None:
            self.device.copy_page(existing, replacement)       # copy-page! before mutation
        if allocation > 0:
            if cap is not None:
                self._commit_claim(cap, allocated)
            else:
                self._commit_take(allocated)
        base = list(r.pages)
        if replacement is not None:
            base[logical_page] = replacement
        pages = base + list(added)
        slots = tuple(Slot(pos // ps, pages[pos // ps], pos % ps) for pos in range(expected, nxt))
        pending = Reservation(expected, int(token_count), logical_page, slots[0].physical_page,
                              page_offset, slots, tuple(allocated), tuple(added), added_count > 0,
                              existing if replacement is not None else None)
        if replacement is not None:
            self._release_page(existing)
        self.routes[cid] = replace(r, pages=tuple(pages), pending=pending)
        return pending

    def reserve_append(self, cid) -> Reservation:
        """page_pool.clj:975-980."""
        return self.reserve_append_range(cid, 1)

    def _validate_entries(self, entries):
        """page_pool.clj:982-1001."""
        entries = list(entries)
        cids = [e["continuation_id"] for e in entries]
        if not entries:
            raise PagePoolError("Append completion requires at least one reservation")
        if len(cids) != len(set(cids)):
            raise PagePoolError("Append completion continuation identities must be unique")
        for e in entries:
            r = self.routes.get(e["continuation_id"])
            if r is None:
                raise PagePoolError("Append reservation continuation is not resident",
                                    continuation_id=e["continuation_id"])
            if e.get("reservation") is None or e["reservation"] != r.pending:
                raise PagePoolError("Append reservation is stale or belongs to another route",
                                    continuation_id=e["continuation_id"])
        return entries

    def commit_appends(self, entries):
        """page_pool.clj:1003-1023: publish the new logical lengths atomically."""
        entries = self._validate_entries(entries)
        out = []
        for e in entries:
            r = self.routes[e["continuation_id"]]
            nr = replace(r, pending=None, token_count=r.token_count + e["reservation"].token_count)
            self.routes[e["continuation_id"]] = nr
            out.append(nr)
        return out

    def commit_append(self, cid, reservation):
        return self.commit_appends([{"continuation_id": cid, "reservation": reservation}])[0]

    def abort_appends(self, entries):
        """page_pool.clj:1031-1061: restore pages, replaced tail and references."""
        entries = self._validate_entries(entries)
        out = []
        for e in entries:
            r = self.routes[e["continuation_id"]]
            res = r.pending
            pages = list(r.pages)
            if res.added_pages:
                pages = pages[:len(pages) - len(res.added_pages)]
            if res.replaced_page is not None:
                pages[res.logical_page] = res.replaced_page
            for p in res.allocated_pages:
                self._release_page(p)
            if res.replaced_page is not None:
                self.refcounts[res.replaced_page] = self.refcounts.get(res.replaced_page, 0) + 1
            nr = replace(r, pending=None, pages=tuple(pages))
            self.routes[e["continuation_id"]] = nr
            out.append(nr)
        return out

    def abort_append(self, cid, reservation):
        return self.abort_appends([{"continuation_id": cid, "reservation": reservation}])[0]

    # ---- dense route values ------------------------------------------------------
    def dense_route_values(self, cids, pages_per_sequence: int | None = None):
        """page_pool.clj:1448-1461 (point-in-time view)."""
        routes = []
        for c in cids:
            r = self.routes.get(c)
            if r is None:
                raise PagePoolError("Batch continuation is not resident", continuation_id=c)
            routes.append(r)
        return dense_values(routes, pages_per_sequence)

    def leased_dense_route_values(self, lease: PageLease, pages_per_sequence: int | None = None):
        """page_pool.clj:1463-1474."""
        if not isinstance(lease, PageLease) or lease.pool is not self:
            raise PagePoolError("Page lease belongs to a different pool")
        if lease.id not in self.leases:
            raise PagePoolError("Page lease has already been released", lease_id=lease.id)
        return dense_values(lease.routes, pages_per_sequence)


def capacity_page_requirement(snapshot: dict, cid, token_capacity: int) -> int:
    """page_pool.clj:369-394: existing pages are credited; a shared partial tail
    that will grow needs one extra copy-on-write page."""
    if cid is None or not isinstance(token_capacity, (int, np.integer)) or token_capacity < 0:
        raise PagePoolError("Capacity requirement arguments are invalid", continuation_id=cid)
    r = snapshot["routes"].get(cid)
    ps = snapshot["page-size"]
    target = page_count(int(token_capacity), ps)
    current = len(r.pages) if r is not None else 0
    shared_partial = (r is not None and r.token_count < token_capacity and r.token_count % ps > 0
                      and snapshot["refcounts"].get(r.pages[-1], 0) > 1)
    return max(0, target - current) + (1 if shared_partial else 0)


def dense_values(routes, pages_per_sequence=None) -> dict:
    """page_pool.clj:1423-1446: fixed-width page table (-1 padded), lengths, starts."""
    routes = list(routes)
    cap = pages_per_sequence if pages_per_sequence is not None else max(
        1, max((len(r.pages) for r in routes), default=0))
    if cap > 2**31 - 1 or any(r.token_count > 2**31 - 1 or r.start_position > 2**31 - 1 for r in routes):
        raise PagePoolError("Dense route values exceed Raster's int32 coordinates")
    if any(len(r.pages) > cap for r in routes):
        raise PagePoolError("Resident route exceeds dense page-table capacity",
                            pages_per_sequence=cap, route_pages=[len(r.pages) for r in routes])
    pt = np.full((len(routes), cap), -1, np.int32)
    for i, r in enumerate(routes):
        pt[i, :len(r.pages)] = r.pages
    return {"page-table": pt.ravel(), "lengths": np.array([r.token_count for r in routes], np.int32),
            "start-positions": np.array([r.start_position for r in routes], np.int32),
            "pages-per-sequence": cap}
