"""Batched append reservations (``src/pretrained/continuation/paged_append.clj``).

One reservation batch covers every layer's append of a step; it is committed
only after the whole step ran, or aborted on failure.  The device write itself
is the routed append inside the decode step (``rstr_step_lanes``) or the
isolated ``rstr_append_run``.
"""
from __future__ import annotations

import itertools

import numpy as np

from .page_pool import PagePool, PagePoolError

_ids = itertools.count(1)


def physical_slot(pool: PagePool, reservation_or_slot) -> int:
    """paged_append.clj:44-57: page * page_size + offset, checked against int32."""
    slot = reservation_or_slot.physical_page * pool.page_size + reservation_or_slot.page_offset
    if slot > 2**31 - 1:
        raise PagePoolError("Paged append slot exceeds Raster's int32 descriptor", slot=slot)
    return slot


class AppendBatch:
    """AppendBatch record (paged_append.clj:18)."""

    def __init__(self, pool, entries, slots):
        self.pool, self.id, self.entries = pool, next(_ids), entries
        self.slots = np.asarray(slots, np.int32)
        self.state = "reserved"

    def slot_values(self) -> np.ndarray:
        """paged_append.clj:132-137."""
        return self.slots.copy()

    def commit(self):
        """commit-batch! (paged_append.clj:139-150)."""
        if self.state != "reserved":
            raise PagePoolError("Append batch has already been completed", batch_id=self.id,
                                state=self.state)
        routes = self.pool.commit_appends(self.entries)
        self.state = "committed"
        return routes

    def abort(self):
        """abort-batch! (paged_append.clj:152-163)."""
        if self.state != "reserved":
            raise PagePoolError("Append batch has already been completed", batch_id=self.id,
                                state=self.state)
        routes = self.pool.abort_appends(self.entries)
        self.state = "aborted"
        return routes


def reserve_batch(pool: PagePool, cids) -> AppendBatch:
    """paged_append.clj:59-100: one slot per continuation; any failure rolls back
    the reservations already taken."""
    if not isinstance(pool, PagePool):
        raise PagePoolError("Paged append requires a DevicePagePool")
    cids = list(cids)
    if not cids:
        raise PagePoolError("Paged append requires at least one continuation")
    if len(cids) != len(set(cids)):
        raise PagePoolError("Paged append continuation identities must be unique", continuation_ids=cids)
    entries = []
    for cid in cids:
        try:
            res = pool.reserve_append(cid)
        except Exception:
            if entries:
                pool.abort_appends(entries)
            raise
        entries.append({"continuation_id": cid, "reservation": res})
    try:
        return AppendBatch(pool, entries, [physical_slot(pool, e["reservation"]) for e in entries])
    except Exception:
        pool.abort_appends(entries)
        raise


def reserve_range(pool: PagePool, cid, token_count: int) -> AppendBatch:
    """paged_append.clj:102-124: consecutive rows for one continuation."""
    if not isinstance(pool, PagePool):
        raise PagePoolError("Paged append requires a DevicePagePool")
    res = pool.reserve_append_range(cid, token_count)
    entries = [{"continuation_id": cid, "reservation": res}]
    try:
        return AppendBatch(pool, entries, [physical_slot(pool, s) for s in res.slots])
    except Exception:
        pool.abort_appends(entries)
        raise
