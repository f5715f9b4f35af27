"""Durable KV chunk export and restore over the page-pool mirror.

Mirrors the chunk half of ``src/pretrained/continuation/page_pool.clj``
(``transfer-runs`` :80-103, ``record-transfer!`` :105-139, ``half-payload``
:1084-1109, ``restore-chunk-plan`` :1111-1145, ``submit-restore-chunk!`` /
``chunk-transfer-complete?`` / ``complete-restore-chunk!`` / ``restore-chunk!``
:1169-1224, ``export-chunk-plan`` :1226-1245, ``exported-chunk`` :1267-1286,
``submit-export-chunk!`` .. ``export-chunk`` :1288-1374) and the payload order of
``attention_state.clj:103-123`` (``payload-plan``).

The host keeps the reference's validation, leasing, durable chunk map
(``:chunk/version 3``) and transfer telemetry.  The device half differs on
purpose: where the reference submits one ranged copy per (slab, layer, physical
run) -- or, for fragmented page-aligned ranges, stages blocks through a Raster
gather/scatter graph (block_transfer.clj:17-199) -- the pool device here moves
the whole range with one gather/scatter kernel and one DMA copy
(``rstr_chunk_export_submit`` / ``rstr_chunk_restore_submit``), whatever the
run structure.  ``transfer_runs`` and ``direct_entries`` still describe the
reference's ranged copies; they are the plan the device kernel is checked
against and what telemetry counts as commands of the reference path.

Device protocol (``pool.device``): ``export_submit(pages, start, count)`` and
``restore_submit(pages, start, count, payload)`` return a transfer with
``done()`` and ``complete()`` -> ``{"bytes", "device_ms", "direction",
"payload"}`` (``hip.Pool`` implements it over the C ABI).
"""
from __future__ import annotations

import time

import numpy as np

from .page_pool import PagePool, PagePoolError, Route

DEFAULT_ALPHA = 0.2  # telemetry.clj:4-6


# ---- layout -----------------------------------------------------------------
def pool_layout(pool: PagePool) -> dict:
    """The pool's resolved attention-state layout (attention_state.clj:53-92 with
    the default K/V descriptor :9-22), fp16 on the device."""
    ept = pool.n_kv * pool.head_dim
    return {"version": 1, "kind": "kv", "token-axis": "position", "dtype": "half",
            "byte-order": "little-endian",
            "slabs": [{"name": "key", "count": pool.n_layers, "elements-per-token": ept},
                      {"name": "value", "count": pool.n_layers, "elements-per-token": ept}]}


def canonical_dtype(dtype):
    """page_pool.clj:52-57."""
    return {"float16": "half", "f16": "half", "float32": "float", "f32": "float"}.get(dtype, dtype)


def payload_plan(layout: dict, token_count: int) -> list:
    """attention_state.clj:103-123: slab order, then layer order, each a
    contiguous slice of ``token_count * elements-per-token`` elements."""
    plan, offset = [], 0
    for slab in layout["slabs"]:
        for layer in range(slab["count"]):
            n = int(token_count) * slab["elements-per-token"]
            plan.append({"slab": slab["name"], "layer": layer, "element-offset": offset, "elements": n})
            offset += n
    return plan


def transfer_runs(route: Route, start: int, token_count: int, page_size: int) -> list:
    """page_pool.clj:80-103: maximal runs of physically consecutive tokens."""
    runs, rel = [], 0
    while rel != token_count:
        logical = start + rel
        page = route.pages[logical // page_size]
        offset = logical % page_size
        n = min(token_count - rel, page_size - offset)
        phys = page * page_size + offset
        if runs and phys == runs[-1]["physical-token"] + runs[-1]["token-count"]:
            runs[-1]["token-count"] += n
        else:
            runs.append({"relative-token": rel, "physical-token": phys, "token-count": n})
        rel += n
    return runs


def direct_entries(layout: dict, plan: list, runs: list) -> list:
    """The reference's ranged copies (direct-restore-entries :1147-1167,
    direct-export-entries :1247-1265): one per (slab, layer, run), as
    ``{slab, layer, pool-element, payload-element, elements}``."""
    per = {s["name"]: s["elements-per-token"] for s in layout["slabs"]}
    out = []
    for e in plan:
        ept = per[e["slab"]]
        for r in runs:
            out.append({"slab": e["slab"], "layer": e["layer"], "pool-element": r["physical-token"] * ept,
                        "payload-element": e["element-offset"] + r["relative-token"] * ept,
                        "elements": r["token-count"] * ept})
    return out


# ---- telemetry ------------------------------------------------------------------
def _observe(current, value: float, alpha: float = DEFAULT_ALPHA) -> dict:
    """telemetry.clj:8-43 (update-observation)."""
    value = float(value)
    if not (np.isfinite(value) and value >= 0.0):
        raise PagePoolError("Telemetry observations must be non-negative and finite", value=value)
    if current is None:
        return {"count": 1, "ewma": value, "minimum": value, "maximum": value, "last": value}
    return {"count": current["count"] + 1, "ewma": alpha * value + (1.0 - alpha) * current["ewma"],
            "minimum": min(current["minimum"], value), "maximum": max(current["maximum"], value), "last": value}


def record_transfer(pool: PagePool, m: dict) -> None:
    """page_pool.clj:105-139: counters keyed (direction, timing-source,
    asynchronous?), the last measurement, and a bytes/ms calibration EWMA."""
    if getattr(pool, "transfers", None) is None:
        pool.transfers = {"counters": {}, "last": None}
    t = pool.transfers
    t["last"] = dict(m)
    key = (m["direction"], m["timing-source"], bool(m.get("asynchronous?")))
    c = t["counters"].setdefault(key, {})
    c["submissions"] = c.get("submissions", 0) + 1
    for k in ("bytes", "commands", "elapsed-ns", "submit-host-ns", "host-wall-ns"):
        c[k] = c.get(k, 0) + int(m.get(k, 0))
    metric = {"upload": "gpu-upload-bytes-per-ms", "download": "gpu-download-bytes-per-ms"}.get(m["direction"])
    wall = int(m.get("host-wall-ns", 0))
    if metric and int(m.get("bytes", 0)) > 0 and wall > 0:
        cal = t.setdefault("calibration", {})
        cal[metric] = _observe(cal.get(metric), m["bytes"] / (wall / 1.0e6))


def transfer_stats(pool: PagePool) -> dict:
    """page_pool.clj:437-444."""
    return getattr(pool, "transfers", None) or {"counters": {}, "last": None}


def _measurement(direction: str, stats: dict, commands: int, submit_ns: int, t0: int) -> dict:
    return {"direction": direction, "timing-source": "device-event", "asynchronous?": True,
            "bytes": stats["bytes"], "commands": commands, "elapsed-ns": int(stats["device_ms"] * 1e6),
            "submit-host-ns": submit_ns, "host-wall-ns": time.perf_counter_ns() - t0}


# ---- restore --------------------------------------------------------------------
def half_payload(payload, source_dtype, elements: int) -> np.ndarray:
    """page_pool.clj:1084-1109: an fp16 payload as is, an f32 payload for the
    device to round to fp16 (nearest even); lengths must match the descriptor."""
    dt = canonical_dtype(source_dtype)
    p = np.asarray(payload)
    if dt == "half" and p.dtype in (np.uint16, np.float16):
        if p.size != elements:
            raise PagePoolError("FP16 payload length differs from its descriptor", expected=elements, actual=p.size)
        return np.ascontiguousarray(p.view(np.uint16).ravel())
    if dt == "float" and p.dtype == np.float32:
        if p.size != elements:
            raise PagePoolError("FP32 payload length differs from its descriptor", expected=elements, actual=p.size)
        return np.ascontiguousarray(p.ravel())
    raise PagePoolError("Payload dtype and representation cannot be restored to FP16",
                        source_dtype=source_dtype, payload_type=str(p.dtype))


def restore_chunk_plan(pool: PagePool, cid, descriptor: dict, payload) -> dict:
    """page_pool.clj:1111-1145."""
    r = pool.route(cid)
    start, count = int(descriptor["chunk/start"]), int(descriptor["chunk/token-count"])
    src_layout = descriptor.get("chunk/layout", {})
    src_att = src_layout.get("attention-state", {})
    src_dtype = src_att.get("dtype", src_layout.get("dtype"))
    layout = pool_layout(pool)
    plan = payload_plan(layout, count)
    expected = sum(e["elements"] for e in plan)
    if r is None:
        raise PagePoolError("Cannot restore into a nonresident continuation", continuation_id=cid)
    if r.pending is not None:
        raise PagePoolError("Cannot restore while an append is pending", continuation_id=cid)
    if start < 0 or count <= 0 or start + count > r.token_count:
        raise PagePoolError("Chunk range is outside the resident continuation", start=start, token_count=count,
                            resident_tokens=r.token_count)
    keys = ("kind", "token-axis", "slabs")
    if {k: src_att.get(k) for k in keys} != {k: layout[k] for k in keys}:
        raise PagePoolError("Chunk attention-state layout differs from the device pool")
    if pool.dtype != "half":
        raise PagePoolError("Chunk restore conversion currently targets FP16 device pools", pool_dtype=pool.dtype)
    return {"route": r, "start": start, "token-count": count, "plan": plan,
            "source": half_payload(payload, src_dtype, expected),
            "runs": transfer_runs(r, start, count, pool.page_size)}


class ChunkTransfer:
    """A submitted restore (page_pool.clj ChunkTransfer): the device transfer,
    the route and the caller's retained resources (closed on completion)."""

    def __init__(self, pool, transfer, route, retained, commands, submit_ns, t0):
        self.pool, self.transfer, self.route, self.retained = pool, transfer, route, list(retained)
        self.commands, self.submit_ns, self.t0 = commands, submit_ns, t0


def submit_restore_chunk(pool: PagePool, cid, descriptor: dict, payload, retained=()) -> ChunkTransfer:
    """page_pool.clj:1169-1184: submits without waiting; ``retained`` objects
    (with ``close()``) are released only after device completion."""
    plan = restore_chunk_plan(pool, cid, descriptor, payload)
    t0 = time.perf_counter_ns()
    tr = pool.device.restore_submit(plan["route"].pages, plan["start"], plan["token-count"], plan["source"])
    return ChunkTransfer(pool, tr, plan["route"], retained, len(plan["plan"]) * len(plan["runs"]),
                         time.perf_counter_ns() - t0, t0)


def _check_owner(pool, obj, kind):
    if obj.pool is not pool:
        raise PagePoolError(f"Chunk {kind} belongs to a different page pool")


def chunk_transfer_complete(pool: PagePool, transfer: ChunkTransfer) -> bool:
    """page_pool.clj:1186-1193."""
    _check_owner(pool, transfer, "transfer")
    return transfer.transfer.done()


def complete_restore_chunk(pool: PagePool, transfer: ChunkTransfer) -> Route:
    """page_pool.clj:1195-1209: waits, records the measurement, releases."""
    _check_owner(pool, transfer, "transfer")
    try:
        stats = transfer.transfer.complete()
        record_transfer(pool, _measurement("upload", stats, transfer.commands, transfer.submit_ns, transfer.t0))
        return transfer.route
    finally:
        for res in transfer.retained:
            res.close()


def restore_chunk(pool: PagePool, cid, descriptor: dict, payload) -> Route:
    """page_pool.clj:1211-1224: scatter one durable payload into an allocated route."""
    return complete_restore_chunk(pool, submit_restore_chunk(pool, cid, descriptor, payload))


# ---- export ---------------------------------------------------------------------
def export_chunk_plan(pool: PagePool, lease, cid, descriptor: dict) -> dict:
    """page_pool.clj:1226-1245."""
    r = lease.routes[0]
    start, count = int(descriptor["chunk/start"]), int(descriptor["chunk/token-count"])
    if r.start_position != 0:
        raise PagePoolError("Durable prefix export requires a zero absolute start position",
                            continuation_id=cid, start_position=r.start_position)
    if start < 0 or count <= 0 or start + count > r.token_count:
        raise PagePoolError("Chunk range is outside the resident continuation", start=start, token_count=count,
                            resident_tokens=r.token_count)
    return {"route": r, "start": start, "token-count": count, "plan": payload_plan(pool_layout(pool), count),
            "runs": transfer_runs(r, start, count, pool.page_size)}


def exported_chunk(pool: PagePool, fingerprint, descriptor: dict, plan: list, payload) -> dict:
    """page_pool.clj:1267-1286: the portable durable chunk (version 3)."""
    durable = dict(pool_layout(pool), dtype="float16", **{"byte-order": "little-endian"})
    out = dict(descriptor)
    out.update({"chunk/version": 3, "chunk/model-fingerprint": fingerprint,
                "chunk/layout": {"dtype": "float16", "byte-order": "little-endian", "attention-state": durable},
                "chunk/slabs": plan, "chunk/payload": payload})
    if len({e["elements"] for e in plan}) == 1:
        out["chunk/elements-per-slab"] = plan[0]["elements"]
    return out


class ChunkExport:
    """A submitted export (page_pool.clj ChunkExport): holds a route lease until
    the device has written the payload."""

    def __init__(self, pool, transfer, route, descriptor, fingerprint, plan, lease, commands, submit_ns, t0):
        self.pool, self.transfer, self.route, self.descriptor = pool, transfer, route, descriptor
        self.fingerprint, self.plan, self.lease = fingerprint, plan, lease
        self.commands, self.submit_ns, self.t0 = commands, submit_ns, t0


def submit_export_chunk(pool: PagePool, cid, fingerprint, descriptor: dict) -> ChunkExport:
    """page_pool.clj:1288-1318: leases the route for the whole download; a
    failed submission releases the lease at once."""
    if pool.dtype != "half":
        raise PagePoolError("Paged chunk export currently requires an FP16 page pool", pool_dtype=pool.dtype)
    lease = pool.acquire_lease([cid])
    try:
        plan = export_chunk_plan(pool, lease, cid, descriptor)
        t0 = time.perf_counter_ns()
        tr = pool.device.export_submit(plan["route"].pages, plan["start"], plan["token-count"])
        return ChunkExport(pool, tr, plan["route"], descriptor, fingerprint, plan["plan"], lease,
                           len(plan["plan"]) * len(plan["runs"]), time.perf_counter_ns() - t0, t0)
    except BaseException:
        pool.release_lease(lease)
        raise


def chunk_export_complete(pool: PagePool, export: ChunkExport) -> bool:
    """page_pool.clj:1320-1327."""
    _check_owner(pool, export, "export")
    return export.transfer.done()


def complete_export_chunk(pool: PagePool, export: ChunkExport) -> dict:
    """page_pool.clj:1329-1345: waits, records, releases the lease, returns the chunk."""
    _check_owner(pool, export, "export")
    try:
        stats = export.transfer.complete()
        record_transfer(pool, _measurement("download", stats, export.commands, export.submit_ns, export.t0))
        return exported_chunk(pool, export.fingerprint, export.descriptor, export.plan, stats["payload"])
    finally:
        pool.release_lease(export.lease)


def export_chunk(pool: PagePool, cid, fingerprint, descriptor: dict) -> dict:
    """page_pool.clj:1347-1374: gather one immutable route range into the
    durable fp16 chunk format."""
    return complete_export_chunk(pool, submit_export_chunk(pool, cid, fingerprint, descriptor))
