"""Synthetic continuous-batching workloads, planned through the control-plane
mirror into device-resident step schedules.

The planner admits requests into fixed decode lanes the way the reference's
worker does (``src/pretrained/continuation/worker.clj:12-111``: retain running
lanes, refill free lanes from the queue, retire on length): each admission
reserves projected capacity (prompt + output, ``residency.clj:159-179`` /
``page_pool.clj:567-611``), allocates the route for the restored prefix (KV
holds prompt-1 rows, the last prompt token is the pending input,
``continuation.clj:1-8``), fills its pages with synthetic fp16 K/V (standing in
for a restored prefix) and primes the lane.  Every step then goes through
``PagedDecoder.step_lanes`` with a recording device, which captures the exact
descriptors, copy-on-write copies and primes the GPU will replay.
"""
from __future__ import annotations

import collections
import time

import numpy as np

from . import residency
from .page_pool import PagePool, PagePoolError
from .paged_decoder import PagedDecoder


class RecordingDevice:
    """Device protocol implementation that records instead of executing."""

    def __init__(self):
        self.cur = None

    def begin(self):
        self.cur = {"fill_pages": [], "cow_pairs": [], "prime_lanes": [], "prime_tokens": []}

    def end(self):
        st, self.cur = self.cur, None
        return st

    def copy_page(self, src, dst):
        self.cur["cow_pairs"].append((src, dst))

    def fill(self, pages):
        self.cur["fill_pages"].extend(int(p) for p in pages)

    def prime_rows(self, lane_tokens):
        for lt in lane_tokens:
            self.cur["prime_lanes"].append(int(lt["lane"]))
            self.cur["prime_tokens"].append(int(lt["token"]))

    def upload(self, desc):
        self.cur.update({k: np.array(v, np.int32) for k, v in desc.items()})

    def run(self):
        pass

    def download_tokens(self):
        return np.zeros(len(self.cur["slots"]), np.int32)


class LiveDevice:
    """Device protocol implementation that executes each call on the HIP decoder
    as the control plane makes it (the live serving loop): fills and
    copy-on-write copies on the pool, primes and one ``rstr_step_lanes`` per step
    on the decoder.  Seconds spent inside ``rstr_step_lanes`` are accumulated."""

    def __init__(self, decoder, pool, fill_seed: int = 7):
        self.decoder, self.pool, self.fill_seed = decoder, pool, fill_seed
        self.cur = None
        self.step_seconds = 0.0
        self.other_seconds = 0.0
        self.phase_ms = collections.Counter()  # summed rstr_step_lanes phases

    def begin(self):
        self.cur = {"fill_pages": [], "cow_pairs": [], "prime_lanes": [], "prime_tokens": []}

    def end(self):
        st, self.cur = self.cur, None
        return st

    def copy_page(self, src, dst):
        t0 = time.perf_counter()
        self.pool.copy_page(int(src), int(dst))
        self.other_seconds += time.perf_counter() - t0

    def fill(self, pages):
        pages = [int(p) for p in pages]
        if pages:
            t0 = time.perf_counter()
            self.pool.fill_synthetic(pages, self.fill_seed)
            self.other_seconds += time.perf_counter() - t0

    def prime_rows(self, lane_tokens):
        if lane_tokens:
            t0 = time.perf_counter()
            self.decoder.prime_lanes([lt["lane"] for lt in lane_tokens], [lt["token"] for lt in lane_tokens])
            self.other_seconds += time.perf_counter() - t0

    def upload(self, desc):
        self._desc = desc

    def run(self):
        t0 = time.perf_counter()
        self._tokens = self.decoder.step_lanes(**self._desc)
        self.step_seconds += time.perf_counter() - t0
        self.phase_ms.update(self.decoder.step_timing())

    def download_tokens(self):
        return self._tokens


class PermutedPages:
    """Device protocol wrapper that places the pool's pages at a fixed permutation
    of the physical page pool: page p of the control plane is physical page
    ``perm[p]`` in every fill, copy-on-write copy, slot and page-table entry the
    wrapped device sees.  The pool keeps its lowest-free-first order
    (page_pool.clj:513-524) over its own ids, so route tables land on scattered
    physical pages, as a long-running pool's free list leaves them (BASELINE.json
    page tables are a random permutation of the physical pool)."""

    def __init__(self, inner, physical_pages: int, page_size: int, seed: int):
        self.inner, self.page_size = inner, int(page_size)
        self.perm = np.random.default_rng(seed).permutation(int(physical_pages)).astype(np.int32)

    def begin(self):
        self.inner.begin()

    def end(self):
        return self.inner.end()

    def copy_page(self, src, dst):
        self.inner.copy_page(int(self.perm[src]), int(self.perm[dst]))

    def fill(self, pages):
        self.inner.fill([int(self.perm[p]) for p in pages])

    def prime_rows(self, lane_tokens):
        self.inner.prime_rows(lane_tokens)

    def upload(self, desc):
        d = dict(desc)
        ps = self.page_size
        slots = np.asarray(desc["slots"], np.int64)
        d["slots"] = np.where(slots >= 0, self.perm[np.maximum(slots, 0) // ps].astype(np.int64) * ps + slots % ps,
                              slots).astype(np.int32)
        pt = np.asarray(desc["page_table"], np.int64)
        d["page_table"] = np.where(pt >= 0, self.perm[np.maximum(pt, 0)], pt).astype(np.int32)
        self.inner.upload(d)

    def run(self):
        self.inner.run()

    def download_tokens(self):
        return self.inner.download_tokens()


class ChurnPlanner:
    """Poisson arrivals, uniform prompt/output lengths, fixed lanes, fixed page pool.
    ``device`` executes the plan as it is made (``LiveDevice``); by default the
    steps are recorded for a device-resident schedule.  ``page_perm_seed`` places
    the pool's pages at a seeded permutation of the physical pool
    (``PermutedPages``)."""

    def __init__(self, cfg: dict, batch: int, page_size: int, physical_pages: int, maxpos: int,
                 seed: int, arrival_mean: float = 4.0, prompt=(128, 4096), output=(32, 512),
                 fill_seed: int = 7, warm_start: bool = True, retain_finished: bool = False, device=None,
                 page_perm_seed: int | None = None):
        self.cfg, self.batch, self.maxpos = cfg, batch, maxpos
        self.rng = np.random.default_rng(seed)
        self.arrival_mean, self.prompt, self.output = arrival_mean, prompt, output
        self.fill_seed = fill_seed
        self.rec = device if device is not None else RecordingDevice()
        if page_perm_seed is not None:
            self.rec = PermutedPages(self.rec, physical_pages, page_size, page_perm_seed)
        self.pool = PagePool(page_size, physical_pages, cfg["n_layers"], cfg["n_kv"], cfg["head_dim"],
                             device=self.rec)
        self.dec = PagedDecoder(self.pool, self.rec, batch_size=batch, maxpos=maxpos)
        self.lanes = [None] * batch
        self.queue = collections.deque()
        self.next_id = 0
        self.warm_start = warm_start
        self.steps_planned = 0
        self.host_seconds = 0.0
        self.retired = 0
        self.rejected_admissions = 0
        # retain_finished: finished continuations stay resident as durable
        # routes (a prefix cache) and admissions evict them by value
        # (residency.clj) when the pool runs short
        self.retain_finished = retain_finished
        self.evicted = 0

    def _arrive(self, n):
        for _ in range(n):
            p = int(self.rng.integers(self.prompt[0], self.prompt[1] + 1))
            o = int(self.rng.integers(self.output[0], self.output[1] + 1))
            self.queue.append({"id": self.next_id, "prompt": p, "output": o,
                               "token": int(self.rng.integers(0, self.cfg["vocab"]))})
            self.next_id += 1

    def _admit(self, lane, req, progress=0):
        cid = req["id"]
        if self.retain_finished:
            plan = residency.reserve_admission(self.pool, cid, req["prompt"] + req["output"],
                                               {st["cid"] for st in self.lanes if st is not None})
            if not plan["admissible?"]:
                self.rejected_admissions += 1
                return False
            self.evicted += len(plan["evictions"])
            cap = plan["capacity-reservation"]
        else:
            try:
                cap = self.pool.reserve_capacity(cid, req["prompt"] + req["output"])
            except PagePoolError:
                self.rejected_admissions += 1
                return False
        route = self.pool.allocate_route(cid, req["prompt"] - 1 + progress, capacity_reservation=cap)
        self.rec.fill(route.pages)
        self.dec.prime_lanes([{"lane": lane, "token": req["token"]}])
        self.lanes[lane] = {"cid": cid, "cap": cap, "left": req["output"] - progress}
        return True

    def plan_step(self) -> dict:
        t0 = time.perf_counter()
        self.rec.begin()
        if self.steps_planned == 0 and self.warm_start:
            # steady-state start: every lane holds a request part-way through its output
            self._arrive(self.batch)
            for lane in range(self.batch):
                req = self.queue.popleft()
                self._admit(lane, req, progress=int(self.rng.integers(0, req["output"])))
        self._arrive(int(self.rng.poisson(self.arrival_mean)))
        for lane in range(self.batch):
            if self.lanes[lane] is None and self.queue:
                if not self._admit(lane, self.queue[0]):
                    break
                self.queue.popleft()
        work = []
        for lane, st in enumerate(self.lanes):
            if st is not None:
                r = self.pool.route(st["cid"])
                work.append({"lane": lane, "continuation_id": st["cid"],
                             "position": r.start_position + r.token_count})
        self.dec.step_lanes(work)
        for lane, st in enumerate(self.lanes):
            if st is None:
                continue
            st["left"] -= 1
            if st["left"] <= 0:
                if self.retain_finished:
                    r = self.pool.route(st["cid"])
                    self.pool.touch_route(st["cid"], {
                        "durable?": True, "last-access": self.steps_planned,
                        "reuse-probability": float(self.rng.uniform(0.0, 1.0)),
                        "recompute-ms": 0.05 * r.token_count, "reload-ms": 0.01 * r.token_count})
                else:
                    self.pool.release_route(st["cid"])
                self.pool.release_capacity(st["cap"])
                self.lanes[lane] = None
                self.retired += 1
        out = self.rec.end()
        out["fill_seed"] = self.fill_seed
        out["active"] = len(work)
        self.steps_planned += 1
        self.host_seconds += time.perf_counter() - t0
        return out


STEP_DESCRIPTORS = ("slots", "row_offsets", "positions", "page_table", "lengths", "start_positions")


class PipelinedLive:
    """The live serving loop with the host control plane one step ahead of the
    GPU, in one thread.  ``planner`` records its steps (a planner built without
    ``device``).  Step n is enqueued with ``rstr_step_lanes_submit`` and the
    planner makes step n+1 while the device runs it; step n+1's fills,
    copy-on-write copies and primes then run on the pool and the decoder in the
    order the device-resident schedule applies them (``enqueue_staged_prelude``:
    fills, copies, primes) -- each of those calls runs after step n in stream
    order -- step n+1 is submitted, and only then are step n's tokens
    collected.  The device receives the same calls in the same order as in the
    sequential loop (``LiveDevice``).  Planning step n+1 ahead is sound here
    because the planner's decisions depend on lengths and arrivals, not on
    token values: pages it frees while step n still reads them are refilled or
    copied only after step n, in stream order."""

    def __init__(self, planner, decoder, pool):
        self.planner, self.decoder, self.pool = planner, decoder, pool
        self.inflight = 0
        self.plan_seconds = 0.0

    def _apply(self, st):
        if len(st["fill_pages"]):
            self.pool.fill_synthetic(st["fill_pages"], st["fill_seed"])
        for src, dst in st["cow_pairs"]:
            self.pool.copy_page(int(src), int(dst))
        if len(st["prime_lanes"]):
            self.decoder.prime_lanes(st["prime_lanes"], st["prime_tokens"])

    def _plan(self):
        t0 = time.perf_counter()
        st = self.planner.plan_step()
        self.plan_seconds += time.perf_counter() - t0
        return st

    def _submit(self, st):
        self.decoder.step_lanes_submit(**{k: st[k] for k in STEP_DESCRIPTORS})
        self.inflight += 1

    def _collect(self):
        self.inflight -= 1
        return self.decoder.step_lanes_collect()

    def start(self):
        """Plan and submit the first step."""
        try:
            st = self._plan()
            self._apply(st)
            self._submit(st)
        except BaseException:
            self._teardown()
            raise
        return st

    def step(self):
        """Plan and submit the next step while the running one finishes;
        returns the finished step's tokens ([batch] int32) and the step just
        submitted.  On an error every submitted step is collected before the
        error propagates."""
        try:
            st = self._plan()
            self._apply(st)
            self._submit(st)
            tokens = self._collect()
        except BaseException:
            self._teardown()
            raise
        return tokens, st

    def finish(self):
        """Wait for the running step; returns its tokens."""
        try:
            tokens = self._collect()
        finally:
            self._teardown()
        return tokens

    def _teardown(self):
        """No submitted step left in flight on the decoder."""
        while self.inflight > 0:
            try:
                self._collect()
            except BaseException:
                self.inflight = 0


class SharedPrefixPlanner:
    """A fixed set of decode lanes whose first ``shared_lanes`` fork one resident
    prefix: contexts log-uniform in ``ctx``; a lane of
    the shared group forks the prefix route at min(ctx, prefix) - 1 rows
    (``fork-route!``, page_pool.clj:679-724) and appends its private rows with a
    range reservation, so the shared partial tail page is copied on the first
    divergent append (page_pool.clj:923-944); the other lanes hold private
    routes.  Every lane then decodes every step (no retirement)."""

    def __init__(self, cfg: dict, batch: int, page_size: int, physical_pages: int, maxpos: int,
                 seed: int, ctx=(256, 8192), shared_lanes: int = 32, prefix: int = 1024, fill_seed: int = 7):
        self.cfg, self.batch, self.maxpos = cfg, batch, maxpos
        self.rng = np.random.default_rng(seed)
        self.ctx, self.shared_lanes, self.prefix = ctx, shared_lanes, prefix
        self.fill_seed = fill_seed
        self.rec = RecordingDevice()
        self.pool = PagePool(page_size, physical_pages, cfg["n_layers"], cfg["n_kv"], cfg["head_dim"],
                             device=self.rec)
        self.dec = PagedDecoder(self.pool, self.rec, batch_size=batch, maxpos=maxpos)
        self.steps_planned = 0
        self.host_seconds = 0.0
        self.retired = 0
        self.rejected_admissions = 0
        self.cow_pages = 0

    def _start(self):
        lo, hi = np.log(self.ctx[0]), np.log(self.ctx[1])
        ctx = np.exp(self.rng.uniform(lo, hi, self.batch)).astype(np.int64)
        root = "prefix"
        r = self.pool.allocate_route(root, self.prefix - 1)
        self.rec.fill(r.pages)
        for lane in range(self.batch):
            c = int(ctx[lane])
            if lane < self.shared_lanes:
                n = min(c, self.prefix) - 1
                self.pool.fork_route(root, lane, n)
                extra = c - 1 - n
                if extra > 0:
                    res = self.pool.reserve_append_range(lane, extra)
                    self.rec.fill(res.added_pages)
                    self.pool.commit_append(lane, res)
            else:
                self.rec.fill(self.pool.allocate_route(lane, c - 1).pages)
            tok = int(self.rng.integers(0, self.cfg["vocab"]))
            self.dec.prime_lanes([{"lane": lane, "token": tok}])
        # the lanes hold their own references; the prefix stays resident for reuse
        self.pool.touch_route(root, {"durable?": True})

    def plan_step(self) -> dict:
        t0 = time.perf_counter()
        self.rec.begin()
        if self.steps_planned == 0:
            self._start()
        work = []
        for lane in range(self.batch):
            r = self.pool.route(lane)
            work.append({"lane": lane, "continuation_id": lane, "position": r.start_position + r.token_count})
        self.dec.step_lanes(work)
        out = self.rec.end()
        self.cow_pages += len(out["cow_pairs"])
        out["fill_seed"] = self.fill_seed
        out["active"] = len(work)
        self.steps_planned += 1
        self.host_seconds += time.perf_counter() - t0
        return out


def step_bytes(cfg: dict, step: dict, weight_bytes: int) -> dict:
    """Algorithmic HBM bytes of one decode step: packed weights once, the visible
    fp16 K+V of every layer (window-limited on local layers; logical rows, which
    equal unique rows when no pages are shared), fp16 appends, embedding gather."""
    L, kvr, d = cfg["n_layers"], cfg["n_kv"] * cfg["head_dim"], cfg["d_model"]
    lengths = np.asarray(step["lengths"], np.int64)
    active = lengths > 0
    per_layer_kv = []
    for layer in range(L):
        glob = cfg["global_pattern"] <= 0 or (layer + 1) % cfg["global_pattern"] == 0
        w = cfg["sliding_window"] if (cfg["sliding_window"] > 0 and not glob) else 0
        vis = np.minimum(lengths, w) if w else lengths
        per_layer_kv.append(int(vis.sum()) * kvr * 2 * 2)
    kv = sum(per_layer_kv)
    appends = int(active.sum()) * L * kvr * 2 * 2
    gather = int(active.sum()) * d * 4
    out = {"weights": weight_bytes, "kv": kv, "kv_per_layer": per_layer_kv, "appends": appends,
           "gather": gather, "total": weight_bytes + kv + appends + gather}
    if "page_table" in step and cfg["sliding_window"] <= 0:
        # physical pages shared by several lanes count once (the rows any lane reads)
        ps = int(step.get("page_size", 16))
        pt = np.asarray(step["page_table"], np.int64).reshape(len(lengths), -1)
        lanes = np.nonzero(active)[0]
        n = lengths[lanes]
        npg = -(-n // ps)
        lane_of = np.repeat(lanes, npg)
        idx = np.arange(int(npg.sum())) - np.repeat(np.cumsum(npg) - npg, npg)
        pg = pt[lane_of, idx]
        rows = np.minimum(ps, np.repeat(n, npg) - idx * ps)
        order = np.argsort(pg, kind="stable")
        pg, rows = pg[order], rows[order]
        starts = np.concatenate([[0], np.flatnonzero(np.diff(pg)) + 1]) if pg.size else np.zeros(0, np.int64)
        ukv = int(np.maximum.reduceat(rows, starts).sum()) * kvr * 2 * 2 if pg.size else 0
        out["kv_unique_per_layer"] = ukv
        out["kv_unique"] = ukv * L
        out["total_unique"] = weight_bytes + ukv * L + appends + gather
    return out


def shared_prefix_routes(B: int, seed: int, page_size: int = 16, mu: float = 7.0, sigma: float = 1.2,
                         lo: int = 16, hi: int = 32768, shared_frac: float = 0.25):
    """The isolated-attention workload's routes: B lanes with
    contexts lognormal(mu, sigma) clipped to [lo, hi], permuted physical page ids,
    and the first ``shared_frac`` of every lane's full pages taken from one shared
    run of pages (a common prefix).  Returns (lengths, page_table, physical_pages,
    shared pages per lane, the generator), the generator positioned after the
    routes' draws (the workload's queries come next)."""
    rng = np.random.default_rng(seed)
    lengths = np.clip(np.rint(np.exp(rng.normal(mu, sigma, B))), lo, hi).astype(np.int32)
    full = lengths // page_size
    npages = -(-lengths // page_size)
    shared_n = np.rint(shared_frac * full).astype(np.int64)
    S = int(shared_n.max())
    physical = S + int((npages - shared_n).sum())
    perm = rng.permutation(physical).astype(np.int32)
    shared_pages, priv_pages = perm[:S], perm[S:]
    pt = np.full((B, int(npages.max())), -1, np.int32)
    used = 0
    for b in range(B):
        k = int(shared_n[b])
        pt[b, :k] = shared_pages[:k]
        n_priv = int(npages[b]) - k
        pt[b, k:npages[b]] = priv_pages[used:used + n_priv]
        used += n_priv
    return lengths, pt, physical, shared_n, rng
