"""Device-local continuous batching for a paged worker
(``src/pretrained/continuation/paged_runtime.clj``).

One runtime thread owns every decoder call.  Handler threads enqueue prompt
prefill jobs, decode jobs and synchronous operations and wait on futures; each
loop turn plans one iteration with the pure scheduler (``rstr.scheduler``) over
the decoder's fixed lanes, primes the rows that need an input token, runs one
lane step and advances every lane.  A one-lane runtime bound to a bulk-prefill
tile (``prefill_range``) spends a whole turn on one exact tile whenever the
lane holds a prefill job with at least a tile of tokens left, so decode work
admitted meanwhile runs before the next tile (paged_runtime.clj:84-135).
"""
from __future__ import annotations

import itertools
import queue
import threading
import time
import uuid
from concurrent.futures import CancelledError, Future

from . import scheduler
from .chunks import _observe

DEFAULT_ALPHA = 0.2


class RuntimeError_(RuntimeError):
    pass


class _Job(dict):
    """A queued unit of work; identity by ``job_id``.  Lanes carry copies of a
    job as it advances; ``cancel`` is one shared cell, so a cancellation marked
    on the registry's copy is seen by the lane's."""


def _record(cal: dict, metric: str, value: float, alpha: float) -> dict:
    cal = dict(cal)
    cal[metric] = _observe(cal.get(metric), value, alpha)
    return cal


class PagedRuntime:
    """open-runtime (paged_runtime.clj:341-436) and the record's close (:321-339)."""

    def __init__(self, decoder, capacity=None, minimum_prefill_tokens=None, eos_ids=(), max_position=None,
                 prime_lanes=None, step_lanes=None, prefill_range=None, prefill_tile_size=None,
                 route_token_count=None, calibration_alpha=DEFAULT_ALPHA, on_error=None):
        dec_cap = getattr(decoder, "batch_size", None)
        capacity = capacity if capacity is not None else (dec_cap or 1)
        if minimum_prefill_tokens is None:
            minimum_prefill_tokens = 1 if capacity > 1 else 0
        max_position = max_position if max_position is not None else getattr(decoder, "maxpos", None)
        dec_tile = getattr(decoder, "prefill_T", None)
        prefill_tile_size = prefill_tile_size if prefill_tile_size is not None else dec_tile
        if prefill_range is None and prefill_tile_size and dec_tile and hasattr(decoder, "prefill_range"):
            prefill_range = lambda d, cid, toks, pos: d.prefill_range(cid, toks, pos)  # noqa: E731
        if not (isinstance(capacity, int) and capacity > 0):
            raise RuntimeError_("Paged runtime capacity must be a positive integer")
        if isinstance(dec_cap, int) and capacity > dec_cap:
            raise RuntimeError_("Paged runtime exceeds the decoder's fixed batch")
        if not (isinstance(minimum_prefill_tokens, int) and 0 <= minimum_prefill_tokens <= capacity):
            raise RuntimeError_("Paged runtime prefill reservation is invalid")
        if not (isinstance(max_position, int) and max_position > 0):
            raise RuntimeError_("Paged runtime requires a positive maximum position")
        if prefill_range is not None and not (capacity == 1 and isinstance(prefill_tile_size, int)
                                              and prefill_tile_size > 0):
            raise RuntimeError_("Bulk prefill requires a positive tile and one runtime lane")
        if prefill_range is not None and dec_tile and prefill_tile_size != dec_tile:
            raise RuntimeError_("Runtime tile must match the decoder's compiled prefill rows")
        if not all(isinstance(e, int) for e in eos_ids):
            raise RuntimeError_("Paged runtime EOS ids must be integers")
        if not (0.0 < float(calibration_alpha) <= 1.0):
            raise RuntimeError_("Runtime calibration alpha must be in (0,1]")
        self.decoder, self.capacity = decoder, capacity
        self.minimum_prefill_tokens = minimum_prefill_tokens
        self.eos_ids, self.max_position = set(eos_ids), max_position
        self.prime_lanes = prime_lanes or (lambda d, values: d.prime_lanes(values))
        self.step_lanes = step_lanes or (lambda d, work: d.step_lanes(work))
        self.prefill_range = prefill_range
        self.prefill_tile_size = prefill_tile_size
        self.route_token_count = route_token_count or (lambda d, cid: d.pool.route(cid).token_count)
        self.alpha = float(calibration_alpha)
        self.on_error = on_error or (lambda e: None)
        self.inbound: queue.Queue = queue.Queue()
        self.registry: dict = {}
        self._arrival = itertools.count()
        self._lock = threading.RLock()
        self._state = {"iterations": 0, "scheduled-tokens": 0, "bulk-prefill-tiles": 0,
                       "bulk-prefill-tokens": 0, "bulk-prefill-nanos": 0, "calibration": {},
                       "lanes": [None] * capacity, "deferred-count": 0}
        self.closed = False
        self.thread = threading.Thread(target=self._run_loop, name="rstr-paged-runtime", daemon=True)
        self.thread.start()

    # ---- lifecycle ------------------------------------------------------------
    def close(self):
        with self._lock:
            if self.closed:
                return
            self.closed = True
            for job in list(self.registry.values()):
                job["cancel"][0] = True
                self._fail(job, RuntimeError_("Paged runtime is closed"))
        self.inbound.put({"type": "stop"})
        self.thread.join(timeout=5)

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def state(self) -> dict:
        """paged_runtime.clj:438-451."""
        with self._lock:
            s = dict(self._state)
            tokens = s["bulk-prefill-tokens"]
            ms = s["bulk-prefill-nanos"] / 1.0e6
            s.update({"prefill-tile-size": self.prefill_tile_size if self.prefill_range else None,
                      "bulk-prefill-milliseconds": ms, "active-job-count": len(self.registry),
                      "inbound-queue-depth": self.inbound.qsize()})
            if tokens > 0:
                s["bulk-prefill-ms-per-token"] = ms / tokens
            return s

    # ---- job plumbing ---------------------------------------------------------
    def _job(self, type_, **values) -> _Job:
        j = _Job(values)
        j.update({"job_id": uuid.uuid4(), "type": type_, "future": Future(), "cancel": [False],
                  "arrival": next(self._arrival)})
        return j

    def _complete(self, job, value):
        with self._lock:
            self.registry.pop(job["job_id"], None)
        if not job["future"].done():
            job["future"].set_result(value)

    def _fail(self, job, error):
        with self._lock:
            self.registry.pop(job["job_id"], None)
        if not job["future"].done():
            job["future"].set_exception(error)

    @staticmethod
    def _cancelled(job) -> bool:
        return job["cancel"][0] or job["future"].cancelled()

    def _await(self, job):
        """paged_runtime.clj:453-470."""
        with self._lock:
            if self.closed:
                raise RuntimeError_("Paged runtime is closed")
            self.registry[job["job_id"]] = job
            self.inbound.put(job)
        return job["future"].result()

    def cancel_assignment(self, assignment_id) -> int:
        """paged_runtime.clj:626-639: marks the jobs; the loop fails them at its next boundary."""
        with self._lock:
            jobs = [j for j in self.registry.values() if j.get("assignment_id") == assignment_id]
            for j in jobs:
                j["cancel"][0] = True
            if jobs:
                self.inbound.put({"type": "wake"})
            return len(jobs)

    def run_operation(self, operation, assignment_id=None):
        """paged_runtime.clj:480-495: a synchronous device/storage operation between iterations."""
        if not callable(operation):
            raise RuntimeError_("Paged runtime operation must be callable")
        return self._await(self._job("operation", assignment_id=assignment_id, operation=operation))

    def run_background_operation(self, assignment_id, operation):
        """paged_runtime.clj:497-539: runs on the calling thread, fenced by cancellation."""
        if not callable(operation):
            raise RuntimeError_("Paged background operation must be callable")
        job = self._job("background", assignment_id=assignment_id)
        with self._lock:
            if self.closed:
                raise RuntimeError_("Paged runtime is closed")
            self.registry[job["job_id"]] = job
        try:
            result = operation(lambda: self._cancelled(job))
            with self._lock:
                if self._cancelled(job):
                    err = CancelledError("Paged background operation was cancelled")
                    self._fail(job, err)
                    raise err
                self._complete(job, result)
                return result
        except BaseException as e:
            if job["job_id"] in self.registry:
                self._fail(job, e)
            raise

    # ---- requests ----------------------------------------------------------------
    def prefill(self, effect: dict) -> dict:
        """paged_runtime.clj:541-573: compute the uncached prompt suffix in lanes."""
        req = effect["request"]
        prompt = list(req["tokens"])
        cid = req.get("continuation_id", req["id"])
        if not prompt:
            raise RuntimeError_("Paged runtime prefill requires a nonempty prompt")
        if not all(isinstance(t, int) for t in prompt):
            raise RuntimeError_("Paged runtime prompt tokens must be integers")
        cached = int(self.route_token_count(self.decoder, cid))
        remaining = len(prompt) - 1 - cached
        if remaining < 0:
            raise RuntimeError_("Resident prefix is longer than the submitted prompt")
        if remaining == 0:
            return {"ok?": True}
        return self._await(self._job("prefill", assignment_id=effect["id"], id=(effect["id"], "prefill"),
                                     phase="prefill", remaining_tokens=remaining, continuation_id=cid,
                                     position=cached, prompt=prompt))

    def decode(self, effect: dict, token_callback=None) -> dict:
        """paged_runtime.clj:575-609: generate until EOS, the budget or the route's capacity."""
        req = effect["request"]
        prompt = list(req["tokens"])
        cid = req.get("continuation_id", req["id"])
        budget = req.get("max_new_tokens")
        if not prompt:
            raise RuntimeError_("Paged runtime decode requires a nonempty prompt")
        if not all(isinstance(t, int) for t in prompt):
            raise RuntimeError_("Paged runtime prompt tokens must be integers")
        if not (isinstance(budget, int) and budget > 0):
            raise RuntimeError_("Paged runtime decode requires a positive token budget")
        processed = len(prompt) - 1
        resident = int(self.route_token_count(self.decoder, cid))
        if processed != resident:
            raise RuntimeError_("Paged decode requires a completely primed prompt")
        return self._await(self._job("decode", assignment_id=effect["id"], id=(effect["id"], "decode"),
                                     phase="decode", remaining_tokens=budget, continuation_id=cid,
                                     position=processed, pending_token=prompt[-1], token_cb=token_callback,
                                     output=[]))

    # ---- the device loop ---------------------------------------------------------
    def _stop_reason(self, job, token, remaining):
        if remaining == 0:
            return "length"
        if token in self.eos_ids:
            return "eos"
        if int(self.route_token_count(self.decoder, job["continuation_id"])) >= self.max_position:
            return "capacity"
        return None

    def _advance(self, result, job):
        """paged_runtime.clj:175-214."""
        if self._cancelled(job):
            return None, ("fail", CancelledError("Paged lane was cancelled"))
        job = _Job({k: v for k, v in job.items() if k != "scheduled_tokens"})
        job["position"] += 1
        job["remaining_tokens"] -= 1
        if job["phase"] == "prefill":
            return (None, ("complete", {"ok?": True})) if job["remaining_tokens"] == 0 else (job, None)
        token = int(result["token"])
        output = job["output"] + [token]
        reason = self._stop_reason(job, token, job["remaining_tokens"])
        if job.get("token_cb"):
            job["token_cb"](token, len(output) - 1)
        if reason:
            return None, ("complete", {"ok?": True, "tokens": output, "stop-reason": reason})
        job["pending_token"], job["output"] = token, output
        return job, None

    def _bulk_job(self, plan):
        item = plan["lanes"][0] if plan["lanes"] else None
        if (self.capacity == 1 and self.prefill_range is not None and item is not None
                and item["phase"] == "prefill" and self.prefill_tile_size <= item["remaining_tokens"]):
            return item
        return None

    def _execute_bulk(self, job, deferred):
        """paged_runtime.clj:95-135: one exact tile for the lane's prefill job."""
        T = self.prefill_tile_size
        pos = job["position"]
        t0 = time.perf_counter_ns()
        self.prefill_range(self.decoder, job["continuation_id"], job["prompt"][pos:pos + T], pos)
        ns = time.perf_counter_ns() - t0
        cancelled = self._cancelled(job)
        remaining = job["remaining_tokens"] - T
        nxt = None
        if not cancelled and remaining > 0:
            nxt = _Job({k: v for k, v in job.items() if k != "scheduled_tokens"})
            nxt.update(position=pos + T, remaining_tokens=remaining)
        with self._lock:
            s = self._state
            s["iterations"] += 1
            s["scheduled-tokens"] += T
            s["bulk-prefill-tiles"] += 1
            s["bulk-prefill-tokens"] += T
            s["bulk-prefill-nanos"] += ns
            s["calibration"] = _record(s["calibration"], "prefill-ms-per-token", ns / 1.0e6 / T, self.alpha)
            s["lanes"] = [self._summary(nxt)]
            s["deferred-count"] = len(deferred)
        if cancelled:
            self._fail(job, CancelledError("Paged lane was cancelled"))
        elif remaining == 0:
            self._complete(job, {"ok?": True})
        return [nxt], deferred

    @staticmethod
    def _summary(job):
        if job is None:
            return None
        return {k: job.get(k) for k in ("id", "phase", "continuation_id", "remaining_tokens")}

    def _execute_lanes(self, lanes, deferred):
        """paged_runtime.clj:216-319."""
        jobs = []
        for j in [l for l in lanes if l is not None] + list(deferred):
            if self._cancelled(j):
                with self._lock:
                    self.registry.pop(j["job_id"], None)
                j["future"].cancel() or self._fail(j, CancelledError("Paged lane was cancelled"))
            else:
                jobs.append(j)
        if not jobs:
            with self._lock:
                self._state.update(lanes=[None] * self.capacity, **{"deferred-count": 0})
            return [None] * self.capacity, []
        it = scheduler.plan_iteration({"max_batched_tokens": self.capacity, "max_sequences": self.capacity,
                                       "prefill_chunk_size": 1, "repair_chunk_size": 1,
                                       "minimum_prefill_tokens": self.minimum_prefill_tokens}, jobs)
        plan = scheduler.plan_work_lanes(self.capacity, [self._lane_key(l) for l in lanes], it["scheduled"])
        deferred = list(it["deferred"]) + list(plan["deferred"])
        by_id = {j["id"]: j for j in jobs}
        plan_lanes = [None if l is None else _Job({**by_id[l["id"]], **l}) for l in plan["lanes"]]
        bulk = self._bulk_job({"lanes": plan_lanes})
        if bulk is not None:
            return self._execute_bulk(bulk, [by_id[d["id"]] for d in deferred])
        refill = {r["id"] for r in plan["refill"]}
        primes = []
        for l in plan_lanes:
            if l is None:
                continue
            if l["phase"] == "prefill":
                primes.append({"lane": l["lane_index"], "token": l["prompt"][l["position"]]})
            elif l["id"] in refill:
                primes.append({"lane": l["lane_index"], "token": l["pending_token"]})
        work = [{"lane": l["lane_index"], "continuation_id": l["continuation_id"], "position": l["position"]}
                for l in plan_lanes if l is not None]
        phases = [l["phase"] for l in plan_lanes if l is not None]
        first_token = any(l["phase"] == "decode" and not l["output"] for l in plan_lanes if l is not None)
        t0 = time.perf_counter_ns()
        if primes:
            self.prime_lanes(self.decoder, primes)
        results = self.step_lanes(self.decoder, work)
        ms = (time.perf_counter_ns() - t0) / 1.0e6
        by_lane = {r["lane"]: r for r in results}
        advanced = [None if l is None else self._advance(by_lane.get(l["lane_index"]), l) for l in plan_lanes]
        next_lanes = [None if a is None else a[0] for a in advanced]
        with self._lock:
            s = self._state
            s["iterations"] += 1
            s["scheduled-tokens"] += len(work)
            cal = _record(s["calibration"], "iteration-ms", ms, self.alpha)
            if phases and all(p == "decode" for p in phases):
                cal = _record(cal, "decode-iteration-ms", ms, self.alpha)
            if phases and all(p == "prefill" for p in phases):
                cal = _record(cal, "prefill-ms-per-token", ms / len(phases), self.alpha)
            if first_token:
                cal = _record(cal, "first-token-ms", ms, self.alpha)
            s["calibration"] = cal
            s["lanes"] = [self._summary(j) for j in next_lanes]
            s["deferred-count"] = len(deferred)
        for l, a in zip(plan_lanes, advanced):
            if a is not None and a[1] is not None:
                action, value = a[1]
                (self._complete if action == "complete" else self._fail)(l, value)
        return next_lanes, [by_id[d["id"]] for d in deferred]

    @staticmethod
    def _lane_key(job):
        return None if job is None else {k: v for k, v in job.items()}

    def _run_loop(self):
        """paged_runtime.clj:285-319."""
        operations, deferred, lanes = [], [], [None] * self.capacity
        try:
            while not self.closed:
                idle = not operations and not deferred and all(l is None for l in lanes)
                incoming = [self.inbound.get()] if idle else []
                while True:
                    try:
                        incoming.append(self.inbound.get_nowait())
                    except queue.Empty:
                        break
                if self.closed:
                    return
                operations += [j for j in incoming if j.get("type") == "operation"]
                deferred += [j for j in incoming if j.get("type") in ("prefill", "decode")]
                if operations:
                    op = operations.pop(0)
                    if self._cancelled(op):
                        self._fail(op, CancelledError("Paged operation was cancelled"))
                    else:
                        try:
                            r = op["operation"]()
                            if self._cancelled(op):
                                self._fail(op, CancelledError("Paged operation was cancelled"))
                            else:
                                self._complete(op, r)
                        except BaseException as e:
                            self._fail(op, e)
                lanes, deferred = self._execute_lanes(lanes, deferred)
        except BaseException as e:  # fail-runtime! (:149-155)
            if not self.closed:
                with self._lock:
                    self.closed = True
                    for job in list(self.registry.values()):
                        job["cancel"][0] = True
                        self._fail(job, e)
                self.on_error(e)


def open_runtime(decoder, **opts) -> PagedRuntime:
    """paged_runtime.clj:341-436."""
    return PagedRuntime(decoder, **opts)
