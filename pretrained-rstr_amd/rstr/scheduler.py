"""Pure iteration and cache-source planning for continuous-batching decode:
the host mirror of ``src/pretrained/continuation/scheduler.clj``.

Requests are dicts with the reference's ``:request/*`` fields in snake case
(``id``, ``phase``, ``remaining_tokens``, ``arrival``, ``continuation_id``,
``position``, ``pending_token``); planner annotations are ``lane_index``,
``scheduled_tokens`` and ``iteration_token``.  No function mutates its input.
Errors are ``SchedulerError`` (the reference's ex-info) with the same message.
"""
from __future__ import annotations

import numbers

PHASES = ("decode", "prefill", "repair")
_PHASE_RANK = {"decode": 0, "repair": 1, "prefill": 2}
_SOURCE_RANK = {"resident-exact": 0, "restore-exact": 1, "recompute-exact": 2, "modular-repair": 3}


class SchedulerError(ValueError):
    def __init__(self, msg: str, **data):
        super().__init__(msg)
        self.data = data


def _is_int(v) -> bool:
    return isinstance(v, numbers.Integral) and not isinstance(v, bool)


def _is_num(v) -> bool:
    return isinstance(v, numbers.Real) and not isinstance(v, bool)


def request(value: dict) -> dict:
    """Validate and normalize one schedulable request (scheduler.clj:11-31);
    ``arrival`` defaults to zero."""
    if value.get("id") is None:
        raise SchedulerError("Scheduled request requires :request/id", request=value)
    if value.get("phase") not in PHASES:
        raise SchedulerError("Scheduled request has an unsupported phase", request=value, supported=PHASES)
    rt = value.get("remaining_tokens")
    if not (_is_int(rt) and rt > 0):
        raise SchedulerError("Scheduled request requires positive remaining tokens", request=value)
    arr = value.get("arrival")
    if not (arr is None or (_is_int(arr) and arr >= 0)):
        raise SchedulerError("Scheduled request arrival must be a non-negative integer", request=value)
    out = dict(value)
    out["arrival"] = int(arr or 0)
    return out


def _scheduled_tokens(req: dict, available: int, chunk_size: int) -> int:
    """scheduler.clj:37-42: decode work is one token per iteration."""
    return min(int(available), int(req["remaining_tokens"]),
               1 if req["phase"] == "decode" else int(chunk_size))


def plan_iteration(opts: dict, requests) -> dict:
    """One continuous-batching iteration within fixed graph capacities
    (scheduler.clj:44-111).  Decode first (latency), then repair, then prefill,
    each by arrival and identity; ``minimum_prefill_tokens`` reserves that token
    budget and one lane whenever non-decode work waits."""
    max_tokens = opts.get("max_batched_tokens")
    max_seqs = opts.get("max_sequences")
    prefill_chunk = opts.get("prefill_chunk_size", 128)
    repair_chunk = opts.get("repair_chunk_size", 128)
    minimum_prefill = opts.get("minimum_prefill_tokens", 0)
    for field, v in (("max_batched_tokens", max_tokens), ("max_sequences", max_seqs),
                     ("prefill_chunk_size", prefill_chunk), ("repair_chunk_size", repair_chunk)):
        if not (_is_int(v) and v > 0):
            raise SchedulerError("Scheduler capacities must be positive integers", field=field, value=v)
    if not (_is_int(minimum_prefill) and minimum_prefill >= 0):
        raise SchedulerError("Minimum prefill reservation must be a non-negative integer",
                             minimum_prefill_tokens=minimum_prefill)
    ordered = sorted((request(r) for r in requests),
                     key=lambda r: (_PHASE_RANK[r["phase"]], r["arrival"], str(r["id"])))
    nondecode = any(r["phase"] != "decode" for r in ordered)
    reserved_tokens = min(int(minimum_prefill), int(max_tokens)) if nondecode else 0
    reserved_lane = nondecode and reserved_tokens > 0
    token_budget, seq_budget = int(max_tokens), int(max_seqs)
    scheduled, deferred = [], []
    for item in ordered:
        decode = item["phase"] == "decode"
        avail_tokens = max(0, token_budget - reserved_tokens) if decode else token_budget
        avail_seqs = max(0, seq_budget - 1) if (decode and reserved_lane) else seq_budget
        if avail_tokens == 0 or avail_seqs == 0:
            deferred.append(item)
            continue
        chunk = repair_chunk if item["phase"] == "repair" else prefill_chunk
        tokens = _scheduled_tokens(item, avail_tokens, chunk)
        token_budget -= tokens
        seq_budget -= 1
        scheduled.append({**item, "scheduled_tokens": tokens})
    return {"scheduled": scheduled, "deferred": deferred,
            "unused_token_capacity": token_budget, "unused_sequence_capacity": seq_budget}


def advance_request(scheduled: dict):
    """Apply one scheduled item: the next request, or None when complete
    (scheduler.clj:113-124)."""
    tokens = scheduled.get("scheduled_tokens")
    rt = scheduled.get("remaining_tokens")
    if not (_is_int(tokens) and tokens > 0 and tokens <= rt):
        raise SchedulerError("Scheduled token count is outside the request", scheduled=scheduled)
    remaining = rt - tokens
    if remaining <= 0:
        return None
    out = {k: v for k, v in scheduled.items() if k != "scheduled_tokens"}
    out["remaining_tokens"] = remaining
    return out


def _protected(lanes) -> set:
    return {(l.get("continuation_id") if l.get("continuation_id") is not None else l["id"])
            for l in lanes if l is not None}


def _fill_lanes(capacity, previous_lanes, candidates, waiting):
    """Retained occupants keep their physical lane; vacancies take ``waiting`` in order."""
    by_id = {r["id"]: r for r in candidates}
    retained = [({**by_id[p["id"]], "lane_index": i} if p is not None and p["id"] in by_id else None)
                for i, p in enumerate(previous_lanes)]
    retained_ids = {r["id"] for r in retained if r is not None}
    waiting = [r for r in waiting if r["id"] not in retained_ids]
    lanes = list(retained)
    wi = 0
    for i in range(capacity):
        if lanes[i] is None and wi < len(waiting):
            lanes[i] = {**waiting[wi], "lane_index": i}
            wi += 1
    refill = [l for l in lanes if l is not None and l["id"] not in retained_ids]
    lane_ids = {l["id"] for l in lanes if l is not None}
    return {"lanes": lanes, "retained": [r for r in retained if r is not None], "refill": refill,
            "retired": [p for p in previous_lanes if p is not None and p["id"] not in lane_ids],
            "deferred": waiting[wi:], "protected_continuation_ids": _protected(lanes)}


def _padded_lanes(capacity, previous_lanes, what):
    if not (_is_int(capacity) and capacity > 0):
        raise SchedulerError(f"{what} lane capacity must be a positive integer", capacity=capacity)
    prev = list(previous_lanes)
    if len(prev) > capacity:
        raise SchedulerError("Previous lane table exceeds decoder capacity" if what == "Decode"
                             else "Previous lane table exceeds execution capacity",
                             capacity=capacity, lane_count=len(prev))
    return prev + [None] * (capacity - len(prev))


def plan_decode_lanes(capacity: int, previous_lanes, requests) -> dict:
    """Retain and refill fixed decode lanes (scheduler.clj:126-182): running
    decode requests keep their lane; vacancies take waiting requests by arrival
    and identity.  Returns lanes, retained, refill, retired, deferred and the
    continuation ids residency must protect."""
    prev = _padded_lanes(capacity, previous_lanes, "Decode")
    runnable = [r for r in (request(x) for x in requests) if r["phase"] == "decode"]
    waiting = sorted(runnable, key=lambda r: (r["arrival"], str(r["id"])))
    return _fill_lanes(int(capacity), prev, runnable, waiting)


def plan_work_lanes(capacity: int, previous_lanes, scheduled) -> dict:
    """Retain and refill fixed execution lanes for an ordered mixed work set
    (scheduler.clj:184-227); vacancies are filled in input order."""
    prev = _padded_lanes(capacity, previous_lanes, "Work")
    items = [request(x) for x in scheduled]
    ids = [r["id"] for r in items]
    if len(ids) != len(set(ids)):
        raise SchedulerError("Scheduled work identities must be unique", request_ids=ids)
    return _fill_lanes(int(capacity), prev, items, items)


def decode_submission(plan: dict) -> dict:
    """Translate a lane plan into paged-decoder lane work and priming rows
    (scheduler.clj:229-263): only refilled lanes are primed; a retained lane
    keeps the embedding its previous step's tail produced."""
    active = [l for l in plan["lanes"] if l is not None]
    refill_ids = {r["id"] for r in plan["refill"]}
    for item in active:
        if item.get("continuation_id") is None:
            raise SchedulerError("Decode lane requires a continuation identity", request=item)
        pos = item.get("position")
        if not (_is_int(pos) and pos >= 0):
            raise SchedulerError("Decode lane requires a non-negative position", request=item)
        if item["id"] in refill_ids and item.get("pending_token") is None:
            raise SchedulerError("A refilled decode lane requires a pending token", request=item)
    return {"lane_work": [{"lane": l["lane_index"], "continuation_id": l["continuation_id"],
                           "position": l["position"]} for l in active],
            "prime_lanes": [{"lane": l["lane_index"], "token": l["pending_token"]}
                            for l in active if l["id"] in refill_ids],
            "protected_continuation_ids": plan["protected_continuation_ids"]}


def complete_decode_iteration(plan: dict, results, eos_ids=()) -> dict:
    """Apply lane-ordered decoder results (scheduler.clj:265-310): every active
    lane needs exactly one result; budgets fall by one, positions advance by one,
    the token becomes the pending token; exhausted budgets and EOS complete."""
    results = list(results)
    by_lane = {r["lane"]: r for r in results}
    active = {l["lane_index"] for l in plan["lanes"] if l is not None}
    if len(results) != len(by_lane) or active != set(by_lane):
        raise SchedulerError("Decode results do not cover active lanes exactly",
                             active_lanes=active, result_lanes=[r["lane"] for r in results])
    eos = set(eos_ids)
    updated = []
    for item in plan["lanes"]:
        if item is None:
            updated.append(None)
            continue
        tok = by_lane[item["lane_index"]].get("token")
        if not _is_int(tok):
            raise SchedulerError("Decode result requires an integer token", lane=item["lane_index"], token=tok)
        updated.append({**item, "remaining_tokens": item["remaining_tokens"] - 1,
                        "position": item["position"] + 1, "pending_token": tok, "iteration_token": tok})

    def complete(x):
        return x is not None and (x["remaining_tokens"] == 0 or x["iteration_token"] in eos)

    completed = [x for x in updated if complete(x)]
    next_lanes = [None if (x is None or complete(x)) else {k: v for k, v in x.items() if k != "iteration_token"}
                  for x in updated]
    return {"lanes": next_lanes, "runnable": [x for x in next_lanes if x is not None], "completed": completed}


def choose_cache_source(candidates, allow_approximate: bool = False, minimum_quality=1.0):
    """Lowest-latency eligible way to establish a prompt continuation
    (scheduler.clj:312-350): exact sources by default; approximate ones need
    ``allow_approximate`` and quality >= ``minimum_quality``; kind rank breaks
    equal-cost ties."""
    if not (_is_num(minimum_quality) and 0.0 <= float(minimum_quality) <= 1.0):
        raise SchedulerError("Minimum cache-source quality must be in [0,1]", minimum_quality=minimum_quality)
    checked = []
    for c in candidates:
        kind = c.get("kind")
        if kind not in _SOURCE_RANK:
            raise SchedulerError("Unknown cache source kind", candidate=c)
        est = c.get("estimated_ms")
        if not (_is_num(est) and float(est) >= 0.0):
            raise SchedulerError("Cache source requires a non-negative estimate", candidate=c)
        exact = c.get("exact?")
        q = c.get("quality")
        checked.append({**c, "exact?": (kind != "modular-repair") if exact is None else exact,
                        "quality": float(q if q is not None else (0.0 if kind == "modular-repair" else 1.0))})
    eligible = [c for c in checked
                if c["exact?"] or (allow_approximate and c["quality"] >= float(minimum_quality))]
    if not eligible:
        return None
    return sorted(eligible, key=lambda c: (c["estimated_ms"], _SOURCE_RANK[c["kind"]]))[0]


def checkpoint_decision(policy: dict) -> dict:
    """Whether asynchronously checkpointing a continuation has positive value
    (scheduler.clj:352-391): net = reuses * saved - (checkpoint + interference),
    admitted when net >= the safety margin."""
    values = {"expected_reuses": policy.get("expected_reuses"),
              "checkpoint_ms": policy.get("checkpoint_ms"),
              "saved_ms_per_reuse": policy.get("saved_ms_per_reuse"),
              "interference_ms": policy.get("interference_ms", 0.0),
              "minimum_net_benefit_ms": policy.get("minimum_net_benefit_ms", 0.0)}
    for field, v in values.items():
        if not (_is_num(v) and float(v) >= 0.0):
            raise SchedulerError("Checkpoint policy fields must be non-negative numbers",
                                 field=field, value=v, policy=policy)
    reuses, ckpt, saved, interf, margin = (float(values[k]) for k in values)
    gross = reuses * saved
    cost = ckpt + interf
    net = gross - cost
    admit = net >= margin
    return {"admit?": admit, "reason": "positive-expected-value" if admit else "insufficient-expected-reuse",
            "expected_reuses": reuses, "checkpoint_ms": ckpt, "saved_ms_per_reuse": saved,
            "interference_ms": interf, "minimum_net_benefit_ms": margin, "gross_saved_ms": gross,
            "cost_ms": cost, "net_benefit_ms": net,
            "break_even_reuses": (cost / saved) if saved > 0 else None}
