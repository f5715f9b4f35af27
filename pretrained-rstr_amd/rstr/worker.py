"""Worker-local continuous decode loop: the host mirror of
``src/pretrained/continuation/worker.clj``.  It joins the pure scheduler to a
paged decoder (``rstr.paged_decoder.PagedDecoder`` or any object with
``batch_size``, ``prime_lanes``, ``step_lanes`` and ``prime_prompts_batch``).
"""
from __future__ import annotations

from . import scheduler


def _capacity(decoder) -> int:
    return int(getattr(decoder, "batch_size", 1) or 1)


def run_decode_iteration(decoder, previous_lanes, requests, eos_ids=()) -> dict:
    """Plan and execute one continuous decode iteration (worker.clj:12-56):
    retain/refill lanes, prime only refilled lanes, step, apply the results.
    No device work is submitted when no lane is active."""
    plan = scheduler.plan_decode_lanes(_capacity(decoder), previous_lanes, requests)
    sub = scheduler.decode_submission(plan)
    results = []
    if sub["lane_work"]:
        if sub["prime_lanes"]:
            decoder.prime_lanes(sub["prime_lanes"])
        results = decoder.step_lanes(sub["lane_work"])
    done = scheduler.complete_decode_iteration(plan, results, eos_ids)
    return {"lanes": done["lanes"], "runnable": done["runnable"], "completed": done["completed"],
            "deferred": plan["deferred"], "results": results, "retained": plan["retained"],
            "refilled": plan["refill"], "retired": plan["retired"],
            "protected_continuation_ids": sub["protected_continuation_ids"],
            "next_protected_continuation_ids": scheduler._protected(done["lanes"])}


def next_ready_requests(iteration: dict, new_arrivals=()) -> list:
    """Retained runnable work, then deferred ready work, then new arrivals
    (worker.clj:58-66)."""
    return list(iteration.get("runnable", ())) + list(iteration.get("deferred", ())) + list(new_arrivals)


def generate_continuously(decoder, continuation_ids, prompts, max_new: int, eos_ids=()) -> list:
    """Independently retiring greedy sequences through the worker loop
    (worker.clj:68-111).  The prompts fill the fixed batch; each lane stops on
    an EOS id (kept in its output) or after ``max_new`` tokens."""
    if isinstance(max_new, bool) or not isinstance(max_new, int) or max_new < 0:
        raise scheduler.SchedulerError("Maximum generated tokens must be a non-negative integer", max_new=max_new)
    cids = list(continuation_ids)
    prompts = [list(p) for p in prompts]
    cap = _capacity(decoder)
    if not (cap == len(cids) == len(prompts)):
        raise scheduler.SchedulerError("Continuous generation must fill the fixed decode batch",
                                       batch_size=cap, continuation_count=len(cids), prompt_count=len(prompts))
    decoder.prime_prompts_batch(cids, prompts)
    if max_new == 0:
        return [[] for _ in range(cap)]
    initial = [{"id": c, "continuation_id": c, "phase": "decode", "remaining_tokens": max_new,
                "pending_token": p[-1], "position": len(p) - 1, "arrival": lane}
               for lane, (c, p) in enumerate(zip(cids, prompts))]
    out_index = {c: i for i, c in enumerate(cids)}
    lanes, ready = initial, initial
    output = [[] for _ in range(cap)]
    while ready:
        it = run_decode_iteration(decoder, lanes, ready, eos_ids)
        for r in it["results"]:
            output[out_index[r["continuation_id"]]].append(r["token"])
        lanes, ready = it["lanes"], next_ready_requests(it, [])
    return output
