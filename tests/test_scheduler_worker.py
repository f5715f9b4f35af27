"""Known-answer tests of the continuous-batching planner and worker loop, one per
reference test in ``test/pretrained/continuation_scheduler_test.clj`` and
``test/pretrained/continuation_worker_test.clj``.  The worker tests use a
recording decoder in place of the reference's ``with-redefs`` of
``paged-decoder/prime-lanes!`` / ``step-lanes!`` / ``prime-prompts-batch!``.
"""
import pytest

from rstr import scheduler, worker
from rstr.scheduler import SchedulerError


def R(**kw):
    return kw


# ---- scheduler (continuation_scheduler_test.clj) ----------------------------
def test_decode_work_precedes_bounded_prefill():
    """:5-24."""
    reqs = [scheduler.request(R(id="long-prompt", phase="prefill", remaining_tokens=500, arrival=0)),
            scheduler.request(R(id="decode-b", phase="decode", remaining_tokens=1, arrival=2)),
            scheduler.request(R(id="decode-a", phase="decode", remaining_tokens=1, arrival=1))]
    plan = scheduler.plan_iteration({"max_batched_tokens": 66, "max_sequences": 3, "prefill_chunk_size": 64}, reqs)
    assert [r["id"] for r in plan["scheduled"]] == ["decode-a", "decode-b", "long-prompt"]
    assert [r["scheduled_tokens"] for r in plan["scheduled"]] == [1, 1, 64]
    assert plan["unused_token_capacity"] == 0
    assert plan["deferred"] == []


def test_iteration_capacity_defers_without_mutating_requests():
    """:26-35."""
    reqs = [R(id="a", phase="decode", remaining_tokens=4, arrival=0),
            R(id="b", phase="decode", remaining_tokens=2, arrival=1)]
    plan = scheduler.plan_iteration({"max_batched_tokens": 1, "max_sequences": 1}, reqs)
    assert [r["id"] for r in plan["scheduled"]] == ["a"]
    assert [r["id"] for r in plan["deferred"]] == ["b"]
    assert scheduler.advance_request(plan["scheduled"][0])["remaining_tokens"] == 3
    assert reqs[0]["remaining_tokens"] == 4


def test_optional_prefill_reservation_prevents_starvation():
    """:37-51."""
    reqs = [R(id=i, phase="decode", remaining_tokens=8) for i in range(4)]
    reqs.append(R(id="waiting-prefill", phase="prefill", remaining_tokens=100))
    plan = scheduler.plan_iteration({"max_batched_tokens": 4, "max_sequences": 4, "minimum_prefill_tokens": 1,
                                     "prefill_chunk_size": 16}, reqs)
    assert [r["id"] for r in plan["scheduled"]] == [0, 1, 2, "waiting-prefill"]
    assert [r["scheduled_tokens"] for r in plan["scheduled"]] == [1, 1, 1, 1]
    assert [r["id"] for r in plan["deferred"]] == [3]


def test_exact_cache_source_is_default_and_approximation_is_explicit():
    """:53-67."""
    cands = [R(kind="recompute-exact", estimated_ms=12.0), R(kind="restore-exact", estimated_ms=8.0),
             R(kind="modular-repair", estimated_ms=3.0, quality=0.97)]
    assert scheduler.choose_cache_source(cands)["kind"] == "restore-exact"
    assert scheduler.choose_cache_source(cands, allow_approximate=True, minimum_quality=0.95)["kind"] == "modular-repair"
    assert scheduler.choose_cache_source(cands, allow_approximate=True, minimum_quality=0.99)["kind"] == "restore-exact"


def test_checkpoint_admission_requires_positive_measured_value():
    """:69-83."""
    base = {"checkpoint_ms": 188.0, "saved_ms_per_reuse": 118.0, "interference_ms": 1.0}
    rejected = scheduler.checkpoint_decision({**base, "expected_reuses": 1.0})
    admitted = scheduler.checkpoint_decision({**base, "expected_reuses": 2.0})
    assert rejected["admit?"] is False and rejected["reason"] == "insufficient-expected-reuse"
    assert admitted["admit?"] is True and admitted["reason"] == "positive-expected-value"
    assert admitted["break_even_reuses"] == 189.0 / 118.0
    assert admitted["net_benefit_ms"] == 47.0


def test_decode_lanes_retain_resident_work_and_refill_only_vacancies():
    """:85-107."""
    left = R(id="left", continuation_id="left-kv", phase="decode", remaining_tokens=4, position=8,
             pending_token=101, arrival=0)
    finished = R(id="finished", continuation_id="finished-kv", phase="decode", remaining_tokens=1, position=5,
                 pending_token=102, arrival=1)
    incoming = R(id="incoming", continuation_id="incoming-kv", phase="decode", remaining_tokens=3, position=2,
                 pending_token=103, arrival=2)
    plan = scheduler.plan_decode_lanes(3, [left, finished, None], [incoming, left])
    sub = scheduler.decode_submission(plan)
    assert [l and l["id"] for l in plan["lanes"]] == ["left", "incoming", None]
    assert [r["id"] for r in plan["retained"]] == ["left"]
    assert [r["id"] for r in plan["refill"]] == ["incoming"]
    assert [r["id"] for r in plan["retired"]] == ["finished"]
    assert plan["protected_continuation_ids"] == {"left-kv", "incoming-kv"}
    assert sub["lane_work"] == [{"lane": 0, "continuation_id": "left-kv", "position": 8},
                                {"lane": 1, "continuation_id": "incoming-kv", "position": 2}]
    # the retained lane keeps the embedding produced by the prior tail
    assert sub["prime_lanes"] == [{"lane": 1, "token": 103}]


def test_decode_lane_overflow_is_deferred_with_stable_priority():
    """:109-116."""
    reqs = [R(id="later", phase="decode", remaining_tokens=1, arrival=2),
            R(id="first", phase="decode", remaining_tokens=1, arrival=0),
            R(id="middle", phase="decode", remaining_tokens=1, arrival=1)]
    plan = scheduler.plan_decode_lanes(2, [], reqs)
    assert [l["id"] for l in plan["lanes"]] == ["first", "middle"]
    assert [r["id"] for r in plan["deferred"]] == ["later"]


def test_mixed_work_lanes_follow_iteration_order_with_stable_refill():
    """:118-131."""
    decode = R(id="decode", continuation_id="decode-kv", phase="decode", remaining_tokens=4)
    old_prefill = R(id="old-prefill", continuation_id="old-kv", phase="prefill", remaining_tokens=8)
    prefill = R(id="prefill", continuation_id="prefill-kv", phase="prefill", remaining_tokens=7)
    plan = scheduler.plan_work_lanes(3, [decode, old_prefill, None], [prefill, decode])
    assert [l and l["id"] for l in plan["lanes"]] == ["decode", "prefill", None]
    assert [r["id"] for r in plan["retained"]] == ["decode"]
    assert [r["id"] for r in plan["refill"]] == ["prefill"]
    assert [r["id"] for r in plan["retired"]] == ["old-prefill"]
    assert plan["protected_continuation_ids"] == {"decode-kv", "prefill-kv"}


def test_decode_results_retire_eos_and_preserve_next_token_state():
    """:133-142."""
    reqs = [R(id="keep", continuation_id="keep-kv", phase="decode", remaining_tokens=3, position=7, pending_token=10),
            R(id="stop", continuation_id="stop-kv", phase="decode", remaining_tokens=3, position=4, pending_token=11)]
    plan = scheduler.plan_decode_lanes(3, [], reqs)
    res = scheduler.complete_decode_iteration(plan, [{"lane": 0, "token": 20}, {"lane": 1, "token": 99}], {99})
    assert [l and l["id"] for l in res["lanes"]] == ["keep", None, None]
    assert res["lanes"][0]["position"] == 8
    assert res["lanes"][0]["pending_token"] == 20
    assert res["lanes"][0]["remaining_tokens"] == 2
    assert [r["id"] for r in res["runnable"]] == ["keep"]
    assert [r["id"] for r in res["completed"]] == ["stop"]
    assert res["completed"][0]["iteration_token"] == 99


@pytest.mark.parametrize("bad,msg", [
    (R(phase="decode", remaining_tokens=1), "requires :request/id"),
    (R(id=1, phase="sample", remaining_tokens=1), "unsupported phase"),
    (R(id=1, phase="decode", remaining_tokens=0), "positive remaining tokens"),
    (R(id=1, phase="decode", remaining_tokens=1, arrival=-1), "non-negative integer"),
])
def test_request_validation(bad, msg):
    with pytest.raises(SchedulerError, match=msg):
        scheduler.request(bad)


def test_results_must_cover_active_lanes_exactly():
    plan = scheduler.plan_decode_lanes(2, [], [R(id="a", continuation_id="a", phase="decode", remaining_tokens=2,
                                                 position=0, pending_token=1)])
    with pytest.raises(SchedulerError, match="cover active lanes"):
        scheduler.complete_decode_iteration(plan, [])


# ---- worker (continuation_worker_test.clj) ----------------------------------
class RecordingDecoder:
    def __init__(self, batch_size, step_results=None, emitted=None):
        self.batch_size = batch_size
        self.calls = []
        self.step_results = step_results
        self.emitted = list(emitted or [])

    def prime_lanes(self, rows):
        self.calls.append(("prime", list(rows)))

    def prime_prompts_batch(self, cids, prompts):
        self.calls.append(("prompts", list(cids), [list(p) for p in prompts]))

    def step_lanes(self, lane_work):
        self.calls.append(("step", [dict(w) for w in lane_work]))
        if self.step_results is not None:
            return self.step_results
        toks = self.emitted.pop(0)
        return [{**w, "token": t} for w, t in zip(lane_work, toks)]


def decode_request(rid, token, position, remaining, arrival):
    return R(id=rid, continuation_id=f"{rid}-kv", phase="decode", remaining_tokens=remaining,
             pending_token=token, position=position, arrival=arrival)


def test_worker_retains_refills_executes_and_retires_lanes():
    """continuation_worker_test.clj:16-45."""
    retained = decode_request("retained", 10, 7, 3, 0)
    departed = decode_request("departed", 11, 4, 2, 1)
    incoming = decode_request("incoming", 12, 2, 4, 2)
    dec = RecordingDecoder(3, step_results=[
        {"lane": 0, "continuation_id": "retained-kv", "position": 7, "token": 20},
        {"lane": 1, "continuation_id": "incoming-kv", "position": 2, "token": 99}])
    it = worker.run_decode_iteration(dec, [retained, departed, None], [incoming, retained], eos_ids={99})
    assert dec.calls == [("prime", [{"lane": 1, "token": 12}]),
                         ("step", [{"lane": 0, "continuation_id": "retained-kv", "position": 7},
                                   {"lane": 1, "continuation_id": "incoming-kv", "position": 2}])]
    assert [l and l["id"] for l in it["lanes"]] == ["retained", None, None]
    assert [r["id"] for r in it["completed"]] == ["incoming"]
    assert [r["id"] for r in it["retired"]] == ["departed"]
    assert it["protected_continuation_ids"] == {"retained-kv", "incoming-kv"}
    assert it["next_protected_continuation_ids"] == {"retained-kv"}
    assert [r["token"] for r in it["results"]] == [20, 99]


def test_empty_worker_iteration_submits_no_device_work():
    """:47-55."""
    dec = RecordingDecoder(2)
    it = worker.run_decode_iteration(dec, [], [])
    assert dec.calls == []
    assert it["lanes"] == [None, None]
    assert it["results"] == []


def test_next_ready_boundary_keeps_policy_coordination_explicit():
    """:57-62."""
    it = {"runnable": [decode_request("running", 1, 1, 2, 0)], "deferred": [decode_request("waiting", 2, 2, 3, 1)]}
    arrivals = [decode_request("new", 3, 0, 4, 2)]
    assert [r["id"] for r in worker.next_ready_requests(it, arrivals)] == ["running", "waiting", "new"]


def test_continuous_generation_retires_eos_lanes_without_stopping_the_batch():
    """:64-88."""
    dec = RecordingDecoder(2, emitted=[[10, 99], [11], [12]])
    out = worker.generate_continuously(dec, ["left", "right"], [[1, 2], [3, 4]], 3, eos_ids={99})
    assert out == [[10, 11, 12], [99]]
    assert dec.calls == [("prompts", ["left", "right"], [[1, 2], [3, 4]]),
                         ("step", [{"lane": 0, "continuation_id": "left", "position": 1},
                                   {"lane": 1, "continuation_id": "right", "position": 1}]),
                         ("step", [{"lane": 0, "continuation_id": "left", "position": 2}]),
                         ("step", [{"lane": 0, "continuation_id": "left", "position": 3}])]
