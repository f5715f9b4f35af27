"""The synthetic continuous-batching planner (``rstr.workload.ChurnPlanner``)
keeps the page pool consistent step after step, with and without retaining
finished continuations as durable routes that admissions evict by value."""
import collections

import pytest

from rstr import configs
from rstr.workload import ChurnPlanner

CFG = configs.MODELS["tiny_llama"]


def _check_pool(pl):
    pool = pl.pool
    refs = collections.Counter()
    for r in pool.routes.values():
        refs.update(r.pages)
    for lease in pool.leases.values():
        refs.update(lease["pages"])
    assert dict(refs) == pool.refcounts
    reserved = [p for e in pool.capacity_reservations.values() for p in e["pages"]]
    assert len(reserved) == len(set(reserved))
    used = set(refs) | set(reserved)
    assert not (used & set(pool.free))
    assert len(used) + len(pool.free) == pool.physical_pages
    for st in pl.lanes:
        if st is not None:
            r = pool.route(st["cid"])
            assert r is not None and r.pending is None
            assert not dict(r.policy).get("durable?")


@pytest.mark.parametrize("retain", [False, True])
def test_planner_keeps_the_pool_consistent(retain):
    pl = ChurnPlanner(CFG, batch=6, page_size=16, physical_pages=160, maxpos=200, seed=11,
                      arrival_mean=1.5, prompt=(8, 60), output=(2, 12), retain_finished=retain)
    for _ in range(80):
        step = pl.plan_step()
        assert 0 < step["active"] <= 6
        _check_pool(pl)
    assert pl.retired > 0
    active = {st["cid"] for st in pl.lanes if st is not None}
    if retain:
        # finished continuations stay resident until an admission needs their pages
        assert pl.evicted > 0
        assert len(pl.pool.routes) > len(active)
    else:
        assert pl.evicted == 0
        assert set(pl.pool.routes) == active


def test_permuted_pages_map_every_page_reference_consistently():
    """``page_perm_seed`` places the pool's pages at a seeded permutation of the
    physical pool: fills, copy-on-write pairs, slots and page-table entries all go
    through the same bijection, so a lane's slot lies in its own mapped page
    table and the recorded steps equal the unpermuted plan mapped page by page."""
    import numpy as np

    kw = dict(batch=6, page_size=16, physical_pages=160, maxpos=200, seed=11, arrival_mean=1.5,
              prompt=(8, 60), output=(2, 12))
    plain = ChurnPlanner(CFG, **kw)
    perm_pl = ChurnPlanner(CFG, **kw, page_perm_seed=1)
    perm = np.random.default_rng(1).permutation(160)
    assert sorted(perm.tolist()) == list(range(160)) and (perm != np.arange(160)).any()
    moved = 0
    for _ in range(40):
        a, b = plain.plan_step(), perm_pl.plan_step()
        assert b["fill_pages"] == [int(perm[p]) for p in a["fill_pages"]]
        assert [tuple(x) for x in b["cow_pairs"]] == [(int(perm[s]), int(perm[d])) for s, d in a["cow_pairs"]]
        pt_a, pt_b = np.asarray(a["page_table"]), np.asarray(b["page_table"])
        assert np.array_equal(pt_b, np.where(pt_a >= 0, perm[np.maximum(pt_a, 0)], -1))
        sa, sb = np.asarray(a["slots"]), np.asarray(b["slots"])
        assert np.array_equal(sb < 0, sa < 0) and np.array_equal(sb % 16, sa % 16)
        assert np.array_equal(sb[sa >= 0] // 16, perm[sa[sa >= 0] // 16])
        for k in ("lengths", "start_positions", "positions", "row_offsets"):
            assert np.array_equal(np.asarray(a[k]), np.asarray(b[k])), k
        for lane in np.nonzero(np.asarray(b["lengths"]) > 0)[0]:
            # the appended row's page is one of the lane's own visible pages
            n = int(b["lengths"][lane])
            assert sb[lane] // 16 == pt_b.reshape(6, -1)[lane, (n - 1) // 16]
        moved += int((pt_b[pt_b >= 0] != pt_a[pt_a >= 0]).sum())
    assert moved > 0


class _FakeDevice:
    """Stands in for the HIP decoder and pool: records every call in stream
    order with the step it precedes (a call made while submitted steps are in
    flight runs after them, as on the session's stream), and checks that at
    most two submitted steps are in flight."""

    def __init__(self, batch):
        self.batch, self.log, self.inflight = batch, [], 0

    def _note(self, *ev):
        self.log.append(ev)

    def fill_synthetic(self, pages, seed):
        self._note("fill", tuple(int(p) for p in pages), int(seed))

    def copy_page(self, src, dst):
        self._note("copy", int(src), int(dst))

    def prime_lanes(self, lanes, tokens):
        self._note("prime", tuple(int(x) for x in lanes), tuple(int(x) for x in tokens))

    def step_lanes(self, **desc):
        import numpy as np
        assert self.inflight == 0
        self._note("step", tuple((k, tuple(np.asarray(v).ravel().tolist())) for k, v in sorted(desc.items())))
        return np.arange(self.batch, dtype=np.int32)

    def step_lanes_submit(self, **desc):
        import numpy as np
        assert self.inflight < 2
        self._note("step", tuple((k, tuple(np.asarray(v).ravel().tolist())) for k, v in sorted(desc.items())))
        self.inflight += 1

    def step_lanes_collect(self):
        import numpy as np
        assert self.inflight > 0
        self.inflight -= 1
        return np.arange(self.batch, dtype=np.int32)

    def step_timing(self):
        return {}


def _effects(log):
    """Per step: the filled pages, copies and primed (lane, token) pairs that
    precede it, then its descriptors."""
    steps, cur = [], {"fill": set(), "copy": [], "prime": set()}
    for ev in log:
        if ev[0] == "fill":
            cur["fill"] |= {(p, ev[2]) for p in ev[1]}
        elif ev[0] == "copy":
            cur["copy"].append(ev[1:])
        elif ev[0] == "prime":
            cur["prime"] |= set(zip(ev[1], ev[2]))
        else:
            steps.append((cur, ev[1]))
            cur = {"fill": set(), "copy": [], "prime": set()}
    return steps


def test_pipelined_live_loop_makes_the_sequential_loops_device_calls():
    """workload.PipelinedLive plans step n+1 while step n is in flight, then
    applies step n+1's fills, copies and primes and submits it before
    collecting step n: per step the device's stream receives the same effects
    and descriptors as from the sequential loop (LiveDevice), with at most two
    steps in flight, through admissions, retirements and value-based
    evictions."""
    from rstr.workload import LiveDevice, PipelinedLive
    kw = dict(batch=6, page_size=16, physical_pages=60, maxpos=192, seed=11, arrival_mean=1.5,
              prompt=(8, 60), output=(2, 12), retain_finished=True)
    n = 40
    seq_dev = _FakeDevice(6)
    seq = ChurnPlanner(CFG, device=LiveDevice(seq_dev, seq_dev), **kw)
    for _ in range(n):
        seq.plan_step()
    pip_dev = _FakeDevice(6)
    pl = ChurnPlanner(CFG, **kw)
    loop = PipelinedLive(pl, pip_dev, pip_dev)
    loop.start()
    for _ in range(n - 1):
        loop.step()
    loop.finish()
    assert pip_dev.inflight == 0 and loop.inflight == 0
    assert pl.retired > 0 and pl.evicted > 0
    a, b = _effects(seq_dev.log), _effects(pip_dev.log)
    assert len(a) == len(b) == n
    for i, ((ea, da), (eb, db)) in enumerate(zip(a, b)):
        assert da == db, i
        assert ea == eb, i


def test_pipelined_live_loop_error_collects_the_running_step():
    """A step whose submission fails surfaces from PipelinedLive.step after the
    step still in flight has been collected: nothing is left in flight on the
    decoder."""
    from rstr.workload import PipelinedLive

    class Failing(_FakeDevice):
        def __init__(self, batch):
            super().__init__(batch)
            self.steps = 0

        def step_lanes_submit(self, **desc):
            self.steps += 1
            if self.steps == 3:
                raise RuntimeError("device step failed")
            super().step_lanes_submit(**desc)
    dev = Failing(6)
    pl = ChurnPlanner(CFG, batch=6, page_size=16, physical_pages=60, maxpos=192, seed=11, arrival_mean=1.5,
                      prompt=(8, 60), output=(2, 12))
    loop = PipelinedLive(pl, dev, dev)
    loop.start()
    with pytest.raises(RuntimeError, match="device step failed"):
        for _ in range(10):
            loop.step()
    assert loop.inflight == 0 and dev.inflight == 0
    assert dev.steps == 3