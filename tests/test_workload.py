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
