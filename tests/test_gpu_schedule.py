"""The bench's timed path: host-planned step schedules uploaded once
(``rstr_schedule_upload``) and replayed on the device (``rstr_schedule_run``:
synthetic prefix fills, copy-on-write page copies, lane primes, one step graph
per step) against the oracle replaying the same recorded steps in the same
order, token for token.  Covers continuous churn (with value-based retention of
finished routes) and forked shared prefixes with copy-on-write."""
import numpy as np
import pytest

import oracle as O
from rstr import configs, hip, workload

CFG = configs.MODELS["tiny_llama"]


def _replay_oracle(od, steps):
    out = []
    for st in steps:
        for pg in st["fill_pages"]:
            od.fill_synthetic(int(pg), int(st["fill_seed"]))
        for src, dst in st["cow_pairs"]:
            od.copy_page(int(src), int(dst))
        if st["prime_lanes"]:
            od.prime_lanes(st["prime_lanes"], st["prime_tokens"])
        out.append(od.step_lanes(st["slots"], st["row_offsets"], st["positions"], st["page_table"],
                                 st["lengths"], st["start_positions"]))
    return np.array(out)


def _check(planner_factory, batch, pages, maxpos, split, n_steps):
    pps = -(-maxpos // 16)
    pl = planner_factory(pages, pps)
    steps = [pl.plan_step() for _ in range(n_steps)]
    om = O.Model(CFG, seed=3)
    od = O.Decoder(om, batch, 16, pages, pps, maxpos, kv_f16=True, split=split)
    try:
        want = _replay_oracle(od, steps)
    finally:
        od.close()
        om.close()
    with hip.Session(0) as sess:
        m = hip.Model(sess, CFG, seed=3)
        p = hip.Pool(m, 16, pages)
        d = hip.Decoder(m, p, batch, pps, maxpos, split)
        d.schedule_upload(steps)
        got, _ = d.schedule_run(0, n_steps)
    for i, st in enumerate(steps):
        act = np.asarray(st["lengths"]) > 0
        assert np.array_equal(got[i][act], want[i][act]), (i, got[i], want[i])
    return pl


@pytest.mark.gpu
def test_schedule_replay_with_churn_matches_oracle():
    print("case schedule churn", flush=True)
    batch, pages, maxpos = 6, 60, 192

    def make(pages, pps):
        return workload.ChurnPlanner(CFG, batch, 16, pages, maxpos, seed=11, arrival_mean=1.5,
                                     prompt=(8, 60), output=(2, 12), retain_finished=True)
    pl = _check(make, batch, pages, maxpos, 16, 40)
    assert pl.retired > 0 and pl.evicted > 0


@pytest.mark.gpu
def test_schedule_replay_with_shared_prefix_forks_matches_oracle():
    print("case schedule shared prefix", flush=True)
    batch, pages, maxpos = 6, 200, 400

    def make(pages, pps):
        return workload.SharedPrefixPlanner(CFG, batch, 16, pages, maxpos, seed=2, ctx=(20, 200),
                                            shared_lanes=3, prefix=64)
    pl = _check(make, batch, pages, maxpos, 32, 12)
    assert pl.cow_pages > 0


@pytest.mark.gpu
def test_pipelined_live_loop_matches_sequential_loop_and_oracle():
    """The live loop with the control plane one step ahead (PipelinedLive: step
    n submitted with rstr_step_lanes_submit, step n+1 planned while it runs,
    its fills and primes applied and step n+1 submitted before step n's tokens
    are collected) gives the tokens of the sequential live loop (LiveDevice:
    every call made as the planner makes it) on the same decoder, step for
    step, through admissions, retirements and value-based evictions; and the
    oracle replaying the pipelined loop's recorded steps agrees."""
    print("case pipelined live loop", flush=True)
    batch, pages, maxpos, split, n = 6, 60, 192, 16, 30
    pps = -(-maxpos // 16)

    def make(device=None):
        return workload.ChurnPlanner(CFG, batch, 16, pages, maxpos, seed=11, arrival_mean=1.5,
                                     prompt=(8, 60), output=(2, 12), retain_finished=True, device=device)
    with hip.Session(0) as sess:
        m = hip.Model(sess, CFG, seed=3)
        p = hip.Pool(m, 16, pages)
        d = hip.Decoder(m, p, batch, pps, maxpos, split)
        dev = workload.LiveDevice(d, p)
        seq_pl = make(dev)
        seq = []
        for _ in range(n):
            seq_pl.plan_step()
            seq.append(np.array(dev.download_tokens()))
        pl = make()
        loop = workload.PipelinedLive(pl, d, p)
        steps = [loop.start()]
        piped = []
        for _ in range(n - 1):
            tok, st = loop.step()
            piped.append(np.array(tok))
            steps.append(st)
        piped.append(np.array(loop.finish()))
    assert pl.retired > 0 and pl.evicted > 0
    om = O.Model(CFG, seed=3)
    od = O.Decoder(om, batch, 16, pages, pps, maxpos, kv_f16=True, split=split)
    try:
        want = _replay_oracle(od, steps)
    finally:
        od.close()
        om.close()
    for i, st in enumerate(steps):
        act = np.asarray(st["lengths"]) > 0
        assert act.any()
        assert np.array_equal(piped[i][act], seq[i][act]), (i, piped[i], seq[i])
        assert np.array_equal(piped[i][act], want[i][act]), (i, piped[i], want[i])


@pytest.mark.gpu
def test_schedule_replay_single_split_direct_output_matches_oracle():
    """Lanes whose visible range is one attention split (maxpos <= split) on a
    head dimension the few-item kernel serves (the tiny Qwen shape, 128): the
    split kernel writes the quantised attention output itself and the step has
    no merge launch.  Continuous churn (lanes retire, idle and refill) replayed
    against the oracle at the same split, token for token."""
    print("case schedule single split", flush=True)
    cfg = configs.MODELS["tiny_qwen"]
    batch, pages, maxpos, split, n_steps = 6, 60, 192, 256, 40
    pps = -(-maxpos // 16)
    pl = workload.ChurnPlanner(cfg, batch, 16, pages, maxpos, seed=11, arrival_mean=1.5,
                               prompt=(8, 60), output=(2, 12), retain_finished=True)
    steps = [pl.plan_step() for _ in range(n_steps)]
    assert pl.retired > 0
    om = O.Model(cfg, seed=3)
    od = O.Decoder(om, batch, 16, pages, pps, maxpos, kv_f16=True, split=split)
    try:
        want = _replay_oracle(od, steps)
    finally:
        od.close()
        om.close()
    with hip.Session(0) as sess:
        m = hip.Model(sess, cfg, seed=3)
        p = hip.Pool(m, 16, pages)
        d = hip.Decoder(m, p, batch, pps, maxpos, split)
        d.schedule_upload(steps)
        got, _ = d.schedule_run(0, n_steps)
    for i, st in enumerate(steps):
        act = np.asarray(st["lengths"]) > 0
        assert np.array_equal(got[i][act], want[i][act]), (i, got[i], want[i])


def _lane_desc(lengths, pps, ps=16):
    """Descriptors of lanes whose routes hold pages b*pps .. b*pps+pps-1, every
    active lane appending its last token."""
    B = len(lengths)
    pt = np.full((B, pps), -1, np.int32)
    slots = np.full(B, -1, np.int32)
    pos = np.zeros(B, np.int32)
    for b, L in enumerate(lengths):
        if L:
            pt[b, :-(-L // ps)] = b * pps + np.arange(-(-L // ps))
            slots[b] = pt[b, (L - 1) // ps] * ps + (L - 1) % ps
            pos[b] = L - 1
    return dict(slots=slots, row_offsets=np.arange(B + 1, dtype=np.int32), positions=pos,
                page_table=pt.ravel(), lengths=np.asarray(lengths, np.int32),
                start_positions=np.zeros(B, np.int32))


@pytest.mark.gpu
@pytest.mark.parametrize("graph", [True, False])
def test_submitted_steps_equal_synchronous_steps(graph):
    """rstr_step_lanes_submit / _collect: two steps in flight, a prime and a
    page copy issued between submissions (they run after the submitted steps in
    stream order), then the tokens collected in submission order, equal the
    synchronous rstr_step_lanes sequence on a twin decoder, tokens and resident
    rows; a third submission and a collection with nothing in flight fail with
    a state error and leave the decoder usable."""
    print(f"case submitted steps graph={graph}", flush=True)
    batch, pps, maxpos, split = 3, 4, 64, 16
    steps = [[5, 9, 0], [6, 10, 0], [7, 11, 3]]
    with hip.Session(0) as sess:
        m = hip.Model(sess, CFG, seed=3)
        twins = []
        for _ in range(2):
            p = hip.Pool(m, 16, batch * pps)
            p.fill_synthetic(np.arange(batch * pps, dtype=np.int32), 5)
            d = hip.Decoder(m, p, batch, pps, maxpos, split)
            d.set_graph(graph)
            twins.append((p, d))
        (p1, d1), (p2, d2) = twins
        for p, d in twins:
            d.prime_lanes([0, 1], [3, 17])
        sync = []
        for i, L in enumerate(steps):
            if i == 2:
                d1.prime_lanes([2], [29])
                p1.copy_page(1, 2 * pps)
            sync.append(d1.step_lanes(**_lane_desc(L, pps)))
        d2.step_lanes_submit(**_lane_desc(steps[0], pps))
        d2.step_lanes_submit(**_lane_desc(steps[1], pps))
        with pytest.raises(hip.RstrError, match="in flight"):
            d2.step_lanes_submit(**_lane_desc(steps[2], pps))
        got = [d2.step_lanes_collect()]
        d2.prime_lanes([2], [29])
        p2.copy_page(1, 2 * pps)
        d2.step_lanes_submit(**_lane_desc(steps[2], pps))
        got += [d2.step_lanes_collect(), d2.step_lanes_collect()]
        with pytest.raises(hip.RstrError, match="no submitted step"):
            d2.step_lanes_collect()
        for i in range(3):
            assert np.array_equal(got[i], sync[i]), (i, got[i], sync[i])
        assert np.array_equal(d2.rows(), d1.rows())
