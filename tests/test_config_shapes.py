"""BASELINE.json configs[1], [2] and [4] at their real shapes as parity cases: the
bench's host-planned schedules replayed on the HIP decoder (fills, copy-on-write
copies, primes, one step graph per step) and on the oracle, token for token.

- config2: Gemma-3-270M-shaped Q4 (18 layers, sliding window 512), 16 lanes,
  contexts U[64, 2048], route pages at a seeded permutation of the physical pool
  (seed 1, as the bench runs it), attention split 32 (the bench's split).
- config3: Qwen3-0.6B-shaped Q4 (28 layers, qk-norm), 64 lanes, contexts
  log-uniform [256, 8192], lanes 0-31 forking one 1024-token prefix with
  copy-on-write on their first divergent append (attention split 640, the
  bench's split).
- config5: Llama-3-8B-shaped Q4 (32 layers), 128 lanes with churn (prompts capped
  at 1024 tokens to bound the oracle's host KV memory), and a few lanes at the
  bench's full prompt range (contexts of 3500-4096 tokens through all 32 layers)."""
import numpy as np
import pytest

import oracle as O
from rstr import configs, hip, workload
from test_gpu_schedule import _replay_oracle

pytestmark = pytest.mark.gpu


def _replay(cfg, planner, batch, pages, maxpos, split, n_steps):
    pps = -(-maxpos // 16)
    steps = [planner.plan_step() for _ in range(n_steps)]
    om = O.Model(cfg, seed=1)
    od = O.Decoder(om, batch, 16, pages, pps, maxpos, kv_f16=True, split=split)
    try:
        want = _replay_oracle(od, steps)
    finally:
        od.close()
        om.close()
    with hip.Session(0) as sess:
        m = hip.Model(sess, cfg, seed=1)
        p = hip.Pool(m, 16, pages)
        d = hip.Decoder(m, p, batch, pps, maxpos, split)
        d.schedule_upload(steps)
        got, _ = d.schedule_run(0, n_steps)
    for i, st in enumerate(steps):
        act = np.asarray(st["lengths"]) > 0
        assert act.any()
        assert np.array_equal(got[i][act], want[i][act]), i
    return steps


def test_config2_shape_schedule_matches_oracle():
    print("case config2 shape", flush=True)
    cfg = configs.GEMMA3_270M
    batch, maxpos = 16, 2048 + 64
    pages = 16 * (maxpos // 16 + 1) + 64
    pl = workload.ChurnPlanner(cfg, batch, 16, pages, maxpos, seed=1, arrival_mean=0.0,
                               prompt=(64, 2048), output=(256, 256), page_perm_seed=1)
    steps = _replay(cfg, pl, batch, pages, maxpos, 32, 3)
    assert max(max(st["lengths"]) for st in steps) > 512  # windowed layers see a partial window
    # route pages are scattered over the physical pool, not lowest-first runs
    pt = np.asarray(steps[-1]["page_table"]).reshape(batch, -1)
    first = pt[:, 0][pt[:, 0] >= 0]
    assert len(set(first.tolist())) == len(first) and first.max() > pages // 2


def test_config3_shape_schedule_matches_oracle():
    print("case config3 shape", flush=True)
    cfg = configs.QWEN3_06B
    batch, maxpos = 64, 8192 + 64
    pages = 9000
    pl = workload.SharedPrefixPlanner(cfg, batch, 16, pages, maxpos, seed=2)
    _replay(cfg, pl, batch, pages, maxpos, 640, 2)
    assert pl.cow_pages > 0


def test_config5_shape_one_step_matches_oracle():
    """The north-star shape (Llama-3-8B Q4, all 32 layers and the 128 256-token
    head) at 128 ragged lanes: the first two planned steps (admission fills, primes,
    one decode step each) give the oracle's tokens in every lane.  Prompts are
    drawn from U[128, 1024] instead of the bench's U[128, 4096] to bound the
    oracle's host KV memory."""
    print("case config5 shape", flush=True)
    cfg = configs.LLAMA3_8B
    batch, maxpos = 128, 1024 + 64
    pages = 128 * (maxpos // 16 + 1)
    pl = workload.ChurnPlanner(cfg, batch, 16, pages, maxpos, seed=5, arrival_mean=4.0,
                               prompt=(128, 1024), output=(32, 64))
    steps = _replay(cfg, pl, batch, pages, maxpos, 256, 2)
    assert all(st["active"] == batch for st in steps)


def test_config5_shape_full_context_lanes_match_oracle():
    """The north-star model with lanes at the bench's full prompt range: 8 lanes
    whose prompts are drawn from U[3500, 4096] (restored prefixes of 3499-4095
    rows), all 32 layers and the head, two planned steps, every lane's tokens
    equal to the oracle's.  Attention runs the many-item split kernel (17 splits of
    256 tokens per lane and kv head)."""
    print("case config5 full context", flush=True)
    cfg = configs.LLAMA3_8B
    batch, maxpos = 8, 4096 + 64
    pages = batch * (maxpos // 16 + 1)
    pl = workload.ChurnPlanner(cfg, batch, 16, pages, maxpos, seed=5, arrival_mean=0.0,
                               prompt=(3500, 4096), output=(32, 64))
    steps = _replay(cfg, pl, batch, pages, maxpos, 256, 2)
    assert all(st["active"] == batch for st in steps)
    assert min(min(st["lengths"]) for st in steps) >= 3500


def test_config5_1lane_shape_matches_oracle():
    """The one-lane end of config5 as the bench runs it: the Llama-3-8B-shaped
    model with one lane (all 32 layers and the head), attention split 64, a
    restored prefix drawn from U[3500, 4096]; two planned steps, tokens equal to
    the oracle's.  At one row every projection streams its weights through a GEMV
    and the down projection computes the gated activation in its staging."""
    print("case config5 one lane", flush=True)
    cfg = configs.LLAMA3_8B
    batch, maxpos = 1, 4096 + 64
    pages = maxpos // 16 + 8
    pl = workload.ChurnPlanner(cfg, batch, 16, pages, maxpos, seed=5, arrival_mean=0.0,
                               prompt=(3500, 4096), output=(32, 64))
    steps = _replay(cfg, pl, batch, pages, maxpos, 64, 2)
    assert all(st["active"] == batch for st in steps)
