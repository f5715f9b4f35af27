"""BASELINE.json configs[1], [2] and [4] at their real shapes as parity cases: the
bench's host-planned schedules replayed on the HIP decoder (fills, copy-on-write
copies, primes, one step graph per step) and on the oracle, token for token.

- config2: Gemma-3-270M-shaped Q4 (18 layers, sliding window 512), 16 lanes,
  contexts U[64, 2048] admitted onto a permuted page pool (attention split 64).
- config3: Qwen3-0.6B-shaped Q4 (28 layers, qk-norm), 64 lanes, contexts
  log-uniform [256, 8192], lanes 0-31 forking one 1024-token prefix with
  copy-on-write on their first divergent append (attention split 128).
- config5: Llama-3-8B-shaped Q4 (32 layers), 128 lanes with churn (prompts capped
  at 1024 tokens to bound the oracle's host KV memory)."""
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
                               prompt=(64, 2048), output=(256, 256))
    steps = _replay(cfg, pl, batch, pages, maxpos, 64, 3)
    assert max(max(st["lengths"]) for st in steps) > 512  # windowed layers see a partial window


def test_config3_shape_schedule_matches_oracle():
    print("case config3 shape", flush=True)
    cfg = configs.QWEN3_06B
    batch, maxpos = 64, 8192 + 64
    pages = 9000
    pl = workload.SharedPrefixPlanner(cfg, batch, 16, pages, maxpos, seed=2)
    _replay(cfg, pl, batch, pages, maxpos, 128, 2)
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
