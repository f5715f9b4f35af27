"""The worker loop (``rstr.worker``) driving real decoders: continuous generation
with independently retiring lanes goes through the page-pool mirror, the
paged-decoder mirror and a step device -- the CPU oracle decoder, or the HIP
decoder through the C ABI.

- CPU: a lane's tokens in a continuously batched run equal its tokens when it
  is generated alone (retiring neighbours never disturb a lane).
- GPU: the HIP run equals the oracle run token for token.
"""
import numpy as np
import pytest

import oracle as O
from rstr import configs, hip, worker
from rstr.page_pool import PagePool
from rstr.paged_decoder import HipStepDevice, PagedDecoder

CFG = configs.MODELS["tiny_llama"]
PS, PAGES, MAXPOS, SPLIT, SEED = 16, 64, 96, 16, 5
PPS = MAXPOS // PS
PROMPTS = [[5, 9, 14, 3, 22], [7, 1, 2, 8, 30], [4, 4, 6, 10, 11]]
MAX_NEW = 7


class OracleStepDevice:
    """The three-call step protocol over the oracle decoder."""

    def __init__(self, od):
        self.od, self._desc, self._tok = od, None, None

    def upload(self, desc):
        self._desc = desc

    def run(self):
        self._tok = self.od.step_lanes(**self._desc)

    def download_tokens(self):
        return self._tok

    def prime_rows(self, lane_tokens):
        if lane_tokens:
            self.od.prime_lanes([lt["lane"] for lt in lane_tokens], [lt["token"] for lt in lane_tokens])


def _oracle_run(prompts, eos, batch):
    om = O.Model(CFG, seed=SEED)
    od = O.Decoder(om, batch, PS, PAGES, PPS, MAXPOS, kv_f16=True, split=SPLIT)
    try:
        pool = PagePool(PS, PAGES, CFG["n_layers"], CFG["n_kv"], CFG["head_dim"], device=od)
        dec = PagedDecoder(pool, OracleStepDevice(od), batch_size=batch, maxpos=MAXPOS, pages_per_sequence=PPS)
        return worker.generate_continuously(dec, [f"c{i}" for i in range(batch)], prompts, MAX_NEW, eos_ids=eos)
    finally:
        od.close()
        om.close()


def _eos_retiring_a_lane_early():
    """An EOS id that exactly one lane emits before its last token and no other
    lane ever emits (so lanes retire at different steps): (eos, lane, free run)."""
    free = _oracle_run(PROMPTS, (), 3)
    for lane in range(3):
        for k in range(MAX_NEW - 1):
            cand = free[lane][k]
            if cand not in free[lane][:k] and all(cand not in free[o] for o in range(3) if o != lane):
                return cand, lane, free
    pytest.skip("no lane-separating EOS candidate in this seeded run")


def test_continuous_generation_equals_lanes_generated_alone():
    eos, early, free = _eos_retiring_a_lane_early()
    batched = _oracle_run(PROMPTS, {eos}, 3)
    assert batched[early][-1] == eos and len(batched[early]) < MAX_NEW
    assert all(len(batched[o]) == MAX_NEW for o in range(3) if o != early)
    for lane, prompt in enumerate(PROMPTS):
        alone = _oracle_run([prompt], {eos}, 1)[0]
        assert batched[lane] == alone, (lane, batched[lane], alone)
        # without EOS the lane would continue with the same prefix
        assert free[lane][:len(alone)] == alone


@pytest.mark.gpu
def test_worker_generation_on_the_gpu_matches_the_oracle():
    print("case worker continuous generation", flush=True)
    eos, early, _ = _eos_retiring_a_lane_early()
    want = _oracle_run(PROMPTS, {eos}, 3)
    with hip.Session(0) as sess:
        m = hip.Model(sess, CFG, seed=SEED)
        p = hip.Pool(m, PS, PAGES)
        d = hip.Decoder(m, p, 3, PPS, MAXPOS, SPLIT)
        pool = PagePool(PS, PAGES, CFG["n_layers"], CFG["n_kv"], CFG["head_dim"], device=p)
        dec = PagedDecoder(pool, HipStepDevice(d), batch_size=3, maxpos=MAXPOS, pages_per_sequence=PPS)
        got = worker.generate_continuously(dec, ["c0", "c1", "c2"], PROMPTS, MAX_NEW, eos_ids={eos})
    assert got == want
    assert got[early][-1] == eos
