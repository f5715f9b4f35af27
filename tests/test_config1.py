"""BASELINE.json configs[0] as a parity case: the Gemma-3-270M-shaped decoder with Q8
weights (all 18 layers, 262 144-token vocabulary, sliding window 512), one lane,
a 32-token prompt of uniform ids (seed 0) and 64 greedy steps, generated through
the paged-decoder mirror on the HIP decoder and on the CPU oracle: the same 64
tokens, and the same final logits bit for bit."""
import numpy as np
import pytest

import oracle as O
from rstr import configs, hip
from rstr.page_pool import PagePool
from rstr.paged_decoder import HipStepDevice, PagedDecoder

pytestmark = pytest.mark.gpu

CFG = configs.with_bits(configs.GEMMA3_270M, 8)
PS, MAXPOS, SPLIT, SEED = 16, 112, 64, 0
PPS = MAXPOS // PS
PAGES = PPS + 1


class OracleStepDevice:
    def __init__(self, od):
        self.od, self._d, self._t = od, None, None

    def upload(self, desc):
        self._d = desc

    def run(self):
        self._t = self.od.step_lanes(**self._d)

    def download_tokens(self):
        return self._t

    def prime_rows(self, lane_tokens):
        if lane_tokens:
            self.od.prime_lanes([x["lane"] for x in lane_tokens], [x["token"] for x in lane_tokens])


def _generate(device, pool_device):
    prompt = [int(x) for x in np.random.default_rng(0).integers(0, CFG["vocab"], 32)]
    pool = PagePool(PS, PAGES, CFG["n_layers"], CFG["n_kv"], CFG["head_dim"], device=pool_device)
    dec = PagedDecoder(pool, device, batch_size=1, maxpos=MAXPOS, pages_per_sequence=PPS)
    return dec.generate("c", prompt, 64)


def test_config1_gemma_q8_one_lane_64_greedy_steps():
    print("case config1 gemma q8", flush=True)
    om = O.Model(CFG, seed=SEED)
    od = O.Decoder(om, 1, PS, PAGES, PPS, MAXPOS, kv_f16=True, split=SPLIT)
    try:
        want = _generate(OracleStepDevice(od), od)
        want_logits = od.logits()
    finally:
        od.close()
        om.close()
    with hip.Session(0) as sess:
        m = hip.Model(sess, CFG, seed=SEED)
        p = hip.Pool(m, PS, PAGES)
        d = hip.Decoder(m, p, 1, PPS, MAXPOS, SPLIT)
        got = _generate(HipStepDevice(d), p)
        got_logits = d.logits()
    assert len(got) == 64
    assert got == want
    assert np.array_equal(got_logits.view(np.uint32), want_logits.view(np.uint32))
