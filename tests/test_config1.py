"""BASELINE.json configs[0] as a parity case: the Gemma-3-270M-shaped decoder with Q8
weights (all 18 layers, 262 144-token vocabulary, sliding window 512), one lane,
a 32-token prompt of uniform ids (seed 0) and 64 greedy steps, generated through
the paged-decoder mirror on the HIP decoder and on the CPU oracle: the same 64
tokens, and the same final logits bit for bit.

The second test ties the fp16-KV HIP path to the reference CPU path's own KV
precision (f32 kc/vc, decoder.clj:304-310), teacher-forced."""
import numpy as np
import pytest

import oracle as O
from lanes import Routes
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


def _config1_case(split):
    om = O.Model(CFG, seed=SEED)
    od = O.Decoder(om, 1, PS, PAGES, PPS, MAXPOS, kv_f16=True, split=split)
    try:
        want = _generate(OracleStepDevice(od), od)
        want_logits = od.logits()
    finally:
        od.close()
        om.close()
    with hip.Session(0) as sess:
        m = hip.Model(sess, CFG, seed=SEED)
        p = hip.Pool(m, PS, PAGES)
        d = hip.Decoder(m, p, 1, PPS, MAXPOS, split)
        got = _generate(HipStepDevice(d), p)
        got_logits = d.logits()
    assert len(got) == 64
    assert got == want
    assert np.array_equal(got_logits.view(np.uint32), want_logits.view(np.uint32))


def test_config1_gemma_q8_one_lane_64_greedy_steps():
    print("case config1 gemma q8", flush=True)
    _config1_case(SPLIT)


def test_config1_single_split_writes_attention_output_directly():
    """The same run with a split of at least the decoder's maxpos: every visible
    range is one split, so the few-item attention kernel writes the quantised
    attention output itself and the step has no merge launch; tokens and final
    logits equal the oracle's at that split, bit for bit."""
    print("case config1 single split", flush=True)
    _config1_case(128)


def _teacher_forced(step, prime, routes, seq, greedy_from=None):
    """Feed seq[i] as the lane's input at step i (positions 0..); with
    greedy_from, tokens after that step come from the run's own argmax and
    extend seq.  Returns the logits of every step."""
    out = []
    for i in range(96):
        prime(seq[i])
        tokens, logits = step(routes.step([0]))
        out.append(np.array(logits, copy=True))
        if greedy_from is not None and i >= greedy_from and len(seq) < 96:
            seq.append(int(tokens[0]))
    return out


def test_config1_teacher_forced_against_f32_kv_reference():
    """configs[0] through the HIP decoder (fp16 KV) against the oracle's f32-KV
    mode, the reference CPU path's KV precision, on the same token sequence
    (the 32-token prompt, then the f32 run's own 64 greedy tokens).

    The north star's bound (max-abs 2e-2, cosine >= 0.9999) is a per-kernel one
    and holds per kernel (test_gpu_kats.py: attention over fp16 vs f32 KV).
    Across 18 layers the int8 activation quantiser turns any rounding difference
    into quantisation-level noise: two f32-KV oracle runs that differ only in
    the attention's summation order (split 16 vs 64) already disagree by
    max-abs ~0.05.  That floor is measured here, and the fp16-KV path must stay
    within twice it, with cosine >= 0.999 at every step and >= 90% of the greedy
    tokens equal; the measured figures are printed."""
    print("case config1 teacher-forced vs f32 KV", flush=True)
    prompt = [int(x) for x in np.random.default_rng(0).integers(0, CFG["vocab"], 32)]
    om = O.Model(CFG, seed=SEED)
    runs = {}
    seq = list(prompt)
    try:
        for split, greedy in ((SPLIT, 31), (16, None)):
            od = O.Decoder(om, 1, PS, PAGES, PPS, MAXPOS, kv_f16=False, split=split)
            try:
                runs[split] = _teacher_forced(
                    lambda desc: (od.step_lanes(**desc), od.logits()[0]),
                    lambda t: od.prime_lanes([0], [t]), Routes(1, PS, PAGES, PPS, seed=0, permute=False),
                    seq, greedy)
            finally:
                od.close()
    finally:
        om.close()
    assert len(seq) == 96
    with hip.Session(0) as sess:
        m = hip.Model(sess, CFG, seed=SEED)
        p = hip.Pool(m, PS, PAGES)
        d = hip.Decoder(m, p, 1, PPS, MAXPOS, SPLIT)
        gpu = _teacher_forced(lambda desc: (d.step_lanes(**desc), d.logits()[0]),
                              lambda t: d.prime_lanes([0], [t]), Routes(1, PS, PAGES, PPS, seed=0, permute=False),
                              seq)

    def stats(a_list, b_list):
        ma, cs, ag = [], [], []
        for a, b in zip(a_list[31:], b_list[31:]):      # the last prompt step and the 64 generated
            a, b = a.astype(np.float64), b.astype(np.float64)
            ma.append(float(np.max(np.abs(a - b))))
            cs.append(float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b))))
            ag.append(int(np.argmax(a)) == int(np.argmax(b)))
        return max(ma), min(cs), sum(ag) / len(ag)

    ref = runs[SPLIT]
    fma, fcos, fag = stats(runs[16], ref)
    gma, gcos, gag = stats(gpu, ref)
    print(f"  f32 KV split 16 vs split {SPLIT} (floor): max-abs {fma:.4f}, min cosine {fcos:.6f}, "
          f"argmax agreement {fag:.3f}", flush=True)
    print(f"  HIP fp16 KV vs f32 KV: max-abs {gma:.4f}, min cosine {gcos:.6f}, argmax agreement {gag:.3f}",
          flush=True)
    assert gma <= 2 * fma
    assert gcos >= 0.999
    assert gag >= 0.9
