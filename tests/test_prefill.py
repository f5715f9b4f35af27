"""Bulk paged prefill tiles (``PagedDecoder.prefill_range``, paged_decoder.clj:638-711):
a prompt's uncached suffix goes through the layers ``prefill_T`` rows at a time
(rows as lanes of a prefill decoder with causal lengths, one M = T projection
tile per linear), then decoding continues.  The result must equal token-by-token
priming bit for bit: the same K/V in every page of every layer and the same
generated tokens.

- CPU: the oracle decoder with prefill tiles vs the oracle decoding token by token.
- GPU: the HIP decode decoder (1 lane) and prefill decoder (``rstr_prefill_range``
  over T rows, layers only) on one pool vs the oracle decoding token by token;
  the prefill decoder's error paths.
"""
import numpy as np
import pytest

import oracle as O
from rstr import configs, hip
from rstr.page_pool import PagePool
from rstr.paged_decoder import PagedDecoder, HipStepDevice, DESCRIPTOR_KEYS

MODELS = ["tiny_llama", "tiny_gemma", "tiny_qwen"]   # plain, windowed + sandwich + dual RoPE, qk-norm
PS, PAGES, MAXPOS, SPLIT, SEED, T = 16, 40, 160, 32, 9, 24
PPS = MAXPOS // PS
MAX_NEW = 5


def _prompt(cfg):
    return [int(x) for x in np.random.default_rng(3).integers(0, cfg["vocab"], 61)]


def prefill_lane_descriptors(desc: dict, batch: int) -> dict:
    """A bulk-prefill tile of one route (T rows, ``row_offsets`` [0, T]) as
    decode-step lanes, the way ``rstr_prefill_range`` runs it: row t becomes
    lane t with the route's page-table row, its own slot and position, and the
    causal length ``position - start + 1``."""
    tokens = np.asarray(desc["tokens"], np.int32)
    T = tokens.size
    assert T <= batch
    row = np.asarray(desc["page_table"], np.int32).ravel()
    start = int(np.asarray(desc["start_positions"]).ravel()[0])
    pos = np.asarray(desc["positions"], np.int32)
    out = {"slots": np.full(batch, -1, np.int32), "row_offsets": np.arange(batch + 1, dtype=np.int32),
           "positions": np.zeros(batch, np.int32), "page_table": np.full((batch, row.size), -1, np.int32),
           "lengths": np.zeros(batch, np.int32), "start_positions": np.zeros(batch, np.int32),
           "lanes": np.arange(T, dtype=np.int32), "tokens": tokens}
    out["slots"][:T] = desc["slots"]
    out["positions"][:T] = pos
    out["lengths"][:T] = pos - start + 1
    out["start_positions"][:T] = start
    out["page_table"][:T] = row
    out["page_table"] = out["page_table"].ravel()
    return out


def _pad_lanes(desc, batch):
    """A one-lane decode step as a ``batch``-lane step whose other lanes are idle."""
    pt = np.asarray(desc["page_table"], np.int32).ravel()
    out = {"slots": np.full(batch, -1, np.int32), "row_offsets": np.arange(batch + 1, dtype=np.int32),
           "positions": np.zeros(batch, np.int32), "page_table": np.full((batch, pt.size), -1, np.int32),
           "lengths": np.zeros(batch, np.int32), "start_positions": np.zeros(batch, np.int32)}
    out["slots"][0] = np.asarray(desc["slots"]).ravel()[0]
    out["positions"][0] = np.asarray(desc["positions"]).ravel()[0]
    out["page_table"][0] = pt
    out["lengths"][0] = np.asarray(desc["lengths"]).ravel()[0]
    out["start_positions"][0] = np.asarray(desc["start_positions"]).ravel()[0]
    out["page_table"] = out["page_table"].ravel()
    return out


class OracleDevice:
    """Step and prefill protocol over one oracle decoder: lane 0 decodes (the
    other lanes idle), a prefill tile uses lanes 0..T-1, and the prompt's last
    token is primed into lane 0 afterwards."""

    def __init__(self, od):
        self.od, self._d, self._p, self._tok, self.tiles = od, None, None, None, 0

    def upload(self, desc):
        self._d = _pad_lanes(desc, self.od.batch)

    def run(self):
        self._tok = self.od.step_lanes(**self._d)[:1]

    def download_tokens(self):
        return self._tok

    def prime_rows(self, lane_tokens):
        if lane_tokens:
            self.od.prime_lanes([lt["lane"] for lt in lane_tokens], [lt["token"] for lt in lane_tokens])

    def copy_page(self, src, dst):
        self.od.copy_page(src, dst)

    def upload_prefill(self, desc):
        self._p = prefill_lane_descriptors(desc, self.od.batch)

    def run_prefill(self):
        self.od.prime_lanes(self._p["lanes"], self._p["tokens"])
        self.od.step_lanes(**{k: self._p[k] for k in DESCRIPTOR_KEYS})
        self.tiles += 1


def _generate(cfg, device, batch_of_pool_device, prefill_T):
    pool = PagePool(PS, PAGES, cfg["n_layers"], cfg["n_kv"], cfg["head_dim"], device=batch_of_pool_device)
    dec = PagedDecoder(pool, device, batch_size=1, maxpos=MAXPOS, pages_per_sequence=PPS, prefill_T=prefill_T)
    toks = dec.generate("c", _prompt(cfg), MAX_NEW)
    return toks, pool.route("c").pages


def _oracle_token_by_token(cfg):
    om = O.Model(cfg, seed=SEED)
    od = O.Decoder(om, 1, PS, PAGES, PPS, MAXPOS, kv_f16=True, split=SPLIT)
    try:
        toks, pages = _generate(cfg, OracleDevice(od), od, None)
        slabs = [(od.slab(s, l).view(np.uint16).copy()) for l in range(cfg["n_layers"]) for s in (0, 1)]
        return toks, pages, slabs
    finally:
        od.close()
        om.close()


def test_prefill_lane_descriptors_are_causal_rows_of_one_route():
    desc = {"tokens": [5, 6, 7], "slots": [33, 34, 35], "row_offsets": [0, 3], "positions": [17, 18, 19],
            "page_table": [4, 2, -1], "lengths": [20], "start_positions": [0]}
    d = prefill_lane_descriptors(desc, 4)
    assert d["lengths"].tolist() == [18, 19, 20, 0]
    assert d["slots"].tolist() == [33, 34, 35, -1]
    assert d["page_table"].reshape(4, 3).tolist() == [[4, 2, -1]] * 3 + [[-1, -1, -1]]
    assert d["row_offsets"].tolist() == [0, 1, 2, 3, 4]


@pytest.mark.parametrize("name", MODELS)
def test_oracle_prefill_tiles_equal_token_by_token_priming(name):
    cfg = configs.MODELS[name]
    want_toks, want_pages, want_slabs = _oracle_token_by_token(cfg)
    om = O.Model(cfg, seed=SEED)
    od = O.Decoder(om, T, PS, PAGES, PPS, MAXPOS, kv_f16=True, split=SPLIT)
    try:
        dev = OracleDevice(od)
        toks, pages = _generate(cfg, dev, od, T)
        assert dev.tiles == (len(_prompt(cfg)) - 1) // T == 2
        assert toks == want_toks
        assert pages == want_pages
        for i, (l, s) in enumerate((l, s) for l in range(cfg["n_layers"]) for s in (0, 1)):
            assert np.array_equal(od.slab(s, l).view(np.uint16), want_slabs[i]), (l, s)
    finally:
        od.close()
        om.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name", MODELS)
def test_gpu_prefill_tiles_equal_oracle_token_by_token(name):
    print("case prefill tiles", name, flush=True)
    cfg = configs.MODELS[name]
    want_toks, want_pages, want_slabs = _oracle_token_by_token(cfg)
    with hip.Session(0) as sess:
        m = hip.Model(sess, cfg, seed=SEED)
        p = hip.Pool(m, PS, PAGES)
        d1 = hip.Decoder(m, p, 1, PPS, MAXPOS, SPLIT)
        pf = hip.Prefill(m, p, T, PPS, MAXPOS, SPLIT)
        dev = HipStepDevice(d1, pf)
        toks, pages = _generate(cfg, dev, p, T)
        assert dev._prefill is not None
        assert toks == want_toks
        assert pages == want_pages
        for i, (l, s) in enumerate((l, s) for l in range(cfg["n_layers"]) for s in (0, 1)):
            assert np.array_equal(p.pages(s, l).view(np.uint16).ravel(), want_slabs[i].ravel()), (l, s)


@pytest.mark.gpu
def test_gpu_prefill_decoder_rejects_decode_calls_and_bad_tiles():
    print("case prefill errors", flush=True)
    cfg = configs.MODELS["tiny_llama"]
    with hip.Session(0) as sess:
        m = hip.Model(sess, cfg, seed=SEED)
        p = hip.Pool(m, PS, PAGES)
        pf = hip.Prefill(m, p, 4, PPS, MAXPOS, SPLIT)
        z = np.zeros(4, np.int32)
        descs = [np.ascontiguousarray(a, np.int32) for a in (z - 1, np.arange(5), z, np.full(4 * PPS, -1), z, z, z)]
        with pytest.raises(hip.RstrError, match="no head"):
            sess.check(hip.lib().rstr_step_lanes(pf.h, *[a.ctypes.data for a in descs]))
        row = np.full(PPS, -1, np.int32)
        row[0] = 3
        # a row outside the route, and a slot that is not the row's own token
        with pytest.raises(hip.RstrError, match="outside the route"):
            pf.prefill_range([1, 2, 3, 4], [48, 49, 50, 51], [0, 1, 2, 3], row, 3, 0)
        with pytest.raises(hip.RstrError, match="slot"):
            pf.prefill_range([1, 2, 3, 4], [48, 49, 51, 50], [0, 1, 2, 3], row, 4, 0)
        with pytest.raises(hip.RstrError, match="prefill-T"):
            hip.Prefill(m, p, MAXPOS + 1, PPS, MAXPOS, SPLIT)
        pf.prefill_range([1, 2, 3, 4], [48, 49, 50, 51], [0, 1, 2, 3], row, 4, 0)
        with pytest.raises(hip.RstrError, match="schedules"):
            sess.check(hip.lib().rstr_schedule_upload(pf.h, None, 1))


@pytest.mark.gpu
def test_gpu_prefill_wide_tiles_at_llama_width_equal_the_oracle():
    """Llama-3-8B width (d 4096, 32/8 heads, hd 128, vocab 128 256; first layer
    only): a 600-token prompt in two 256-row tiles plus an 87-token scalar tail
    writes the same K/V as the oracle primed token by token, and the next
    tokens agree."""
    print("case prefill llama width", flush=True)
    cfg = dict(configs.MODELS["llama3_8b"], n_layers=1)
    ps, maxpos, split, tile = 16, 640, 256, 256
    pps, pages = maxpos // ps, maxpos // ps + 2
    prompt = [int(x) for x in np.random.default_rng(8).integers(0, cfg["vocab"], 600)]

    def gen(device, pool_device, prefill_T):
        pool = PagePool(ps, pages, cfg["n_layers"], cfg["n_kv"], cfg["head_dim"], device=pool_device)
        dec = PagedDecoder(pool, device, batch_size=1, maxpos=maxpos, pages_per_sequence=pps, prefill_T=prefill_T)
        return dec.generate("c", prompt, 3), pool.route("c").pages

    om = O.Model(cfg, seed=SEED)
    od = O.Decoder(om, 1, ps, pages, pps, maxpos, kv_f16=True, split=split)
    try:
        want, want_pages = gen(OracleDevice(od), od, None)
        want_slabs = [od.slab(s, 0).view(np.uint16).copy() for s in (0, 1)]
    finally:
        od.close()
        om.close()
    with hip.Session(0) as sess:
        m = hip.Model(sess, cfg, seed=SEED)
        p = hip.Pool(m, ps, pages)
        d1 = hip.Decoder(m, p, 1, pps, maxpos, split)
        pf = hip.Prefill(m, p, tile, pps, maxpos, split)
        got, pages_got = gen(HipStepDevice(d1, pf), p, tile)
        got_slabs = [p.pages(s, 0).view(np.uint16).ravel() for s in (0, 1)]
    assert got == want and pages_got == want_pages
    for a, b in zip(got_slabs, want_slabs):
        assert np.array_equal(a, b.ravel())
