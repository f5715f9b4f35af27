"""Pool offsets beyond 2^32 bytes: a Llama-3-8B-width pool of 140 000 pages
(4.6 GB per layer slab, the order of the config5 bench pool) in which one lane's
route lives on the highest page ids and another lane's on the lowest, holding the
same K/V and fed the same tokens.  Every path that addresses pages (the attention
DMA, the append fused into the QKV epilogue, the step descriptors) must give both
lanes bit-identical tokens, logits and appended K/V rows."""
import numpy as np
import pytest

from rstr import configs, hip

pytestmark = pytest.mark.gpu


def test_high_page_ids_equal_low_page_ids():
    print("case large pool: 140000 pages, routes at both ends", flush=True)
    cfg = dict(configs.MODELS["llama3_8b"], n_layers=2)
    ps, P, n_pg, prefix, pps = 16, 140_000, 33, 512, 40
    ept = cfg["n_kv"] * cfg["head_dim"]
    pe = ps * ept
    hi = np.arange(P - n_pg, P, dtype=np.int32)
    lo = np.arange(1, 1 + n_pg, dtype=np.int32)
    assert int(hi[0]) * pe * 2 > 2**32  # byte offset of the high route's first page
    rng = np.random.default_rng(3)
    with hip.Session(0) as sess:
        m = hip.Model(sess, cfg, seed=4)
        p = hip.Pool(m, ps, P)
        for slab in (0, 1):
            for layer in range(cfg["n_layers"]):
                data = rng.standard_normal((prefix // ps, ps, ept)).astype(np.float16)
                p.upload(slab, layer, int(hi[0]) * pe, data)
                p.upload(slab, layer, int(lo[0]) * pe, data)
        d = hip.Decoder(m, p, 2, pps, pps * ps, 256)
        d.prime_lanes([0, 1], [77, 77])
        pt = np.full((2, pps), -1, np.int32)
        pt[0, :n_pg] = hi
        pt[1, :n_pg] = lo
        for t in range(3):
            pos = prefix + t
            slots = [int(pt[b, pos // ps]) * ps + pos % ps for b in (0, 1)]
            toks = d.step_lanes(slots, [0, 1, 2], [pos, pos], pt.ravel(), [pos + 1, pos + 1], [0, 0])
            lg = d.logits()
            assert toks[0] == toks[1], t
            assert np.isfinite(lg).all()
            assert np.array_equal(lg[0].view(np.uint32), lg[1].view(np.uint32)), t
        for slab in (0, 1):
            for layer in range(cfg["n_layers"]):
                a = p.download(slab, layer, int(hi[32]) * pe, 3 * ept)
                b = p.download(slab, layer, int(lo[32]) * pe, 3 * ept)
                assert np.array_equal(a, b) and np.any(a != 0), (slab, layer)
        d.close()
        p.close()
