"""The allocation-free attention entry (rstr_attention_run_static) against the
allocating one (rstr_attention_run): the same results bit for bit on two calls
in a row, the second smaller (the staging array keeps the first call's
contents), and a clear rejection, with no device work, of a call whose staging
would exceed the array."""
from __future__ import annotations

import math

import numpy as np
import pytest

from rstr import configs, hip, workload

pytestmark = pytest.mark.gpu


def _cfg(n_q, n_kv, hd):
    c = dict(configs.TINY_LLAMA)
    c.update(n_layers=1, d_model=128, d_ff=128, vocab=64, n_q=n_q, n_kv=n_kv, head_dim=hd)
    return c


def test_static_attention_equals_the_allocating_entry():
    print("case no-alloc attention", flush=True)
    with hip.Session(0) as sess:
        # call 1: BASELINE configs[3]'s routes (128 lanes, contexts to 20 160, shared pages)
        lengths, pt, physical, _, rng = workload.shared_prefix_routes(128, 4)
        m = hip.Model(sess, _cfg(32, 8, 128), seed=1)
        p = hip.Pool(m, 16, physical)
        p.fill_synthetic(np.arange(physical, dtype=np.int32), 4)
        q = rng.standard_normal((128, 32, 128)).astype(np.float32)
        scale = 1.0 / math.sqrt(128)
        want = p.attention(0, q, pt, lengths, scale=scale, split=256)
        got = p.attention(0, q, pt, lengths, scale=scale, split=256, static=True)
        assert np.array_equal(got, want)
        # call 2: fewer, shorter lanes with a window and another split
        lengths2 = np.array([1, 0, 300, 2049, 77], np.int32)
        pt2 = pt[:5, : int(-(-lengths2.max() // 16))].copy()
        q2 = rng.standard_normal((5, 32, 128)).astype(np.float32)
        want2 = p.attention(0, q2, pt2, lengths2, window=700, scale=scale, split=32)
        got2 = p.attention(0, q2, pt2, lengths2, window=700, scale=scale, split=32, static=True)
        assert np.array_equal(got2, want2)
        assert np.all(got2[1] == 0)
        # a call whose partials would exceed the staging array is refused up front
        big = np.full(1024, 4096, np.int32)
        big_pt = np.tile(np.arange(256, dtype=np.int32) % physical, (1024, 1))
        qb = np.zeros((1024, 32, 128), np.float32)
        with pytest.raises(hip.RstrError, match="static staging maximum"):
            p.attention(0, qb, big_pt, big, scale=scale, split=16, static=True)
        # and the entry still works after the refusal
        got3 = p.attention(0, q2, pt2, lengths2, window=700, scale=scale, split=32, static=True)
        assert np.array_equal(got3, want2)
