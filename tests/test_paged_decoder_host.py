"""Known-answer tests of the paged-decoder host half, ported from
``test/pretrained/continuation_paged_decoder_test.clj``.  The fixture follows
the reference's (``:86-99``): a 2-layer model with 2 query heads, 1 kv head,
head width 4, 4-token pages, 4 physical pages, maxpos 8 (so 2 pages per
sequence).  The device records the descriptor uploads, the run and the token
download in the order the reference's ``gpu/upload-ranges!``,
``gpu-link/run!`` and ``gpu/download`` calls are asserted.
"""
import numpy as np
import pytest

from rstr.page_pool import PagePool, PagePoolError
from rstr.paged_decoder import DESCRIPTOR_KEYS, PagedDecoder


class RecordingDevice:
    def __init__(self, tokens, fail_run=None, fail_prefill=None):
        self.calls, self.uploads = [], []
        self.tokens = tokens
        self.fail_run, self.fail_prefill = fail_run, fail_prefill

    def upload(self, desc):
        self.uploads.append(desc)
        self.calls.append(("upload", tuple(desc)))

    def run(self):
        self.calls.append(("run",))
        if self.fail_run:
            raise RuntimeError(self.fail_run)

    def download_tokens(self):
        self.calls.append(("download", "tokbuf"))
        return np.asarray(self.tokens, np.int32)

    def prime_rows(self, lane_tokens):
        self.calls.append(("prime", [lt["token"] for lt in lane_tokens]))

    def copy_page(self, src, dst):
        self.calls.append(("copy", src, dst))

    def upload_prefill(self, desc):
        self.uploads.append(desc)
        self.calls.append(("upload_prefill",))

    def run_prefill(self):
        self.calls.append(("run_prefill",))
        if self.fail_prefill:
            raise RuntimeError(self.fail_prefill)


def fixture(batch=1, tokens=(42,), prefill_T=None, **dev):
    device = RecordingDevice(list(tokens), **dev)
    pool = PagePool(4, 4, n_layers=2, n_kv=1, head_dim=4, device=device)
    decoder = PagedDecoder(pool, device, batch_size=batch, maxpos=8, prefill_T=prefill_T)
    return pool, decoder, device


def test_staged_step_publishes_only_after_every_layer_completes():
    """continuation_paged_decoder_test.clj:190-207."""
    pool, dec, dev = fixture()
    dec.allocate_continuation("request")
    assert dec.step("request", 0) == 42
    assert pool.route("request").token_count == 1
    assert dev.calls == [("upload", DESCRIPTOR_KEYS), ("run",), ("download", "tokbuf")]
    assert DESCRIPTOR_KEYS == ("slots", "row_offsets", "positions", "page_table", "lengths", "start_positions")


def test_fixed_batch_publishes_independent_routes_in_lane_order():
    """continuation_paged_decoder_test.clj:209-226."""
    pool, dec, dev = fixture(batch=2, tokens=(41, 42))
    for c in ("left", "right"):
        dec.allocate_continuation(c)
    assert dec.step_batch(["left", "right"], [0, 0]) == [41, 42]
    assert [pool.route(c).token_count for c in ("left", "right")] == [1, 1]
    assert list(dev.uploads[-1]["row_offsets"]) == [0, 1, 2]
    assert list(dev.uploads[-1]["positions"]) == [0, 0]


def test_inactive_lanes_neither_reserve_nor_publish_pages():
    """continuation_paged_decoder_test.clj:228-246."""
    pool, dec, dev = fixture(batch=3, tokens=(40, 41, 42))
    dec.allocate_continuation("middle")
    out = dec.step_lanes([{"lane": 1, "continuation_id": "middle", "position": 0}])
    assert out == [{"lane": 1, "continuation_id": "middle", "position": 0, "token": 41}]
    assert pool.route("middle").token_count == 1
    d = dev.uploads[-1]
    assert list(d["slots"]) == [-1, 0, -1], "only the occupied lane receives an append destination"
    assert list(d["lengths"]) == [0, 1, 0], "inactive attention routes have zero logical length"
    assert list(d["page_table"]) == [-1, -1, 0, -1, -1, -1], "inactive page-table rows contain only padding"


def test_fixed_batch_primes_equal_work_suffixes_at_independent_positions(monkeypatch):
    """continuation_paged_decoder_test.clj:248-268."""
    pool, dec, dev = fixture(batch=2, tokens=(0, 0))
    pool.allocate_route("left", 1)
    pool.allocate_route("right", 0)
    calls = []
    monkeypatch.setattr(dec, "decode_tokens", lambda ids, toks, pos: calls.append(("decode", list(ids), list(toks), list(pos))))
    monkeypatch.setattr(dec, "prime_tokens", lambda toks: calls.append(("prime", list(toks))) or dec)
    assert dec.prime_prompts_batch(["left", "right"], [[10, 11, 12, 13], [20, 21, 22]]) is dec
    assert calls == [("decode", ["left", "right"], [11, 20], [1, 0]),
                     ("decode", ["left", "right"], [12, 21], [2, 1]),
                     ("prime", [13, 22])]


def test_failed_layer_leaves_partial_page_writes_unreachable():
    """continuation_paged_decoder_test.clj:270-281."""
    pool, dec, dev = fixture(fail_run="linked decode failed")
    dec.allocate_continuation("request")
    with pytest.raises(RuntimeError, match="linked decode failed"):
        dec.step("request", 0)
    r = pool.route("request")
    assert r.token_count == 0
    assert r.pending is None


def test_positions_must_extend_the_logical_route():
    """continuation_paged_decoder_test.clj:283-287."""
    pool, dec, dev = fixture()
    dec.allocate_continuation("request", start_position=9)
    with pytest.raises(PagePoolError, match="does not extend"):
        dec.step("request", 8)


def test_restored_prompts_compute_only_the_uncached_suffix(monkeypatch):
    """continuation_paged_decoder_test.clj:289-304."""
    pool, dec, dev = fixture()
    pool.allocate_route("request", 2)
    calls = []
    monkeypatch.setattr(dec, "decode_token", lambda cid, tok, pos: calls.append(("decode", cid, tok, pos)))
    monkeypatch.setattr(dec, "prime_token", lambda tok: calls.append(("prime", tok)) or dec)
    assert dec.prime_prompt("request", [10, 11, 12, 13, 14]) is dec
    assert calls == [("decode", "request", 12, 2), ("decode", "request", 13, 3), ("prime", 14)]


def test_bulk_prefill_publishes_a_complete_range_after_the_linked_run():
    """continuation_paged_decoder_test.clj:306-336."""
    pool, dec, dev = fixture(prefill_T=3)
    dec.allocate_continuation("request")
    assert dec.prefill_range("request", [10, 11, 12], 0) is dec
    assert pool.route("request").token_count == 3
    assert dev.calls == [("upload_prefill",), ("run_prefill",)]
    d = dev.uploads[-1]
    assert list(d["slots"]) == [0, 1, 2]
    assert list(d["row_offsets"]) == [0, 3]
    assert list(d["positions"]) == [0, 1, 2]


def test_prompt_priming_uses_complete_bulk_tiles_and_a_scalar_tail(monkeypatch):
    """continuation_paged_decoder_test.clj:338-364."""
    pool, dec, dev = fixture(prefill_T=3)
    pool.allocate_route("request", 1)
    calls = []
    monkeypatch.setattr(dec, "prefill_range", lambda cid, toks, pos: calls.append(("prefill", cid, list(toks), pos)) or dec)
    monkeypatch.setattr(dec, "decode_token", lambda cid, tok, pos: calls.append(("decode", cid, tok, pos)))
    monkeypatch.setattr(dec, "prime_token", lambda tok: calls.append(("prime", tok)) or dec)
    assert dec.prime_prompt("request", [10, 11, 12, 13, 14, 15, 16]) is dec
    assert calls == [("prefill", "request", [11, 12, 13], 1), ("decode", "request", 14, 4),
                     ("decode", "request", 15, 5), ("prime", 16)]


def test_failed_bulk_prefill_keeps_the_range_unpublished():
    """continuation_paged_decoder_test.clj:366-388."""
    pool, dec, dev = fixture(prefill_T=3, fail_prefill="prefill failed")
    dec.allocate_continuation("request")
    with pytest.raises(RuntimeError, match="prefill failed"):
        dec.prefill_range("request", [10, 11, 12], 0)
    assert pool.route("request").token_count == 0
    assert pool.route("request").pending is None


def test_routed_append_slots_follow_the_reference_boundary():
    """continuation_paged_append_device_test.clj:35-59: 2-token pages, 3
    physical pages; route a (0 tokens) then b (3 tokens) append at physical
    slots [4 3] (page*page_size + offset), published only on commit."""
    from rstr import paged_append
    pool = PagePool(2, 3, n_layers=1, n_kv=1, head_dim=4, device=RecordingDevice([]))
    pool.allocate_route("a", 0)
    pool.allocate_route("b", 3)
    batch = paged_append.reserve_batch(pool, ["a", "b"])
    assert list(batch.slot_values()) == [4, 3]
    assert [pool.route(c).token_count for c in ("a", "b")] == [0, 3]
    batch.commit()
    assert [pool.route(c).token_count for c in ("a", "b")] == [1, 4]
