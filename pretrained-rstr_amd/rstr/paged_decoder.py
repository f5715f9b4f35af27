"""Paged autoregressive execution over a resident decoder
(``src/pretrained/continuation/paged_decoder.clj``).

The host half of a step: validate lanes, reserve one append row per active
lane, pin the prospective routes, build the fixed-width descriptors, run the
device step, publish the new lengths, return tokens.  The device half is an
object with ``upload(desc)``, ``run()``, ``download_tokens()``, ``prime_rows``
(and, for bulk prefill, ``upload_prefill``/``run_prefill``) -- the HIP adapter
below, or a recording fake in tests, standing where the reference calls
``gpu/upload-ranges!``, ``gpu-link/run!`` and ``gpu/download``.
"""
from __future__ import annotations

import numpy as np

from . import paged_append
from .page_pool import PagePool, PagePoolError


class HipStepDevice:
    """Adapter from the three-call device protocol to one ``rstr_step_lanes`` call
    (which uploads, replays the step graph and downloads the tokens).  With a
    ``prefill`` (``hip.Prefill`` on the same model and pool) it also runs
    bulk-prefill tiles through ``rstr_prefill_range``."""

    def __init__(self, decoder, prefill=None):
        self.decoder = decoder
        self.prefill = prefill
        self._desc = None
        self._tokens = None
        self._prefill = None

    def upload(self, desc: dict):
        self._desc = desc

    def run(self):
        self._tokens = self.decoder.step_lanes(**self._desc)

    def download_tokens(self):
        return self._tokens

    def prime_rows(self, lane_tokens):
        if lane_tokens:
            self.decoder.prime_lanes([lt["lane"] for lt in lane_tokens], [lt["token"] for lt in lane_tokens])

    def upload_prefill(self, desc: dict):
        if self.prefill is None:
            raise PagePoolError("Paged decoder has no resident bulk-prefill executable")
        self._prefill = desc

    def run_prefill(self):
        d = self._prefill
        self.prefill.prefill_range(d["tokens"], d["slots"], d["positions"], d["page_table"],
                                   int(np.asarray(d["lengths"]).ravel()[0]),
                                   int(np.asarray(d["start_positions"]).ravel()[0]))


DESCRIPTOR_KEYS = ("slots", "row_offsets", "positions", "page_table", "lengths", "start_positions")


class PagedDecoder:
    """PagedDecoder record (paged_decoder.clj:24-30) over a page pool and a device."""

    def __init__(self, pool: PagePool, device, batch_size: int = 1, maxpos: int = 64,
                 pages_per_sequence: int | None = None, prefill_T: int | None = None):
        """open! (paged_decoder.clj:321-420) minus graph linking."""
        if not isinstance(batch_size, int) or batch_size <= 0:
            raise PagePoolError("Decode batch size must be positive", batch_size=batch_size)
        self.pool, self.device = pool, device
        self.batch_size, self.maxpos, self.prefill_T = batch_size, maxpos, prefill_T
        self.pages_per_sequence = pages_per_sequence or -(-maxpos // pool.page_size)
        self.closed = False

    def _require_open(self):
        if self.closed:
            raise PagePoolError("Paged decoder is closed")

    # ---- routes and priming -----------------------------------------------
    def allocate_continuation(self, cid, start_position: int = 0):
        """paged_decoder.clj:436-447."""
        self._require_open()
        return self.pool.allocate_route(cid, 0, start_position=start_position)

    def prime_token(self, token):
        """paged_decoder.clj:449-457."""
        self._require_open()
        if self.batch_size != 1:
            raise PagePoolError("Use prime-tokens! with a batched paged decoder", batch_size=self.batch_size)
        self.device.prime_rows([{"lane": 0, "token": token}])
        return self

    def prime_tokens(self, tokens):
        """paged_decoder.clj:459-467 -> decoder_gpu.clj:1228-1246."""
        self._require_open()
        tokens = list(tokens)
        if len(tokens) != self.batch_size:
            raise PagePoolError("Resident token batch does not match the bound decoder",
                                expected=self.batch_size, actual=len(tokens))
        self.device.prime_rows([{"lane": i, "token": t} for i, t in enumerate(tokens)])
        return self

    def prime_lanes(self, lane_tokens):
        """paged_decoder.clj:462-471 -> decoder_gpu.clj:1248-1271."""
        self._require_open()
        lanes = [lt["lane"] for lt in lane_tokens]
        if len(lanes) != len(set(lanes)) or not all(
                isinstance(l, (int, np.integer)) and 0 <= l < self.batch_size for l in lanes):
            raise PagePoolError("Resident token lanes are invalid for the bound decoder",
                                batch_size=self.batch_size, lanes=lanes)
        self.device.prime_rows(list(lane_tokens))
        return self

    # ---- the lane step -----------------------------------------------------
    def _checked_active_lanes(self, lane_work):
        """paged_decoder.clj:473-492."""
        work = sorted(({**w, "position": int(w["position"])} for w in lane_work), key=lambda w: w["lane"])
        lanes = [w["lane"] for w in work]
        cids = [w["continuation_id"] for w in work]
        if not work:
            raise PagePoolError("Paged execution requires at least one active lane")
        if not (all(isinstance(l, (int, np.integer)) and 0 <= l < self.batch_size for l in lanes)
                and len(lanes) == len(set(lanes))):
            raise PagePoolError("Active decode lanes are invalid for the bound decoder",
                                batch_size=self.batch_size, lanes=lanes)
        if any(c is None for c in cids) or len(cids) != len(set(cids)):
            raise PagePoolError("Active decode continuation identities must be unique")
        return work

    def scatter_route_values(self, lanes, compact):
        """paged_decoder.clj:494-510: compact per-route rows into fixed lanes."""
        B, pps = self.batch_size, self.pages_per_sequence
        pt = np.full(B * pps, -1, np.int32)
        lengths = np.zeros(B, np.int32)
        starts = np.zeros(B, np.int32)
        for row, lane in enumerate(lanes):
            pt[lane * pps:(lane + 1) * pps] = compact["page-table"][row * pps:(row + 1) * pps]
            lengths[lane] = compact["lengths"][row]
            starts[lane] = compact["start-positions"][row]
        return {"page_table": pt, "lengths": lengths, "start_positions": starts}

    def step_lanes(self, lane_work):
        """paged_decoder.clj:512-583: reserve, lease, upload six descriptors, run,
        release the lease, commit, download the tokens; abort on failure."""
        self._require_open()
        B = self.batch_size
        work = self._checked_active_lanes(lane_work)
        lanes = [w["lane"] for w in work]
        cids = [w["continuation_id"] for w in work]
        for w in work:
            r = self.pool.route(w["continuation_id"])
            if r is None:
                raise PagePoolError("Continuation is not resident", continuation_id=w["continuation_id"])
            expected = r.start_position + r.token_count
            if expected != w["position"]:
                raise PagePoolError("Paged decode position does not extend the resident route",
                                    continuation_id=w["continuation_id"], expected=expected,
                                    actual=w["position"])
            if not r.token_count < self.maxpos:
                raise PagePoolError("Paged decode reached its route capacity",
                                    continuation_id=w["continuation_id"], token_count=r.token_count,
                                    capacity=self.maxpos)
        batch = paged_append.reserve_batch(self.pool, cids)
        try:
            lease = self.pool.acquire_prospective_lease(batch.entries)
            try:
                compact = self.pool.leased_dense_route_values(lease, self.pages_per_sequence)
                rv = self.scatter_route_values(lanes, compact)
                slots = np.full(B, -1, np.int32)
                positions = np.zeros(B, np.int32)
                compact_slots = batch.slot_values()
                for row, w in enumerate(work):
                    slots[w["lane"]] = compact_slots[row]
                    positions[w["lane"]] = w["position"]
                self.device.upload({"slots": slots, "row_offsets": np.arange(B + 1, dtype=np.int32),
                                    "positions": positions, "page_table": rv["page_table"],
                                    "lengths": rv["lengths"], "start_positions": rv["start_positions"]})
                self.device.run()
            finally:
                self.pool.release_lease(lease)
            batch.commit()
            tokens = self.device.download_tokens()
            return [{**w, "token": int(tokens[w["lane"]])} for w in work]
        except BaseException:
            if batch.state == "reserved":
                batch.abort()
            raise

    def step_batch(self, cids, positions):
        """paged_decoder.clj:585-609."""
        cids, positions = list(cids), [int(p) for p in positions]
        if not (len(cids) == self.batch_size == len(positions)):
            raise PagePoolError("Paged step does not match the bound decode batch",
                                batch_size=self.batch_size)
        out = self.step_lanes([{"lane": i, "continuation_id": c, "position": p}
                               for i, (c, p) in enumerate(zip(cids, positions))])
        return [o["token"] for o in out]

    def step(self, cid, position):
        """paged_decoder.clj:611-623."""
        if self.batch_size != 1:
            raise PagePoolError("Use step-batch! with a batched paged decoder", batch_size=self.batch_size)
        return self.step_batch([cid], [position])[0]

    def decode_token(self, cid, token, position):
        """paged_decoder.clj:625-629."""
        self.prime_token(token)
        return self.step(cid, position)

    def decode_tokens(self, cids, tokens, positions):
        """paged_decoder.clj:631-636."""
        self.prime_tokens(tokens)
        return self.step_batch(cids, positions)

    # ---- prompts -------------------------------------------------------------
    def prefill_range(self, cid, tokens, start_position):
        """paged_decoder.clj:638-711: one complete multi-row tile, published after the run."""
        self._require_open()
        tile = self.prefill_T
        tokens = list(tokens)
        r = self.pool.route(cid)
        if r is None:
            raise PagePoolError("Continuation is not resident", continuation_id=cid)
        expected = r.start_position + r.token_count
        if not tile or not hasattr(self.device, "run_prefill"):
            raise PagePoolError("Paged decoder has no resident bulk-prefill executable")
        if self.batch_size != 1:
            raise PagePoolError("Bulk prompt prefill currently supports one sequence")
        if len(tokens) != tile:
            raise PagePoolError("Prompt tile does not match the bound prefill row count",
                                prefill_T=tile, token_count=len(tokens))
        if expected != start_position:
            raise PagePoolError("Paged prefill range does not extend the resident route",
                                continuation_id=cid, expected=expected, actual=start_position)
        if r.token_count + tile > self.maxpos:
            raise PagePoolError("Paged prefill range exceeds route capacity", continuation_id=cid)
        batch = paged_append.reserve_range(self.pool, cid, tile)
        try:
            lease = self.pool.acquire_prospective_lease(batch.entries)
            try:
                rv = self.pool.leased_dense_route_values(lease, self.pages_per_sequence)
                self.device.upload_prefill({
                    "tokens": np.asarray(tokens, np.int32), "slots": batch.slot_values(),
                    "row_offsets": np.array([0, tile], np.int32),
                    "positions": np.arange(start_position, start_position + tile, dtype=np.int32),
                    "page_table": rv["page-table"], "lengths": rv["lengths"],
                    "start_positions": rv["start-positions"]})
                self.device.run_prefill()
            finally:
                self.pool.release_lease(lease)
            batch.commit()
            return self
        except BaseException:
            if batch.state == "reserved":
                batch.abort()
            raise

    def prime_prompts_batch(self, cids, prompts):
        """paged_decoder.clj:713-749: equal missing suffixes, final tokens left pending."""
        self._require_open()
        cids, prompts = list(cids), [list(p) for p in prompts]
        if not (len(cids) == self.batch_size == len(prompts) and all(prompts)):
            raise PagePoolError("Prompt batch does not match the bound decoder", batch_size=self.batch_size)
        routes = [self.pool.route(c) or self.allocate_continuation(c) for c in cids]
        cached = [r.token_count for r in routes]
        processed = [len(p) - 1 for p in prompts]
        missing = [p - c for p, c in zip(processed, cached)]
        if not all(r.start_position == 0 for r in routes):
            raise PagePoolError("Paged prompt priming requires zero absolute starts")
        if any(m < 0 for m in missing):
            raise PagePoolError("A resident prefix is longer than its prompt")
        if len(set(missing)) != 1:
            raise PagePoolError("Fixed decode lanes require equal missing suffix lengths", missing=missing)
        for off in range(missing[0]):
            pos = [c + off for c in cached]
            self.decode_tokens(cids, [p[q] for p, q in zip(prompts, pos)], pos)
        return self.prime_tokens([p[-1] for p in prompts])

    def generate_batch(self, cids, prompts, max_new: int):
        """paged_decoder.clj:751-772."""
        cids, prompts = list(cids), [list(p) for p in prompts]
        self.prime_prompts_batch(cids, prompts)
        positions = [len(p) - 1 for p in prompts]
        out = [[] for _ in prompts]
        while len(out[0]) < max_new and all(self.pool.route(c).token_count < self.maxpos for c in cids):
            toks = self.step_batch(cids, positions)
            positions = [p + 1 for p in positions]
            for o, t in zip(out, toks):
                o.append(t)
        return out

    def prime_prompt(self, cid, prompt):
        """paged_decoder.clj:774-813: only the uncached suffix is computed."""
        self._require_open()
        prompt = list(prompt)
        if not prompt:
            raise PagePoolError("Paged prompt priming requires a nonempty prompt")
        r = self.pool.route(cid) or self.allocate_continuation(cid)
        cached, processed = r.token_count, len(prompt) - 1
        if r.start_position != 0:
            raise PagePoolError("Paged prompt priming requires a zero absolute start position")
        if cached > processed:
            raise PagePoolError("Resident prefix is longer than the prompt's processed prefix")
        tile = self.prefill_T
        bulk_end = cached + tile * ((processed - cached) // tile) if tile else cached
        if tile:
            for p in range(cached, bulk_end, tile):
                self.prefill_range(cid, prompt[p:p + tile], p)
        for p in range(bulk_end, processed):
            self.decode_token(cid, prompt[p], p)
        return self.prime_token(prompt[-1])

    def generate(self, cid, prompt, max_new: int, eos_ids=()):
        """paged_decoder.clj:815-838."""
        self._require_open()
        prompt = list(prompt)
        if not prompt:
            raise PagePoolError("Paged generation requires a nonempty prompt")
        pos = len(prompt) - 1
        self.prime_prompt(cid, prompt)
        out = []
        while len(out) < max_new and self.pool.route(cid).token_count < self.maxpos:
            t = self.step(cid, pos)
            out.append(t)
            if t in eos_ids:
                break
            pos += 1
        return out

    def close(self):
        """paged_decoder.clj:840-854 (idempotent)."""
        self.closed = True
