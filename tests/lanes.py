"""Minimal lane/route bookkeeping for kernel-level parity tests.

It produces the six step descriptors exactly as ``step-lanes!`` lays them out
(``src/pretrained/continuation/paged_decoder.clj:494-578``): inactive lanes get
slot -1, length 0, start 0, position 0 and a -1 page-table row.  Routes take
pages from a (optionally permuted) free list; no sharing or copy-on-write here
(the page-pool mirror covers those).
"""
from __future__ import annotations

import numpy as np


class Routes:
    def __init__(self, batch, page_size, physical_pages, pps, seed=0, permute=True):
        rng = np.random.default_rng(seed)
        order = rng.permutation(physical_pages) if permute else np.arange(physical_pages)
        self.free = [int(p) for p in order]
        self.batch, self.ps, self.pps = batch, page_size, pps
        self.pages = [[] for _ in range(batch)]
        self.length = [0] * batch
        self.start = [0] * batch

    def _need_page(self, b):
        if self.length[b] % self.ps == 0 and self.length[b] // self.ps == len(self.pages[b]):
            self.pages[b].append(self.free.pop(0))
            return self.pages[b][-1]
        return None

    def prefix(self, b, n):
        """Grow lane b by n tokens of restored prefix; returns the new pages."""
        new = []
        for _ in range(n):
            p = self._need_page(b)
            if p is not None:
                new.append(p)
            self.length[b] += 1
        return new

    def step(self, active):
        """Reserve one appended row in each active lane; return the descriptors."""
        B, ps = self.batch, self.ps
        slots = np.full(B, -1, np.int32)
        pos = np.zeros(B, np.int32)
        lengths = np.zeros(B, np.int32)
        starts = np.zeros(B, np.int32)
        pt = np.full((B, self.pps), -1, np.int32)
        for b in active:
            self._need_page(b)
            t = self.length[b]
            slots[b] = self.pages[b][t // ps] * ps + t % ps
            self.length[b] += 1
            lengths[b] = self.length[b]
            starts[b] = self.start[b]
            pos[b] = self.start[b] + t
            pt[b, :len(self.pages[b])] = self.pages[b]
        return dict(slots=slots, row_offsets=np.arange(B + 1, dtype=np.int32), positions=pos,
                    page_table=pt, lengths=lengths, start_positions=starts)

    def table(self):
        B = self.batch
        pt = np.full((B, self.pps), -1, np.int32)
        for b in range(B):
            pt[b, :len(self.pages[b])] = self.pages[b]
        return pt, np.array(self.length, np.int32)
