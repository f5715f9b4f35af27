"""CPU restatement of the durable KV chunk gather/scatter.

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` as the checker of the device
chunk transfer, never by the product path.

A chunk of ``count`` tokens starting at logical token ``start`` of a route
with logical pages ``pages`` is the concatenation, in payload-plan order
(attention_state.clj:103-123: slab K then V, layer 0..L-1), of the route's
token rows; a token's row lives at physical token ``page * page_size + offset``
of its slab (page_pool.clj:80-103 transfer-runs, :879-890 token-range-view).
Rows are gathered here one token at a time; the tests pin this against the
reference's own ranged-copy plan (one slice per physical run, whose offsets
the reference's tests fix) and against round trips.
"""
from __future__ import annotations

import numpy as np


def token_rows(pages, page_size: int, start: int, count: int) -> np.ndarray:
    """Physical token index of each chunk token."""
    logical = start + np.arange(count)
    return np.asarray(pages, np.int64)[logical // page_size] * page_size + logical % page_size


def gather(slabs, pages, page_size: int, start: int, count: int) -> np.ndarray:
    """slabs: 2L arrays [physical_pages * page_size, ept] (K layers, then V
    layers) -> the dense payload (fp16 bits as uint16)."""
    rows = token_rows(pages, page_size, start, count)
    return np.concatenate([np.asarray(s)[rows].ravel() for s in slabs])


def scatter(slabs, pages, page_size: int, start: int, count: int, payload) -> None:
    """Inverse of ``gather`` in place; an f32 payload rounds to fp16 to nearest
    even (numpy's float32 -> float16 conversion)."""
    payload = np.asarray(payload)
    if payload.dtype == np.float32:
        with np.errstate(over="ignore"):  # beyond 65504 rounds to infinity, as the device does
            payload = payload.astype(np.float16).view(np.uint16)
    rows = token_rows(pages, page_size, start, count)
    ept = np.asarray(slabs[0]).shape[1]
    per = count * ept
    for i, s in enumerate(slabs):
        s[rows] = payload[i * per:(i + 1) * per].reshape(count, ept)
