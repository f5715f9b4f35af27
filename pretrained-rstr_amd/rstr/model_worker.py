"""One real-model paged worker (``src/pretrained/continuation/model_worker.clj``).

``open_worker`` assembles what the reference's ``open-worker!`` (:52-130) does
for the decode path -- a device session, the model bound from a checkpoint
directory (``load-lm {:gpu? true}``) with its compatibility fingerprint, the
page pool and a one-lane paged decoder (``:batch-size 1``, optionally with a
bulk-prefill tile) -- and closes them in order (``ModelWorker.close``, :18-35).
The continuation manager, its Datahike catalog and the controller handlers
the reference attaches are control plane and stay out of this build; durable
prefixes move through ``rstr.chunks`` on ``worker.pool``.
"""
from __future__ import annotations

from . import hip, loader
from .page_pool import PagePool
from .paged_decoder import HipStepDevice, PagedDecoder


class WorkerError(ValueError):
    pass


def default_measurements(worker_id, max_position: int) -> dict:
    """model_worker.clj:37-50: deployment-constant scheduling measurements."""
    return {"worker/node": str(worker_id).lstrip(":"), "worker/queue-ms": 0.0,
            "worker/max-context": int(max_position), "worker/prefill-ms-per-token": 10.0,
            "worker/first-token-ms": 10.0, "worker/gpu-restore-bytes-per-ms": 1000000.0,
            "worker/tier-throughput-bytes-per-ms": {}, "worker/object-store?": False}


class ModelWorker:
    """model_worker.clj:18-35: the assembled worker; ``close`` is idempotent and
    tears down decoder, pool and session in that order."""

    def __init__(self, worker_id, sess, model, cfg, pool, decoder, prefill, paged, worker_opts, measurements,
                 eos_ids, chunk_size):
        self.id, self.sess, self.model, self.cfg = worker_id, sess, model, cfg
        self.pool, self.decoder, self.prefill, self.paged = pool, decoder, prefill, paged
        self.worker_opts, self.measurements = worker_opts, measurements
        self.eos_ids, self.chunk_size = eos_ids, chunk_size
        self.closed = False

    def generate(self, cid, prompt, max_new: int):
        """Greedy continuation of one route (paged-decoder generate!, stopping at EOS)."""
        return self.paged.generate(cid, prompt, max_new, eos_ids=self.eos_ids)

    def close(self):
        if self.closed:
            return
        self.closed = True
        try:
            for obj in (self.prefill, self.decoder):
                if obj is not None:
                    obj.close()
        finally:
            try:
                if self.pool is not None and self.pool.device is not None:
                    self.pool.device.close()
            finally:
                if self.model is not None:
                    self.model.close()
                self.sess.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


def open_worker(model_directory: str, fingerprint: str, worker_id=":worker-a", device: int = 0,
                max_position: int = 1024, page_size: int = 16, physical_pages: int | None = None,
                chunk_size: int = 16, eos_ids=None, measurements=None, prefill_T: int | None = None,
                split: int = 64, weight_bits: int | None = None) -> ModelWorker:
    """model_worker.clj:52-130 for the decode path: validates the options, binds
    the checkpoint and opens pool and decoder; anything opened is closed again
    if a later step fails.  ``split`` is the attention history tile (it fixes
    the attention's reduction order); a one-lane decoder has few work items, and
    64-token tiles made a Llama-3-8B-shaped step at 512 tokens of context 17%
    shorter than 256-token ones (2.82 vs 3.38 ms)."""
    if not isinstance(fingerprint, str):
        raise WorkerError("Model worker requires a compatibility fingerprint")
    max_position, page_size = int(max_position), int(page_size)
    pps = (max_position + page_size - 1) // page_size
    physical_pages = int(physical_pages or 4 * pps)
    hf = loader.load_hf(model_directory)
    if eos_ids is None:
        e = hf["config"].get("eos_token_id")
        eos_ids = set(e if isinstance(e, list) else ([] if e is None else [e]))
    sess = hip.Session(device)
    opened = []
    try:
        model, cfg = loader.bind_hf(sess, model_directory, weight_bits)
        opened.append(model)
        dev_pool = hip.Pool(model, page_size, physical_pages)
        opened.append(dev_pool)
        decoder = hip.Decoder(model, dev_pool, 1, pps, max_position, split)
        opened.append(decoder)
        prefill = hip.Prefill(model, dev_pool, prefill_T, pps, max_position, split) if prefill_T else None
        if prefill is not None:
            opened.append(prefill)
        pool = PagePool(page_size, physical_pages, cfg["n_layers"], cfg["n_kv"], cfg["head_dim"], "half",
                        device=dev_pool)
        paged = PagedDecoder(pool, HipStepDevice(decoder, prefill), batch_size=1, maxpos=max_position,
                             pages_per_sequence=pps, prefill_T=prefill_T)
        opts = {"worker/id": worker_id, "worker/epoch": 0, "worker/models": {fingerprint},
                "worker/free-pages": physical_pages, "worker/evictable-pages": 0}
        return ModelWorker(worker_id, sess, model, cfg, pool, decoder, prefill, paged, opts,
                           measurements or default_measurements(worker_id, max_position), set(eos_ids),
                           int(chunk_size))
    except BaseException:
        for obj in reversed(opened):
            try:
                obj.close()
            except Exception:
                pass
        sess.close()
        raise
