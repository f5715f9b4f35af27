"""ctypes binding of ``librstr_hip.so`` (declared in ``include/rstr_hip.h``).

This is the Python twin of the JDK 21 FFM binding a Clojure caller would use:
thin handles, plain int32/f32 arrays, negative status codes
turned into :class:`RstrError` carrying the library's message, the way the
reference raises ``ex-info``.  No computation happens here; every call goes to
the HIP library, and loading fails loudly if the library is missing.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG, "lib", "librstr_hip.so")

ROLE = dict(embed=0, final_norm=1, attn_norm=2, q=3, k=4, v=5, o=6, q_norm=7, k_norm=8,
            post_attn_norm=9, ffn_pre_norm=10, ffn_post_norm=11, gate=12, up=13, down=14)
KERNEL_CLASSES = ("qgemm", "head", "attn_split", "attn_merge", "qkv_post", "rows", "tail")

EXPORTS = (
    "rstr_session_open", "rstr_session_close", "rstr_last_error", "rstr_open_error",
    "rstr_session_memory",
    "rstr_model_bind", "rstr_model_bind_raw", "rstr_model_bind_synthetic", "rstr_model_close", "rstr_model_weight_bytes",
    "rstr_model_export_linear", "rstr_pool_open", "rstr_pool_close", "rstr_pool_copy_page",
    "rstr_pool_upload", "rstr_pool_download", "rstr_pool_fill_synthetic", "rstr_chunk_export_submit",
    "rstr_chunk_restore_submit", "rstr_transfer_done", "rstr_transfer_complete", "rstr_chunk_bench", "rstr_decoder_open",
    "rstr_decoder_close", "rstr_prime_lanes", "rstr_prime_rows", "rstr_step_lanes",
    "rstr_step_lanes_submit", "rstr_step_lanes_collect",
    "rstr_decode_logits", "rstr_decoder_read_rows", "rstr_decoder_set_graph", "rstr_decoder_step_timing",
    "rstr_prefill_open",
    "rstr_prefill_range", "rstr_append_run", "rstr_tail_run", "rstr_linear_run",
    "rstr_attention_run", "rstr_attention_run_static",
    "rstr_attention_bench", "rstr_schedule_upload", "rstr_schedule_run",
    "rstr_decoder_profile_steps",
)


class RstrError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class Desc(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n_layers", "d_model", "d_ff", "n_q", "n_kv", "head_dim", "vocab", "weight_bits",
        "gain_offset", "qk_norm", "sandwich", "ffn_geglu", "rope_dual", "global_pattern",
        "sliding_window", "embed_scale_sqrt_d")] + [
        ("eps", C.c_float), ("attn_scale", C.c_float),
        ("rope_global", C.c_double), ("rope_local", C.c_double)]


class Tensor(C.Structure):
    _fields_ = [("layer", C.c_int32), ("role", C.c_int32), ("data", C.c_void_p),
                ("elements", C.c_int64)]


class RawTensor(C.Structure):
    _fields_ = [("layer", C.c_int32), ("role", C.c_int32), ("dtype", C.c_int32), ("data", C.c_void_p),
                ("elements", C.c_int64)]


RAW_DTYPES = {"F32": 0, "F16": 1, "BF16": 2}


class TransferStats(C.Structure):
    _fields_ = [("bytes", C.c_int64), ("device_ms", C.c_float), ("direction", C.c_int32)]


class StagedStep(C.Structure):
    _fields_ = [("slots", C.c_void_p), ("row_offsets", C.c_void_p), ("positions", C.c_void_p),
                ("page_table", C.c_void_p), ("lengths", C.c_void_p),
                ("start_positions", C.c_void_p), ("fill_pages", C.c_void_p),
                ("n_fill", C.c_int32), ("fill_seed", C.c_uint64), ("cow_pairs", C.c_void_p),
                ("n_cow", C.c_int32), ("prime_lanes", C.c_void_p), ("prime_tokens", C.c_void_p),
                ("n_prime", C.c_int32)]


_lib = None


def lib():
    """Load the HIP library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP extension missing: {LIB_PATH} (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        P, i32, i64, u64, f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64, C.c_float
        sig = {
            "rstr_session_open": (i32, [i32, C.POINTER(P)]),
            "rstr_session_close": (i32, [P]),
            "rstr_last_error": (C.c_char_p, [P]),
            "rstr_open_error": (C.c_char_p, []),
            "rstr_session_memory": (i32, [P, C.POINTER(i64), C.POINTER(i64)]),
            "rstr_model_bind": (i32, [P, P, P, i32, C.POINTER(P)]),
            "rstr_model_bind_synthetic": (i32, [P, P, u64, C.POINTER(P)]),
            "rstr_model_bind_raw": (i32, [P, P, P, i32, C.POINTER(P)]),
            "rstr_model_close": (i32, [P]),
            "rstr_model_weight_bytes": (i64, [P]),
            "rstr_model_export_linear": (i32, [P, i32, i32, P, P]),
            "rstr_pool_open": (i32, [P, i32, i32, C.POINTER(P)]),
            "rstr_pool_close": (i32, [P]),
            "rstr_pool_copy_page": (i32, [P, i32, i32]),
            "rstr_pool_upload": (i32, [P, i32, i32, i64, P, i64]),
            "rstr_pool_download": (i32, [P, i32, i32, i64, P, i64]),
            "rstr_pool_fill_synthetic": (i32, [P, P, i32, u64]),
            "rstr_chunk_export_submit": (i32, [P, P, i32, i32, i32, P, C.POINTER(P)]),
            "rstr_chunk_restore_submit": (i32, [P, P, i32, i32, i32, P, i32, C.POINTER(P)]),
            "rstr_transfer_done": (i32, [P]),
            "rstr_chunk_bench": (i32, [P, P, i32, i32, i32, i32, i32, C.POINTER(f32)]),
            "rstr_transfer_complete": (i32, [P, C.POINTER(TransferStats)]),
            "rstr_decoder_open": (i32, [P, P, i32, i32, i32, i32, C.POINTER(P)]),
            "rstr_decoder_close": (i32, [P]),
            "rstr_prime_lanes": (i32, [P, i32, P, P]),
            "rstr_prime_rows": (i32, [P, i32, P, P]),
            "rstr_step_lanes": (i32, [P, P, P, P, P, P, P, P]),
            "rstr_step_lanes_submit": (i32, [P, P, P, P, P, P, P]),
            "rstr_step_lanes_collect": (i32, [P, P]),
            "rstr_decode_logits": (i32, [P, P]),
            "rstr_decoder_read_rows": (i32, [P, P]),
            "rstr_decoder_set_graph": (i32, [P, i32]),
            "rstr_decoder_step_timing": (i32, [P, P, i32]),
            "rstr_linear_run": (i32, [P, i32, i32, i32, P, P, i32, i32, P]),
            "rstr_prefill_open": (i32, [P, P, i32, i32, i32, i32, C.POINTER(P)]),
            "rstr_prefill_range": (i32, [P, P, P, P, P, i32, i32]),
            "rstr_append_run": (i32, [P, i32, i32, P, P, P]),
            "rstr_tail_run": (i32, [P, i32, i32, i32, P, P, P, P]),
            "rstr_attention_run": (i32, [P, i32, i32, i32, i32, i32, f32, P, P, P, P, i32, P, P, P]),
            "rstr_attention_run_static": (i32, [P, i32, i32, i32, i32, i32, f32, P, P, P, P, i32, P, P, P]),
            "rstr_attention_bench": (i32, [P, i32, i32, i32, i32, i32, f32, P, P, i32, P, i32,
                                           C.POINTER(f32), C.POINTER(f32)]),
            "rstr_schedule_upload": (i32, [P, P, i32]),
            "rstr_schedule_run": (i32, [P, i32, i32, P, C.POINTER(f32)]),
            "rstr_decoder_profile_steps": (i32, [P, i32, i32, P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def make_desc(cfg: dict) -> Desc:
    d = Desc()
    for name, _ in Desc._fields_:
        setattr(d, name, cfg[name])
    return d


class Session:
    """A device session (raster.gpu.core/make-session)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        rc = lib().rstr_session_open(device, C.byref(h))
        if rc != 0:
            raise RstrError(rc, lib().rstr_open_error().decode())
        self.h = h
        self.children = []   # open models, pools, decoders (closed before the session)

    def _adopt(self, obj):
        self.children.append(obj)

    def memory(self):
        """(free, total) device bytes."""
        f, t = C.c_int64(), C.c_int64()
        self.check(lib().rstr_session_memory(self.h, C.byref(f), C.byref(t)))
        return f.value, t.value

    def check(self, rc: int):
        if rc != 0:
            raise RstrError(rc, lib().rstr_last_error(self.h).decode())

    def close(self):
        if self.h:
            order = {"Decoder": 0, "Prefill": 0, "Pool": 1, "Model": 2}
            for obj in sorted(self.children, key=lambda o: order.get(type(o).__name__, 3)):
                obj.close()
            self.children = []
            lib().rstr_session_close(self.h)
            self.h = None

    def tail(self, logits, emb):
        """The decode tail on given logits [rows][vocab] and embedding [vocab][d]
        (decode-tail!): (tokens [rows], gathered rows [rows][d])."""
        logits, emb = _f32(logits), _f32(emb)
        rows, vocab = logits.shape
        d = emb.shape[1]
        if emb.shape[0] != vocab:
            raise ValueError("embedding rows differ from the vocabulary")
        tok = np.empty(rows, np.int32)
        out = np.empty((rows, d), np.float32)
        self.check(lib().rstr_tail_run(self.h, rows, vocab, d, _p(logits), _p(emb), _p(tok), _p(out)))
        return tok, out

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


class Model:
    """Resident quantised model (decoder-gpu/bind-decode! weights)."""

    def __init__(self, sess: Session, cfg: dict, seed: int | None = None, tensors=None, raw_tensors=None):
        """``tensors``: (layer, role, f32 array); ``raw_tensors``: (layer, role,
        "F32" | "F16" | "BF16", array of the stored elements -- float32, float16
        or the bf16 bit patterns as uint16), e.g. views of a mapped checkpoint."""
        self.sess, self.cfg = sess, dict(cfg)
        self._desc = make_desc(cfg)
        h = C.c_void_p()
        if raw_tensors is not None:
            keep = []
            arr = (RawTensor * len(raw_tensors))()
            for i, (layer, role, dtype, data) in enumerate(raw_tensors):
                code = RAW_DTYPES[dtype]
                data = np.ascontiguousarray(data).reshape(-1)
                if data.itemsize != (4 if code == 0 else 2):
                    raise ValueError(f"{dtype} tensor with {data.dtype} elements")
                keep.append(data)
                arr[i] = RawTensor(layer, ROLE[role] if isinstance(role, str) else role, code,
                                   data.ctypes.data, data.size)
            rc = lib().rstr_model_bind_raw(sess.h, C.byref(self._desc), C.cast(arr, C.c_void_p),
                                           len(raw_tensors), C.byref(h))
        elif tensors is None:
            rc = lib().rstr_model_bind_synthetic(sess.h, C.byref(self._desc), int(seed), C.byref(h))
        else:
            keep = []
            arr = (Tensor * len(tensors))()
            for i, (layer, role, data) in enumerate(tensors):
                data = _f32(data).ravel()
                keep.append(data)
                arr[i] = Tensor(layer, ROLE[role] if isinstance(role, str) else role,
                                data.ctypes.data, data.size)
            rc = lib().rstr_model_bind(sess.h, C.byref(self._desc), C.cast(arr, C.c_void_p),
                                       len(tensors), C.byref(h))
        sess.check(rc)
        self.h = h
        sess._adopt(self)

    @property
    def weight_bytes(self) -> int:
        return int(lib().rstr_model_weight_bytes(self.h))

    LINEAR_FORMS = {"auto": 0, "tile": 1, "wave_gemv": 2, "wg_gemv": 3}

    def linear(self, layer: int, role: str, xq, xs, splits: int, form: str = "auto") -> np.ndarray:
        """One resident projection on int8 activations (rstr_linear_run): role
        "q" is the fused [q|k|v] tensor, "gate" the fused [gate|up] one, "embed"
        the tied head."""
        xq = np.ascontiguousarray(np.asarray(xq, np.int8))
        xs = np.ascontiguousarray(np.asarray(xs, np.float32))
        rows, k = xq.shape
        n = {"q": (self.cfg["n_q"] + 2 * self.cfg["n_kv"]) * self.cfg["head_dim"], "o": self.cfg["d_model"],
             "gate": 2 * self.cfg["d_ff"], "down": self.cfg["d_model"], "embed": self.cfg["vocab"]}[role]
        y = np.empty((rows, n), np.float32)
        self.sess.check(lib().rstr_linear_run(self.h, layer, ROLE[role], rows, _p(xq), _p(xs), splits,
                                              self.LINEAR_FORMS[form], _p(y)))
        return y

    def export_linear(self, layer: int, role: str):
        cfg = self.cfg
        from_shape = {"q": (cfg["n_q"] * cfg["head_dim"], cfg["d_model"]),
                      "k": (cfg["n_kv"] * cfg["head_dim"], cfg["d_model"]),
                      "v": (cfg["n_kv"] * cfg["head_dim"], cfg["d_model"]),
                      "o": (cfg["d_model"], cfg["n_q"] * cfg["head_dim"]),
                      "gate": (cfg["d_ff"], cfg["d_model"]), "up": (cfg["d_ff"], cfg["d_model"]),
                      "down": (cfg["d_model"], cfg["d_ff"]), "embed": (cfg["vocab"], cfg["d_model"])}
        n, k = from_shape[role]
        per = 16 if cfg["weight_bits"] == 4 else 32
        wq = np.empty((n, k // 32, per), np.uint8 if cfg["weight_bits"] == 4 else np.int8)
        ws = np.empty((n, k // 32), np.uint16)
        self.sess.check(lib().rstr_model_export_linear(self.h, layer, ROLE[role], _p(wq), _p(ws)))
        return wq, ws

    def close(self):
        if self.h:
            lib().rstr_model_close(self.h)
            self.h = None


class Pool:
    """fp16 page pool slabs (page-pool/open-pool! device side)."""

    def __init__(self, model: Model, page_size: int, physical_pages: int):
        self.model, self.sess = model, model.sess
        self.page_size, self.physical_pages = page_size, physical_pages
        h = C.c_void_p()
        self.sess.check(lib().rstr_pool_open(model.h, page_size, physical_pages, C.byref(h)))
        self.h = h
        self.sess._adopt(self)

    @property
    def page_elems(self) -> int:
        c = self.model.cfg
        return self.page_size * c["n_kv"] * c["head_dim"]

    def copy_page(self, src: int, dst: int):
        self.sess.check(lib().rstr_pool_copy_page(self.h, src, dst))

    def upload(self, slab: int, layer: int, dst_element: int, data: np.ndarray):
        data = np.ascontiguousarray(data).view(np.uint16).ravel()
        self.sess.check(lib().rstr_pool_upload(self.h, slab, layer, dst_element, _p(data), data.size))

    def download(self, slab: int, layer: int, src_element: int = 0, elements: int | None = None):
        if elements is None:
            elements = self.physical_pages * self.page_elems - src_element
        out = np.empty(elements, np.uint16)
        self.sess.check(lib().rstr_pool_download(self.h, slab, layer, src_element, _p(out), elements))
        return out

    def pages(self, slab: int, layer: int) -> np.ndarray:
        c = self.model.cfg
        return self.download(slab, layer).view(np.float16).reshape(
            self.physical_pages, self.page_size, c["n_kv"], c["head_dim"])

    def fill_synthetic(self, pages, seed: int):
        pages = _i32(pages)
        self.sess.check(lib().rstr_pool_fill_synthetic(self.h, _p(pages), pages.size, seed))

    def append(self, layer, k_rows, v_rows, slots):
        """Routed append (paged-append run!): f32 rows -> fp16 at the given slots."""
        k_rows, v_rows, slots = _f32(k_rows), _f32(v_rows), _i32(slots)
        self.sess.check(lib().rstr_append_run(self.h, layer, slots.size, _p(k_rows), _p(v_rows),
                                              _p(slots)))

    def chunk_elements(self, token_count: int) -> int:
        """Payload elements of a durable chunk of ``token_count`` tokens."""
        c = self.model.cfg
        return 2 * c["n_layers"] * token_count * c["n_kv"] * c["head_dim"]

    def export_submit(self, pages, start: int, token_count: int) -> "Transfer":
        """Gather tokens [start, start+token_count) of the route over ``pages`` into a
        durable fp16 payload (filled when the transfer completes)."""
        pages = _i32(pages).ravel()
        out = np.empty(self.chunk_elements(token_count), np.uint16)
        h = C.c_void_p()
        self.sess.check(lib().rstr_chunk_export_submit(self.h, _p(pages), pages.size, int(start), int(token_count),
                                                      _p(out), C.byref(h)))
        return Transfer(self.sess, h, out, (pages, out))

    def restore_submit(self, pages, start: int, token_count: int, payload) -> "Transfer":
        """Scatter a durable payload (fp16 bits as uint16, or float32) into the route's pages."""
        pages = _i32(pages).ravel()
        payload = np.ascontiguousarray(payload)
        if payload.dtype == np.float16:
            payload = payload.view(np.uint16)
        if payload.dtype == np.uint16:
            dtype = 0
        elif payload.dtype == np.float32:
            dtype = 1
        else:
            raise ValueError("Payload dtype and representation cannot be restored to FP16")
        if payload.size != self.chunk_elements(token_count):
            raise ValueError("payload length differs from its descriptor")
        h = C.c_void_p()
        self.sess.check(lib().rstr_chunk_restore_submit(self.h, _p(pages), pages.size, int(start), int(token_count),
                                                       _p(payload), dtype, C.byref(h)))
        return Transfer(self.sess, h, None, (pages, payload))

    def chunk_bench(self, pages, start: int, token_count: int, mode: int, iters: int) -> float:
        """Average ms of the gather (mode 0) / scatter (mode 1) kernel alone."""
        pages = _i32(pages).ravel()
        ms = C.c_float()
        self.sess.check(lib().rstr_chunk_bench(self.h, _p(pages), pages.size, int(start), int(token_count),
                                               int(mode), int(iters), C.byref(ms)))
        return ms.value

    def attention(self, layer, q, page_table, lengths, start_positions=None, positions=None,
                  window=0, scale=None, split=256, static=False):
        """Isolated routed attention (paged-attention/run!) with f32 q/out;
        ``static`` selects the allocation-free entry (rstr_attention_run_static)."""
        c = self.model.cfg
        q = _f32(q)
        B, n_q, hd = q.shape
        lengths = _i32(lengths)
        starts = _i32(start_positions if start_positions is not None else np.zeros(B))
        if positions is None:
            positions = np.where(lengths > 0, starts + lengths - 1, 0)
        pos = _i32(positions)
        pt = _i32(page_table)
        rows = _i32(np.arange(B + 1))
        out = np.empty_like(q)
        scale = c["attn_scale"] if scale is None else scale
        fn = lib().rstr_attention_run_static if static else lib().rstr_attention_run
        self.sess.check(fn(self.h, layer, B, n_q, split, window, scale, _p(q), _p(rows), _p(pos), _p(pt),
                           pt.shape[1], _p(lengths), _p(starts), _p(out)))
        return out

    def attention_bench(self, layer, q, page_table, lengths, window=0, scale=None, split=256,
                        iters=20):
        c = self.model.cfg
        q = _f32(q)
        B, n_q, hd = q.shape
        pt, lengths = _i32(page_table), _i32(lengths)
        a, b = C.c_float(), C.c_float()
        scale = c["attn_scale"] if scale is None else scale
        self.sess.check(lib().rstr_attention_bench(self.h, layer, B, n_q, split, window, scale, _p(q),
                                                   _p(pt), pt.shape[1], _p(lengths), iters,
                                                   C.byref(a), C.byref(b)))
        return a.value, b.value

    def close(self):
        """Frees the slabs; refused (RstrError) while chunk transfers are in flight."""
        if self.h:
            self.sess.check(lib().rstr_pool_close(self.h))
            self.h = None


class Transfer:
    """A submitted chunk export/restore; keeps its host buffers alive until completion."""

    def __init__(self, sess: Session, h, payload, retained):
        self.sess, self.h, self.payload, self._retained = sess, h, payload, retained

    def done(self) -> bool:
        if self.h is None:  # completed
            return True
        rc = lib().rstr_transfer_done(self.h)
        if rc < 0:
            self.sess.check(rc)
        return rc == 1

    def complete(self) -> dict:
        """Wait, release the transfer; returns {bytes, device_ms, direction, payload}."""
        if self.h is None:
            raise RstrError(-4, "transfer already completed")
        st = TransferStats()
        h, self.h = self.h, None
        self.sess.check(lib().rstr_transfer_complete(h, C.byref(st)))
        self._retained = None
        return {"bytes": int(st.bytes), "device_ms": float(st.device_ms),
                "direction": "download" if st.direction == 1 else "upload", "payload": self.payload}


class Decoder:
    """Paged lane decoder (paged-decoder/open! + step-lanes!)."""

    def __init__(self, model: Model, pool: Pool, batch: int, pages_per_seq: int, maxpos: int,
                 split: int = 256):
        self.model, self.pool, self.sess = model, pool, model.sess
        self.batch, self.pps, self.maxpos, self.split = batch, pages_per_seq, maxpos, split
        h = C.c_void_p()
        self.sess.check(lib().rstr_decoder_open(model.h, pool.h, batch, pages_per_seq, maxpos, split,
                                                C.byref(h)))
        self.h = h
        self._keep = []
        self.sess._adopt(self)

    def set_graph(self, enabled: bool):
        self.sess.check(lib().rstr_decoder_set_graph(self.h, 1 if enabled else 0))

    STEP_TIMING = ("validate", "prior_sync", "pack", "enqueue", "device_wait", "handback", "call", "device_step")

    def step_timing(self) -> dict:
        """Phases (ms) of the last step_lanes call (rstr_decoder_step_timing)."""
        out = np.zeros(len(self.STEP_TIMING), np.float64)
        self.sess.check(lib().rstr_decoder_step_timing(self.h, _p(out), out.size))
        return dict(zip(self.STEP_TIMING, out.tolist()))

    def prime_lanes(self, lanes, tokens):
        lanes, tokens = _i32(lanes), _i32(tokens)
        self.sess.check(lib().rstr_prime_lanes(self.h, lanes.size, _p(lanes), _p(tokens)))

    def prime_rows(self, lanes, rows):
        lanes, rows = _i32(lanes), _f32(rows)
        self.sess.check(lib().rstr_prime_rows(self.h, lanes.size, _p(lanes), _p(rows)))

    def step_lanes(self, slots, row_offsets, positions, page_table, lengths, start_positions):
        args = [_i32(a) for a in (slots, row_offsets, positions, page_table, lengths, start_positions)]
        out = np.empty(self.batch, np.int32)
        self.sess.check(lib().rstr_step_lanes(self.h, *[_p(a) for a in args], _p(out)))
        return out

    def step_lanes_submit(self, slots, row_offsets, positions, page_table, lengths, start_positions):
        """Enqueue one step without waiting (rstr_step_lanes_submit); at most two in flight."""
        args = [_i32(a) for a in (slots, row_offsets, positions, page_table, lengths, start_positions)]
        self.sess.check(lib().rstr_step_lanes_submit(self.h, *[_p(a) for a in args]))

    def step_lanes_collect(self) -> np.ndarray:
        """Tokens of the oldest submitted step (rstr_step_lanes_collect)."""
        out = np.empty(self.batch, np.int32)
        self.sess.check(lib().rstr_step_lanes_collect(self.h, _p(out)))
        return out

    def logits(self) -> np.ndarray:
        out = np.empty((self.batch, self.model.cfg["vocab"]), np.float32)
        self.sess.check(lib().rstr_decode_logits(self.h, _p(out)))
        return out

    def rows(self) -> np.ndarray:
        out = np.empty((self.batch, self.model.cfg["d_model"]), np.float32)
        self.sess.check(lib().rstr_decoder_read_rows(self.h, _p(out)))
        return out

    def schedule_upload(self, steps):
        """steps: list of dicts with the six descriptors (+ optional fill_pages, fill_seed,
        cow_pairs)."""
        keep = []
        arr = (StagedStep * len(steps))()
        for i, st in enumerate(steps):
            f = {}
            for k in ("slots", "row_offsets", "positions", "page_table", "lengths", "start_positions"):
                a = _i32(st[k])
                keep.append(a)
                f[k] = a.ctypes.data
            fill = _i32(st.get("fill_pages", []))
            cow = _i32(st.get("cow_pairs", np.zeros((0, 2))))
            pl = _i32(st.get("prime_lanes", []))
            ptk = _i32(st.get("prime_tokens", []))
            keep += [fill, cow, pl, ptk]
            arr[i] = StagedStep(f["slots"], f["row_offsets"], f["positions"], f["page_table"],
                                f["lengths"], f["start_positions"],
                                fill.ctypes.data if fill.size else None, fill.size,
                                int(st.get("fill_seed", 0)),
                                cow.ctypes.data if cow.size else None, cow.size // 2,
                                pl.ctypes.data if pl.size else None,
                                ptk.ctypes.data if ptk.size else None, pl.size)
        self.sess.check(lib().rstr_schedule_upload(self.h, C.cast(arr, C.c_void_p), len(steps)))
        self._keep = keep

    def schedule_run(self, first: int, count: int):
        out = np.empty((count, self.batch), np.int32)
        ms = C.c_float()
        self.sess.check(lib().rstr_schedule_run(self.h, first, count, _p(out), C.byref(ms)))
        return out, ms.value

    def profile_steps(self, first: int, count: int):
        ms = np.zeros(len(KERNEL_CLASSES), np.float32)
        n = np.zeros(len(KERNEL_CLASSES), np.int32)
        self.sess.check(lib().rstr_decoder_profile_steps(self.h, first, count, _p(ms), _p(n)))
        return {k: (float(ms[i]), int(n[i])) for i, k in enumerate(KERNEL_CLASSES)}

    def close(self):
        if self.h:
            lib().rstr_decoder_close(self.h)
            self.h = None


class Prefill:
    """Bulk-prefill decoder over ``rows`` tile rows (the ``:prefill-T`` link of
    paged-decoder/open!, layers only) and prefill-range!'s run."""

    def __init__(self, model: Model, pool: Pool, rows: int, pages_per_seq: int, maxpos: int,
                 split: int = 256):
        self.model, self.pool, self.sess = model, pool, model.sess
        self.rows, self.pps, self.maxpos, self.split = rows, pages_per_seq, maxpos, split
        h = C.c_void_p()
        self.sess.check(lib().rstr_prefill_open(model.h, pool.h, rows, pages_per_seq, maxpos, split,
                                                C.byref(h)))
        self.h = h
        self.sess._adopt(self)

    def set_graph(self, enabled: bool):
        self.sess.check(lib().rstr_decoder_set_graph(self.h, 1 if enabled else 0))

    def prefill_range(self, tokens, slots, positions, page_table, length: int, start_position: int):
        tokens, slots, positions, page_table = (_i32(a).ravel() for a in (tokens, slots, positions, page_table))
        if tokens.size != self.rows or slots.size != self.rows or positions.size != self.rows:
            raise ValueError("Prompt tile does not match the bound prefill row count")
        if page_table.size != self.pps:
            raise ValueError("page table row does not match pages_per_seq")
        self.sess.check(lib().rstr_prefill_range(self.h, _p(tokens), _p(slots), _p(positions),
                                                 _p(page_table), int(length), int(start_position)))

    def rows_out(self) -> np.ndarray:
        """The tile's final hidden rows [rows][d_model] (before the head)."""
        out = np.empty((self.rows, self.model.cfg["d_model"]), np.float32)
        self.sess.check(lib().rstr_decoder_read_rows(self.h, _p(out)))
        return out

    def close(self):
        if self.h:
            lib().rstr_decoder_close(self.h)
            self.h = None
