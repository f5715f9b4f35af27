"""ctypes wrapper of the CPU oracle (``liboracle.so``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg, always as the checker or the timed CPU
baseline, never as a product path.  See ``rstr_oracle.h`` for the reference
citations of each function.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

ROLE = dict(embed=0, final_norm=1, attn_norm=2, q=3, k=4, v=5, o=6, q_norm=7, k_norm=8,
            post_attn_norm=9, ffn_pre_norm=10, ffn_post_norm=11, gate=12, up=13, down=14)


class Desc(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n_layers", "d_model", "d_ff", "n_q", "n_kv", "head_dim", "vocab", "weight_bits",
        "gain_offset", "qk_norm", "sandwich", "ffn_geglu", "rope_dual", "global_pattern",
        "sliding_window", "embed_scale_sqrt_d")] + [
        ("eps", C.c_float), ("attn_scale", C.c_float),
        ("rope_global", C.c_double), ("rope_local", C.c_double)]


def make_desc(cfg: dict) -> Desc:
    d = Desc()
    for name, _ in Desc._fields_:
        setattr(d, name, cfg[name])
    return d


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        i32, i64, u64, f32, f64 = C.c_int32, C.c_int64, C.c_uint64, C.c_float, C.c_double
        sig = {
            "orc_f32_to_f16": (C.c_uint16, [f32]),
            "orc_f16_to_f32": (f32, [C.c_uint16]),
            "orc_exp": (f32, [f32]),
            "orc_gelu_tanh": (f32, [f32]),
            "orc_silu": (f32, [f32]),
            "orc_splitmix64": (u64, [u64]),
            "orc_tensor_key": (u64, [u64, i32, i32]),
            "orc_normal": (f32, [u64, u64, f64, f64]),
            "orc_normal_fill": (None, [u64, u64, i64, f64, f64, P]),
            "orc_quant_q4": (None, [P, i64, i64, P, P]),
            "orc_quant_q8": (None, [P, i64, i64, P, P]),
            "orc_act_scale": (f32, [f32]),
            "orc_set_act_scale_plain": (None, [i32]),
            "orc_quant_act": (None, [P, i32, i32, P, P]),
            "orc_qlinear": (None, [i32, P, P, i32, i32, P, P, i32, P]),
            "orc_sumsq": (f32, [P, i32]),
            "orc_rmsnorm": (None, [P, P, f32, f32, i32, i32, P]),
            "orc_rope_table": (None, [f64, i32, i32, P, P]),
            "orc_rope": (None, [P, i32, i32, i32, P, P, P, P]),
            "orc_dot_canon": (f32, [P, P, i32, i32]),
            "orc_attention": (None, [P, P, P, i32, i32, i32, i32, i32, i32, P, i32, P, i32, f32,
                                     i32, P]),
            "orc_argmax_rows": (None, [P, i32, i32, P]),
            "orc_model_synthetic": (P, [P, u64]),
            "orc_model_free": (None, [P]),
            "orc_model_set_tensor": (i32, [P, i32, i32, P, i64]),
            "orc_model_tensor": (i64, [P, i32, i32, P, P]),
            "orc_model_norm": (i64, [P, i32, i32, P]),
            "orc_embed_row": (None, [P, i32, P]),
            "orc_decoder_open": (P, [P, i32, i32, i32, i32, i32, i32, i32]),
            "orc_decoder_free": (None, [P]),
            "orc_prime_lanes": (None, [P, i32, P, P]),
            "orc_prime_rows": (None, [P, i32, P, P]),
            "orc_step_lanes": (i32, [P, P, P, P, P, P, P, P]),
            "orc_logits": (P, [P]),
            "orc_r0": (P, [P]),
            "orc_copy_page": (None, [P, i32, i32]),
            "orc_fill_synthetic": (None, [P, i32, u64]),
            "orc_slab": (P, [P, i32, i32]),
            "orc_last_error": (C.c_char_p, []),
            "orc_num_threads": (C.c_int, []),
            "orc_stream_triad": (C.c_double, [C.c_int64, C.c_int32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


# ---- numerics --------------------------------------------------------------

def f32_to_f16_bits(x) -> np.ndarray:
    x = f32(x).ravel()
    return np.array([lib().orc_f32_to_f16(float(v)) for v in x], dtype=np.uint16)


def exp(x: float) -> float:
    return lib().orc_exp(float(x))


def normal(key: int, start: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_normal_fill(key, start, n, mean, std, ptr(out))
    return out


def tensor_key(seed: int, layer: int, role: int) -> int:
    return lib().orc_tensor_key(seed, layer, role)


def quant_q4(w: np.ndarray):
    w = f32(w)
    rows, cols = w.shape
    nib = np.empty((rows, cols // 32, 16), np.uint8)
    sc = np.empty((rows, cols // 32), np.uint16)
    lib().orc_quant_q4(ptr(w), rows, cols, ptr(nib), ptr(sc))
    return nib, sc


def quant_q8(w: np.ndarray):
    w = f32(w)
    rows, cols = w.shape
    q = np.empty((rows, cols // 32, 32), np.int8)
    sc = np.empty((rows, cols // 32), np.uint16)
    lib().orc_quant_q8(ptr(w), rows, cols, ptr(q), ptr(sc))
    return q, sc


def quant_act(x: np.ndarray):
    x = f32(x)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty((rows, cols // 32), np.float32)
    lib().orc_quant_act(ptr(x), rows, cols, ptr(q), ptr(s))
    return q, s


def qlinear(bits: int, wq: np.ndarray, ws: np.ndarray, xq: np.ndarray, xs: np.ndarray) -> np.ndarray:
    n_out = ws.shape[0]
    rows, k_in = xq.shape
    if k_in % 128:
        raise ValueError("input width must be a multiple of 128 (4 quarters of 32-blocks)")
    y = np.empty((rows, n_out), np.float32)
    lib().orc_qlinear(bits, ptr(np.ascontiguousarray(wq)), ptr(np.ascontiguousarray(ws)), n_out, k_in,
                      ptr(np.ascontiguousarray(xq)), ptr(f32(xs)), rows, ptr(y))
    return y


def rmsnorm(x: np.ndarray, g: np.ndarray, gain_offset: float, eps: float) -> np.ndarray:
    x = f32(x)
    rows, n = x.shape
    y = np.empty_like(x)
    lib().orc_rmsnorm(ptr(x), ptr(f32(g)), gain_offset, eps, rows, n, ptr(y))
    return y


def rope_table(theta: float, hd: int, maxpos: int):
    c = np.empty((maxpos, hd // 2), np.float32)
    s = np.empty((maxpos, hd // 2), np.float32)
    lib().orc_rope_table(theta, hd, maxpos, ptr(c), ptr(s))
    return c, s


def rope(x: np.ndarray, pos, cos_t, sin_t) -> np.ndarray:
    x = f32(x)
    rows, heads, hd = x.shape
    y = np.empty_like(x)
    lib().orc_rope(ptr(x), rows, heads, hd, ptr(i32(pos)), ptr(f32(cos_t)), ptr(f32(sin_t)), ptr(y))
    return y


def attention(q, kpages, vpages, page_table, lengths, window: int, scale: float, split: int):
    """q: [B, n_q, hd] f32; pages: [P, page_size, n_kv, hd] (float16 or float32)."""
    q = f32(q)
    B, n_q, hd = q.shape
    P, ps, n_kv, hd2 = kpages.shape
    assert hd2 == hd
    kv_f16 = 1 if kpages.dtype == np.float16 else 0
    kp = np.ascontiguousarray(kpages)
    vp = np.ascontiguousarray(vpages)
    pt = i32(page_table)
    out = np.empty((B, n_q, hd), np.float32)
    lib().orc_attention(ptr(q), ptr(kp), ptr(vp), kv_f16, ps, n_kv, hd, n_q, B, ptr(pt), pt.shape[1],
                        ptr(i32(lengths)), window, scale, split, ptr(out))
    return out


def argmax_rows(logits: np.ndarray) -> np.ndarray:
    logits = f32(logits)
    rows, vocab = logits.shape
    out = np.empty(rows, np.int32)
    lib().orc_argmax_rows(ptr(logits), rows, vocab, ptr(out))
    return out


# ---- model / decoder ---------------------------------------------------------

class Model:
    def __init__(self, cfg: dict, seed: int):
        self.cfg = dict(cfg)
        self.seed = seed
        self._desc = make_desc(cfg)
        self.h = lib().orc_model_synthetic(C.byref(self._desc), seed)
        if not self.h:
            raise ValueError(lib().orc_last_error().decode())

    def close(self):
        if self.h:
            lib().orc_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor(self, layer: int, role: str):
        cfg = self.cfg
        nb_bytes = lib().orc_model_tensor(self.h, layer, ROLE[role], None, None)
        if nb_bytes < 0:
            raise KeyError(role)
        n, k = linear_shape(cfg, role)
        per = 16 if cfg["weight_bits"] == 4 else 32
        dt = np.uint8 if cfg["weight_bits"] == 4 else np.int8
        wq = np.empty((n, k // 32, per), dt)
        ws = np.empty((n, k // 32), np.uint16)
        lib().orc_model_tensor(self.h, layer, ROLE[role], ptr(wq), ptr(ws))
        return wq, ws

    def set_tensor(self, layer: int, role: str, values) -> None:
        """Replace one tensor by host values (e.g. a checkpoint's, widened to f32)."""
        v = f32(values).ravel()
        if lib().orc_model_set_tensor(self.h, layer, ROLE[role], ptr(v), v.size) != 0:
            raise ValueError(f"tensor {role} of layer {layer}: unknown role or {v.size} elements do not fit")

    def norm(self, layer: int, role: str) -> np.ndarray:
        n = lib().orc_model_norm(self.h, layer, ROLE[role], None)
        if n < 0:
            raise KeyError(role)
        out = np.empty(n, np.float32)
        lib().orc_model_norm(self.h, layer, ROLE[role], ptr(out))
        return out

    def embed_row(self, token: int) -> np.ndarray:
        out = np.empty(self.cfg["d_model"], np.float32)
        lib().orc_embed_row(self.h, token, ptr(out))
        return out


def linear_shape(cfg: dict, role: str):
    d, ff, qd, kvr = cfg["d_model"], cfg["d_ff"], cfg["n_q"] * cfg["head_dim"], cfg["n_kv"] * cfg["head_dim"]
    return {"q": (qd, d), "k": (kvr, d), "v": (kvr, d), "o": (d, qd), "gate": (ff, d), "up": (ff, d),
            "down": (d, ff), "embed": (cfg["vocab"], d)}[role]


class Decoder:
    """Oracle twin of the C-ABI paged decoder (same descriptors, same results)."""

    def __init__(self, model: Model, batch: int, page_size: int, physical_pages: int,
                 pages_per_seq: int, maxpos: int, kv_f16: bool = True, split: int = 256):
        self.model = model
        self.batch, self.page_size, self.physical_pages = batch, page_size, physical_pages
        self.pps, self.maxpos, self.kv_f16, self.split = pages_per_seq, maxpos, kv_f16, split
        self.h = lib().orc_decoder_open(model.h, batch, page_size, physical_pages, pages_per_seq,
                                        maxpos, 1 if kv_f16 else 0, split)
        if not self.h:
            raise ValueError(lib().orc_last_error().decode())

    def close(self):
        if self.h:
            lib().orc_decoder_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prime_lanes(self, lanes, tokens):
        lanes, tokens = i32(lanes), i32(tokens)
        lib().orc_prime_lanes(self.h, len(lanes), ptr(lanes), ptr(tokens))

    def prime_rows(self, lanes, rows):
        lanes, rows = i32(lanes), f32(rows)
        lib().orc_prime_rows(self.h, lanes.size, ptr(lanes), ptr(rows))

    def step_lanes(self, slots, row_offsets, positions, page_table, lengths, start_positions):
        out = np.empty(self.batch, np.int32)
        args = [i32(a) for a in (slots, row_offsets, positions, page_table, lengths, start_positions)]
        rc = lib().orc_step_lanes(self.h, *[ptr(a) for a in args], ptr(out))
        if rc != 0:
            raise ValueError(lib().orc_last_error().decode())
        return out

    def logits(self) -> np.ndarray:
        cfg = self.model.cfg
        p = lib().orc_logits(self.h)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)),
                                     shape=(self.batch, cfg["vocab"])).copy()

    def r0(self) -> np.ndarray:
        p = lib().orc_r0(self.h)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)),
                                     shape=(self.batch, self.model.cfg["d_model"])).copy()

    def copy_page(self, src: int, dst: int):
        lib().orc_copy_page(self.h, src, dst)

    def fill_synthetic(self, page: int, seed: int):
        lib().orc_fill_synthetic(self.h, page, seed)

    def slab(self, slab: int, layer: int) -> np.ndarray:
        cfg = self.model.cfg
        p = lib().orc_slab(self.h, slab, layer)
        dt = C.c_uint16 if self.kv_f16 else C.c_float
        shape = (self.physical_pages, self.page_size, cfg["n_kv"], cfg["head_dim"])
        arr = np.ctypeslib.as_array(C.cast(p, C.POINTER(dt)), shape=shape)
        return arr.view(np.float16) if self.kv_f16 else arr
