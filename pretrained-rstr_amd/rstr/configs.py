"""Model descriptors of the benchmark configurations.

The field set mirrors ``rstr_model_desc`` (include/rstr_hip.h), which is the data
form of the reference's architecture descriptors:
``src/pretrained/arch/gemma3.clj:29-37``, ``arch/qwen3.clj:87-93`` and
``arch/llama.clj:142-148`` plus the HF hyper-parameters read by
``src/pretrained/decoder.clj:31-56``.
"""
from __future__ import annotations

import math

FIELDS = ("n_layers", "d_model", "d_ff", "n_q", "n_kv", "head_dim", "vocab", "weight_bits",
          "gain_offset", "qk_norm", "sandwich", "ffn_geglu", "rope_dual", "global_pattern",
          "sliding_window", "embed_scale_sqrt_d", "eps", "attn_scale", "rope_global", "rope_local")


def _desc(**kw) -> dict:
    base = dict(weight_bits=4, gain_offset=0, qk_norm=0, sandwich=0, ffn_geglu=0, rope_dual=0,
                global_pattern=0, sliding_window=0, embed_scale_sqrt_d=0, eps=1e-6,
                rope_global=10000.0, rope_local=10000.0)
    base.update(kw)
    base.setdefault("attn_scale", 1.0 / math.sqrt(base["head_dim"]))
    missing = [f for f in FIELDS if f not in base]
    assert not missing, missing
    return base


# Gemma-3-270M shape (gemma3.clj flags: gain offset 1, embed scale sqrt(d), qk-norm,
# sandwich norms, GeGLU, dual RoPE, every 6th layer global, sliding window 512).
GEMMA3_270M = _desc(n_layers=18, d_model=640, d_ff=2048, n_q=4, n_kv=1, head_dim=256, vocab=262144,
                    gain_offset=1, qk_norm=1, sandwich=1, ffn_geglu=1, rope_dual=1,
                    global_pattern=6, sliding_window=512, embed_scale_sqrt_d=1, eps=1e-6,
                    attn_scale=1.0 / math.sqrt(256.0), rope_global=1e6, rope_local=1e4)

# Qwen3-0.6B shape (qwen3.clj: plain RMSNorm, qk-norm, SwiGLU, single RoPE 1e6).
QWEN3_06B = _desc(n_layers=28, d_model=1024, d_ff=3072, n_q=16, n_kv=8, head_dim=128, vocab=151936,
                  qk_norm=1, eps=1e-6, rope_global=1e6, rope_local=1e6)

# Llama-3-8B shape (llama.clj: plain RMSNorm, SwiGLU, single RoPE), theta 500000, eps 1e-5.
LLAMA3_8B = _desc(n_layers=32, d_model=4096, d_ff=14336, n_q=32, n_kv=8, head_dim=128, vocab=128256,
                  eps=1e-5, rope_global=500000.0, rope_local=500000.0)

# Small shapes with the same flag sets, for parity runs the CPU oracle finishes quickly.
TINY_GEMMA = _desc(n_layers=3, d_model=256, d_ff=512, n_q=4, n_kv=1, head_dim=64, vocab=1024,
                   gain_offset=1, qk_norm=1, sandwich=1, ffn_geglu=1, rope_dual=1, global_pattern=3,
                   sliding_window=24, embed_scale_sqrt_d=1, attn_scale=1.0 / 8.0, rope_global=1e6,
                   rope_local=1e4)
TINY_QWEN = _desc(n_layers=2, d_model=256, d_ff=384, n_q=4, n_kv=2, head_dim=128, vocab=2048,
                  qk_norm=1, rope_global=1e6, rope_local=1e6)
TINY_LLAMA = _desc(n_layers=2, d_model=256, d_ff=512, n_q=8, n_kv=2, head_dim=64, vocab=2048,
                   eps=1e-5, rope_global=500000.0, rope_local=500000.0)

MODELS = {"gemma3_270m": GEMMA3_270M, "qwen3_06b": QWEN3_06B, "llama3_8b": LLAMA3_8B,
          "tiny_gemma": TINY_GEMMA, "tiny_qwen": TINY_QWEN, "tiny_llama": TINY_LLAMA}


def with_bits(cfg: dict, bits: int) -> dict:
    out = dict(cfg)
    out["weight_bits"] = bits
    return out
