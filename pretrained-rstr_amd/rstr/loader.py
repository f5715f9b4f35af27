"""HF checkpoint ingestion for the resident decoder.

Mirrors ``load-hf`` (``src/pretrained/decoder.clj:31-56``), the architecture
descriptors (``src/pretrained/arch/gemma3.clj:8-37``, ``arch/qwen3.clj:20-45``,
``arch/llama.clj:22-45``: role -> tensor-name templates and flags) and
``load-lm {:gpu? true}`` (``src/pretrained/lm.clj:28-49``): a model directory
(``config.json`` + ``model.safetensors``, or shards listed by
``model.safetensors.index.json``) becomes a resident quantised model.

The reference converts every tensor to a host float array, quantises on the
CPU and caches the packed stream on disk (``quantize-stream`` and its "QSTR"
cache, decoder.clj:92-189) because that quantisation takes ~30 s.  Here the
files are memory-mapped and each tensor goes to the device in its stored dtype
(``rstr_model_bind_raw``), where it is widened exactly and packed by the same
Q4/Q8 kernel as every other bind -- no host f32 copy of the model, and no
quantisation pass long enough to be worth caching.
"""
from __future__ import annotations

import json
import math
import os

from . import safetensors as st

# role of this build (``hip.ROLE``) <- reference role (decoder descriptors)
ROLES = {"embed": "embed", "final-norm": "final_norm", "attn-q": "q", "attn-k": "k", "attn-v": "v",
         "attn-o": "o", "attn-q-norm": "q_norm", "attn-k-norm": "k_norm", "attn-norm": "attn_norm",
         "attn-post-norm": "post_attn_norm", "ffn-pre-norm": "ffn_pre_norm", "ffn-post-norm": "ffn_post_norm",
         "ffn-gate": "gate", "ffn-up": "up", "ffn-down": "down"}

_L = "layers.%d."
DESCRIPTORS = {
    "gemma3": {
        "hf-arch": {"gemma3_text", "Gemma3ForCausalLM", "Gemma3ForConditionalGeneration", "gemma3"},
        "names": {"embed": "embed_tokens.weight", "final-norm": "norm.weight",
                  "attn-q": _L + "self_attn.q_proj.weight", "attn-k": _L + "self_attn.k_proj.weight",
                  "attn-v": _L + "self_attn.v_proj.weight", "attn-o": _L + "self_attn.o_proj.weight",
                  "attn-q-norm": _L + "self_attn.q_norm.weight", "attn-k-norm": _L + "self_attn.k_norm.weight",
                  "attn-norm": _L + "input_layernorm.weight",
                  "attn-post-norm": _L + "post_attention_layernorm.weight",
                  "ffn-pre-norm": _L + "pre_feedforward_layernorm.weight",
                  "ffn-post-norm": _L + "post_feedforward_layernorm.weight",
                  "ffn-gate": _L + "mlp.gate_proj.weight", "ffn-up": _L + "mlp.up_proj.weight",
                  "ffn-down": _L + "mlp.down_proj.weight"},
        "flags": {"gain-offset": 1, "embed-scale-sqrt-d": 1, "qk-norm": 1, "sandwich": 1, "geglu": 1,
                  "rope-dual": 1, "global-layer-pattern": 6, "sliding-window": 512},
        "bits": 4},
    "qwen3": {
        "hf-arch": {"qwen3", "Qwen3ForCausalLM"},
        "names": {"embed": "embed_tokens.weight", "final-norm": "norm.weight",
                  "attn-q": _L + "self_attn.q_proj.weight", "attn-k": _L + "self_attn.k_proj.weight",
                  "attn-v": _L + "self_attn.v_proj.weight", "attn-o": _L + "self_attn.o_proj.weight",
                  "attn-q-norm": _L + "self_attn.q_norm.weight", "attn-k-norm": _L + "self_attn.k_norm.weight",
                  "attn-norm": _L + "input_layernorm.weight",
                  "ffn-pre-norm": _L + "post_attention_layernorm.weight",
                  "ffn-gate": _L + "mlp.gate_proj.weight", "ffn-up": _L + "mlp.up_proj.weight",
                  "ffn-down": _L + "mlp.down_proj.weight"},
        "flags": {"gain-offset": 0, "embed-scale-sqrt-d": 0, "qk-norm": 1, "sandwich": 0, "geglu": 0,
                  "rope-dual": 0, "global-layer-pattern": 0, "sliding-window": 0},
        "bits": 8},   # qwen3.clj:47-50 quantises Qwen3 to Q8
    "llama": {
        "hf-arch": {"llama", "LlamaForCausalLM"},
        "names": {"embed": "embed_tokens.weight", "final-norm": "norm.weight",
                  "attn-q": _L + "self_attn.q_proj.weight", "attn-k": _L + "self_attn.k_proj.weight",
                  "attn-v": _L + "self_attn.v_proj.weight", "attn-o": _L + "self_attn.o_proj.weight",
                  "attn-norm": _L + "input_layernorm.weight",
                  "ffn-pre-norm": _L + "post_attention_layernorm.weight",
                  "ffn-gate": _L + "mlp.gate_proj.weight", "ffn-up": _L + "mlp.up_proj.weight",
                  "ffn-down": _L + "mlp.down_proj.weight"},
        "flags": {"gain-offset": 0, "embed-scale-sqrt-d": 0, "qk-norm": 0, "sandwich": 0, "geglu": 0,
                  "rope-dual": 0, "global-layer-pattern": 0, "sliding-window": 0},
        "bits": 4},
}


class LoaderError(ValueError):
    pass


def _weights(dir_: str) -> dict:
    """name (without the optional "model." prefix, decoder.clj:39-44) -> (lazy file, stored name)."""
    index = os.path.join(dir_, "model.safetensors.index.json")
    if os.path.exists(index):
        files = sorted(set(json.load(open(index))["weight_map"].values()))
    else:
        files = ["model.safetensors"]
    out = {}
    for f in files:
        lazy = st.load_safetensors_lazy(os.path.join(dir_, f))
        for name in lazy["tensors"]:
            out[name[6:] if name.startswith("model.") else name] = (lazy, name)
    return out


def load_hf(dir_: str) -> dict:
    """decoder.clj:31-56: hyper-parameters from config.json (optional fields
    default as there), weights by normalised name (mapped, not read)."""
    cfg = json.load(open(os.path.join(dir_, "config.json")))
    if "text_config" in cfg and "num_hidden_layers" not in cfg:
        cfg = dict(cfg["text_config"], architectures=cfg.get("architectures"), model_type=cfg.get("model_type"))
    head_dim = cfg.get("head_dim") or cfg["hidden_size"] // cfg["num_attention_heads"]
    return {"config": cfg, "dir": dir_, "weights": _weights(dir_),
            "n-layers": cfg["num_hidden_layers"], "d-model": cfg["hidden_size"],
            "d-ff": cfg["intermediate_size"], "n-q": cfg["num_attention_heads"],
            "n-kv": cfg.get("num_key_value_heads") or cfg["num_attention_heads"], "head-dim": head_dim,
            "vocab": cfg["vocab_size"], "eps": float(cfg.get("rms_norm_eps") or 1.0e-6),
            "rope-global": float(cfg.get("rope_theta") or 10000.0),
            "rope-local": float(cfg.get("rope_local_base_freq") or 10000.0),
            "attn-scale": 1.0 / math.sqrt(float(cfg.get("query_pre_attn_scalar") or head_dim))}


def architecture(hf: dict) -> str:
    """The registered architecture of a checkpoint (loader registry by HF arch,
    arch/*.clj register-architecture!)."""
    cfg = hf["config"]
    keys = {cfg.get("model_type")} | set(cfg.get("architectures") or [])
    for name, d in DESCRIPTORS.items():
        if keys & d["hf-arch"]:
            return name
    raise LoaderError(f"unsupported architecture {sorted(k for k in keys if k)}")


def model_config(hf: dict, arch: str, bits: int | None = None) -> dict:
    """The ``rstr_model_desc`` fields of this checkpoint (hyper-parameters of
    load-hf plus the descriptor flags)."""
    f = DESCRIPTORS[arch]["flags"]
    cfg = {"n_layers": hf["n-layers"], "d_model": hf["d-model"], "d_ff": hf["d-ff"], "n_q": hf["n-q"],
           "n_kv": hf["n-kv"], "head_dim": hf["head-dim"], "vocab": hf["vocab"],
           "weight_bits": bits or DESCRIPTORS[arch]["bits"], "gain_offset": f["gain-offset"],
           "qk_norm": f["qk-norm"], "sandwich": f["sandwich"], "ffn_geglu": f["geglu"],
           "rope_dual": f["rope-dual"], "global_pattern": f["global-layer-pattern"],
           "sliding_window": f["sliding-window"], "embed_scale_sqrt_d": f["embed-scale-sqrt-d"],
           "eps": hf["eps"], "attn_scale": hf["attn-scale"], "rope_global": hf["rope-global"],
           "rope_local": hf["rope-local"] if f["rope-dual"] else hf["rope-global"]}
    return cfg


def raw_tensors(hf: dict, arch: str) -> list:
    """(layer, role, stored dtype, mapped view) for every tensor the descriptor
    names (role-name, decoder.clj:62-69); layer -1 for globals."""
    names = DESCRIPTORS[arch]["names"]
    out = []
    for role, tmpl in names.items():
        layers = range(hf["n-layers"]) if "%d" in tmpl else [None]
        for layer in layers:
            name = tmpl % layer if layer is not None else tmpl
            entry = hf["weights"].get(name)
            if entry is None:
                raise LoaderError(f"checkpoint has no tensor {name}")
            lazy, stored = entry
            dtype = lazy["tensors"][stored]["dtype"]
            if dtype not in ("F32", "F16", "BF16"):
                raise LoaderError(f"tensor {name}: unsupported dtype {dtype}")
            out.append((-1 if layer is None else layer, ROLES[role], dtype, st.tensor_view(lazy, stored)))
    return out


def bind_hf(sess, dir_: str, bits: int | None = None):
    """load-lm {:gpu? true} (lm.clj:28-49): map the checkpoint and bind it to
    the device.  Returns (hip.Model, cfg)."""
    from . import hip
    hf = load_hf(dir_)
    arch = architecture(hf)
    cfg = model_config(hf, arch, bits)
    return hip.Model(sess, cfg, raw_tensors=raw_tensors(hf, arch)), cfg
