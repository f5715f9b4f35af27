"""Checkpoint ingestion on the GPU: a model bound from a mapped SafeTensors
checkpoint in its stored dtype (``rstr_model_bind_raw``: bf16 / f16 / f32
widened and packed on the device) equals the model bound from the f32 widening
of the same tensors (``rstr_model_bind``), whose packing the oracle pins: the
same packed weights (checked against the oracle quantiser) and the same greedy
tokens and logits, bit for bit, for Llama- (bf16, Q4), Qwen- (f16, Q8) and
Gemma-shaped (f32, Q4) checkpoints."""
import json
import os

import numpy as np
import pytest

import oracle as O
from rstr import hip, loader, safetensors as st

torch = pytest.importorskip("torch")
from safetensors.torch import save_file  # noqa: E402

pytestmark = pytest.mark.gpu

SHAPES = {
    "llama": ({"architectures": ["LlamaForCausalLM"], "model_type": "llama", "rope_theta": 500000.0,
               "rms_norm_eps": 1e-5}, torch.bfloat16),
    "qwen3": ({"architectures": ["Qwen3ForCausalLM"], "model_type": "qwen3", "rope_theta": 1e6,
               "head_dim": 64}, torch.float16),
    "gemma3": ({"architectures": ["Gemma3ForCausalLM"], "model_type": "gemma3_text", "rope_theta": 1e6,
                "rope_local_base_freq": 1e4, "head_dim": 64, "query_pre_attn_scalar": 64, "num_hidden_layers": 6},
               torch.float32),
}


def _write_checkpoint(d, arch):
    extra, dtype = SHAPES[arch]
    cfg = {"num_hidden_layers": 2, "hidden_size": 256, "intermediate_size": 512, "num_attention_heads": 4,
           "num_key_value_heads": 2, "vocab_size": 1024}
    cfg.update(extra)
    os.makedirs(d, exist_ok=True)
    json.dump(cfg, open(os.path.join(d, "config.json"), "w"))
    hd = cfg.get("head_dim") or cfg["hidden_size"] // cfg["num_attention_heads"]
    dm, ff, qd, kd = 256, 512, cfg["num_attention_heads"] * hd, cfg["num_key_value_heads"] * hd
    shapes = {"embed": (cfg["vocab_size"], dm), "final-norm": (dm,), "attn-q": (qd, dm), "attn-k": (kd, dm),
              "attn-v": (kd, dm), "attn-o": (dm, qd), "attn-q-norm": (hd,), "attn-k-norm": (hd,),
              "attn-norm": (dm,), "attn-post-norm": (dm,), "ffn-pre-norm": (dm,), "ffn-post-norm": (dm,),
              "ffn-gate": (ff, dm), "ffn-up": (ff, dm), "ffn-down": (dm, ff)}
    g = torch.Generator().manual_seed(11)
    ts = {}
    for role, tmpl in loader.DESCRIPTORS[arch]["names"].items():
        layers = range(cfg["num_hidden_layers"]) if "%d" in tmpl else [None]
        for l in layers:
            name = "model." + (tmpl % l if l is not None else tmpl)
            shp = shapes[role]
            t = torch.randn(*shp, generator=g) * (0.05 if len(shp) == 2 else 0.1)
            if len(shp) == 1 and arch != "gemma3":
                t = t + 1.0
            ts[name] = t.to(dtype).contiguous()
    save_file(ts, os.path.join(d, "model.safetensors"))


def _decode(m, cfg, steps=6):
    p = hip.Pool(m, 16, 8)
    d = hip.Decoder(m, p, 2, 4, 64, 16)
    d.prime_lanes([0, 1], [5, 17])
    toks, logits = [], []
    pt = np.array([[0, 1, 2, 3], [4, 5, 6, 7]], np.int32)
    for t in range(steps):
        slots = pt[:, t // 16] * 16 + t % 16
        toks.append(d.step_lanes(slots, [0, 1, 2], [t, t], pt.ravel(), [t + 1, t + 1], [0, 0]))
        logits.append(d.logits())
    d.close()
    p.close()
    return np.array(toks), np.array(logits)


@pytest.mark.parametrize("arch", ["llama", "qwen3", "gemma3"])
def test_checkpoint_bind_equals_the_f32_bind(tmp_path, arch):
    print("case loader", arch, flush=True)
    _write_checkpoint(str(tmp_path), arch)
    hf = loader.load_hf(str(tmp_path))
    assert loader.architecture(hf) == arch
    cfg = loader.model_config(hf, arch)
    raw = loader.raw_tensors(hf, arch)
    f32 = [(l, r, st.to_f32(v, dt)) for l, r, dt, v in raw]
    with hip.Session(0) as sess:
        m_raw, cfg2 = loader.bind_hf(sess, str(tmp_path))
        assert cfg2 == cfg
        m_f32 = hip.Model(sess, cfg, tensors=f32)
        quant = O.quant_q4 if cfg["weight_bits"] == 4 else O.quant_q8
        for l, r, w in f32:
            if r in ("q", "k", "v", "o", "gate", "up", "down", "embed"):
                a, b = m_raw.export_linear(l, r), m_f32.export_linear(l, r)
                ew, es = quant(np.asarray(w, np.float32).reshape(w.shape[0], -1))
                assert np.array_equal(a[0], ew) and np.array_equal(a[1], es), (l, r)
                assert np.array_equal(b[0], ew) and np.array_equal(b[1], es), (l, r)
        t1, g1 = _decode(m_raw, cfg)
        t2, g2 = _decode(m_f32, cfg)
        assert np.array_equal(t1, t2)
        assert np.array_equal(g1.view(np.uint32), g2.view(np.uint32))
        assert np.isfinite(g1).all()


def test_raw_bind_rejects_bad_tensors(tmp_path):
    print("case loader errors", flush=True)
    _write_checkpoint(str(tmp_path), "llama")
    hf = loader.load_hf(str(tmp_path))
    cfg = loader.model_config(hf, "llama")
    raw = loader.raw_tensors(hf, "llama")
    with hip.Session(0) as sess:
        with pytest.raises(hip.RstrError, match="size mismatch"):
            hip.Model(sess, cfg, raw_tensors=[(l, r, dt, v[:1] if r == "down" else v) for l, r, dt, v in raw])
        with pytest.raises(hip.RstrError, match="missing"):
            hip.Model(sess, cfg, raw_tensors=[t for t in raw if t[1] != "final_norm"])
        with pytest.raises(ValueError, match="BF16 tensor with float32"):
            hip.Model(sess, cfg, raw_tensors=[(l, r, dt, np.zeros(4, np.float32)) for l, r, dt, v in raw])
