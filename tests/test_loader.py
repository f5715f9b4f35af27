"""Checkpoint ingestion host side: the SafeTensors reader (``rstr.safetensors``,
mirroring safetensors.clj) against an independent writer (the ``safetensors``
package over torch tensors, bf16 included) and torch's own bf16/f16 -> f32
conversion; ``load-hf`` hyper-parameters, name normalisation, shards and the
architecture descriptors (``rstr.loader``)."""
import json
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")
from safetensors.torch import save_file  # noqa: E402

from rstr import loader, safetensors as st  # noqa: E402


def _tiny_llama_hf(d, dtype=torch.bfloat16, prefix="model.", shards=1, cfg_extra=None, drop=None):
    os.makedirs(d, exist_ok=True)
    cfg = {"architectures": ["LlamaForCausalLM"], "model_type": "llama", "num_hidden_layers": 2,
           "hidden_size": 256, "intermediate_size": 512, "num_attention_heads": 8, "num_key_value_heads": 2,
           "vocab_size": 2048, "rms_norm_eps": 1e-5, "rope_theta": 500000.0, "tie_word_embeddings": True}
    cfg.update(cfg_extra or {})
    json.dump(cfg, open(os.path.join(d, "config.json"), "w"))
    g = torch.Generator().manual_seed(7)
    ts = {}
    hd = cfg.get("head_dim") or cfg["hidden_size"] // cfg["num_attention_heads"]
    kvh = cfg["num_key_value_heads"] or cfg["num_attention_heads"]
    qd, kd, dm, ff = cfg["num_attention_heads"] * hd, kvh * hd, 256, 512
    ts[prefix + "embed_tokens.weight"] = torch.randn(2048, dm, generator=g) * 0.02
    ts[prefix + "norm.weight"] = 1 + torch.randn(dm, generator=g) * 0.02
    for l in range(2):
        p = f"{prefix}layers.{l}."
        for nm, shp in (("self_attn.q_proj", (qd, dm)), ("self_attn.k_proj", (kd, dm)),
                        ("self_attn.v_proj", (kd, dm)), ("self_attn.o_proj", (dm, qd)),
                        ("mlp.gate_proj", (ff, dm)), ("mlp.up_proj", (ff, dm)), ("mlp.down_proj", (dm, ff))):
            ts[p + nm + ".weight"] = torch.randn(*shp, generator=g) * 0.02
        ts[p + "input_layernorm.weight"] = 1 + torch.randn(dm, generator=g) * 0.02
        ts[p + "post_attention_layernorm.weight"] = 1 + torch.randn(dm, generator=g) * 0.02
    ts = {k: v.to(dtype).contiguous() for k, v in ts.items() if k != drop}
    if shards == 1:
        save_file(ts, os.path.join(d, "model.safetensors"))
    else:
        names = sorted(ts)
        wmap = {}
        for i in range(shards):
            part = {n: ts[n] for n in names[i::shards]}
            fn = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
            save_file(part, os.path.join(d, fn))
            wmap.update({n: fn for n in part})
        json.dump({"metadata": {}, "weight_map": wmap}, open(os.path.join(d, "model.safetensors.index.json"), "w"))
    return cfg, ts


@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "BF16"), (torch.float16, "F16"), (torch.float32, "F32")])
def test_reader_matches_an_independent_writer_and_torch_widening(tmp_path, dtype, name):
    _, ts = _tiny_llama_hf(str(tmp_path), dtype)
    lazy = st.load_safetensors_lazy(str(tmp_path / "model.safetensors"))
    assert set(lazy["tensors"]) == set(ts)
    for k, t in ts.items():
        info = lazy["tensors"][k]
        assert info["dtype"] == name and info["shape"] == list(t.shape)
        got = st.read_tensor(lazy, k)["data"]
        want = t.to(torch.float32).numpy()
        assert got.dtype == np.float32 and np.array_equal(got.view(np.uint32), want.view(np.uint32)), k
        view = st.tensor_view(lazy, k)
        assert view.shape == tuple(t.shape) and not view.flags.writeable


def test_bf16_widening_is_the_upper_half_of_an_f32():
    bits = np.array([0x3F80, 0xBF80, 0x7F80, 0xFF80, 0x0001, 0x7FC1, 0x4049], np.uint16)
    want = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(torch.float32).numpy()
    got = st.to_f32(bits, "BF16")
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert got[0] == 1.0 and got[1] == -1.0 and np.isinf(got[2]) and np.isnan(got[5])


def test_load_hf_reads_the_reference_hyper_parameters(tmp_path):
    cfg, _ = _tiny_llama_hf(str(tmp_path))
    hf = loader.load_hf(str(tmp_path))
    assert (hf["n-layers"], hf["d-model"], hf["d-ff"], hf["n-q"], hf["n-kv"], hf["head-dim"], hf["vocab"]) == \
        (2, 256, 512, 8, 2, 32, 2048)
    assert hf["eps"] == 1e-5 and hf["rope-global"] == 500000.0 and hf["rope-local"] == 10000.0
    assert hf["attn-scale"] == pytest.approx(1 / np.sqrt(32))
    # the "model." prefix is normalised away (decoder.clj:39-44)
    assert "layers.0.self_attn.q_proj.weight" in hf["weights"] and "embed_tokens.weight" in hf["weights"]
    arch = loader.architecture(hf)
    assert arch == "llama"
    mc = loader.model_config(hf, arch)
    assert mc["weight_bits"] == 4 and mc["qk_norm"] == 0 and mc["rope_local"] == 500000.0
    tensors = loader.raw_tensors(hf, arch)
    assert len(tensors) == 2 + 2 * 9
    assert {(l, r) for l, r, _, _ in tensors} >= {(-1, "embed"), (-1, "final_norm"), (1, "down"), (0, "ffn_pre_norm")}
    assert all(dt == "BF16" for _, _, dt, _ in tensors)


def test_bare_names_shards_and_defaults(tmp_path):
    _tiny_llama_hf(str(tmp_path), prefix="", shards=3,
                   cfg_extra={"num_key_value_heads": None, "rms_norm_eps": None, "head_dim": 64,
                              "query_pre_attn_scalar": 256})
    hf = loader.load_hf(str(tmp_path))
    assert hf["n-kv"] == 8 and hf["eps"] == 1e-6 and hf["head-dim"] == 64
    assert hf["attn-scale"] == pytest.approx(1 / 16)
    assert len({id(v[0]) for v in hf["weights"].values()}) == 3


def test_architectures_and_missing_tensors(tmp_path):
    _tiny_llama_hf(str(tmp_path / "a"), drop="model.layers.1.mlp.up_proj.weight")
    hf = loader.load_hf(str(tmp_path / "a"))
    with pytest.raises(loader.LoaderError, match="layers.1.mlp.up_proj.weight"):
        loader.raw_tensors(hf, "llama")
    _tiny_llama_hf(str(tmp_path / "b"), cfg_extra={"architectures": ["MambaForCausalLM"], "model_type": "mamba"})
    with pytest.raises(loader.LoaderError, match="unsupported architecture"):
        loader.architecture(loader.load_hf(str(tmp_path / "b")))
    for mt, arch in (("qwen3", "qwen3"), ("gemma3_text", "gemma3")):
        hf = {"config": {"model_type": mt}}
        assert loader.architecture(hf) == arch
    g = loader.model_config({"n-layers": 2, "d-model": 256, "d-ff": 512, "n-q": 4, "n-kv": 1, "head-dim": 64,
                             "vocab": 1024, "eps": 1e-6, "attn-scale": 0.125, "rope-global": 1e6,
                             "rope-local": 1e4}, "gemma3")
    assert (g["gain_offset"], g["sandwich"], g["ffn_geglu"], g["rope_dual"], g["global_pattern"],
            g["sliding_window"], g["embed_scale_sqrt_d"], g["rope_local"]) == (1, 1, 1, 1, 6, 512, 1, 1e4)
    assert loader.model_config({**{k: 1 for k in ("n-layers", "d-model", "d-ff", "n-q", "n-kv", "head-dim", "vocab")},
                                "eps": 1e-6, "attn-scale": 1.0, "rope-global": 1e6, "rope-local": 1e4},
                               "qwen3")["weight_bits"] == 8


def test_truncated_files_are_rejected(tmp_path):
    p = tmp_path / "x.safetensors"
    p.write_bytes(b"\x10\x00")
    with pytest.raises(st.SafetensorsError, match="truncated"):
        st.load_safetensors_lazy(str(p))
    p.write_bytes((100).to_bytes(8, "little") + b"{}")
    with pytest.raises(st.SafetensorsError, match="truncated"):
        st.load_safetensors_lazy(str(p))
