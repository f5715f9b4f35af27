"""Serving assembly: compatibility fingerprints (``rstr.model_identity``, the
properties ``test/pretrained/model_identity_test.clj`` checks), the worker's
default measurements and option validation (``rstr.model_worker``), and on the
GPU a worker opened from a checkpoint directory generating the same tokens as
the CPU oracle decoding the same checkpoint (its tensors widened to f32 and
quantised by the oracle), with and without a bulk-prefill tile, then closing
in order.

Fingerprint bytes are parity unpinned: the reference encodes the manifest with
the ``boring`` archival format (model_identity.clj:62), which is absent here;
this build hashes canonical JSON of the same manifest, so digests are stable and
sensitive to the same fields but not byte-equal to the reference's."""
import numpy as np
import pytest

from rstr import model_identity as mi
from rstr import model_worker as mw


def _fixture_model(d):
    return {"dir": None if d is None else str(d), "arch": "Fixture",
            "config": {"hidden_size": 2, "num_hidden_layers": 1},
            "desc": {"arch": ":fixture", "flags": {"rope": ":single"}}}


def test_fingerprints_weights_layout_and_execution_variant(tmp_path):
    """model_identity_test.clj:15-37."""
    (tmp_path / "model.safetensors").write_bytes(bytes([1, 2, 3]))
    m = _fixture_model(tmp_path)
    a, b = mi.compatibility_fingerprint(m), mi.compatibility_fingerprint(m)
    assert a == b and a.startswith("sha256:")
    assert a != mi.compatibility_fingerprint(m, execution_variant=":q8")
    (tmp_path / "model.safetensors").write_bytes(bytes([1, 2, 4]))
    assert a != mi.compatibility_fingerprint(m)


def test_accepts_an_immutable_external_weights_id():
    """model_identity_test.clj:39-48."""
    m = _fixture_model(None)
    assert mi.compatibility_fingerprint(m, weights_id="hf-revision:abc") == \
        mi.compatibility_fingerprint(m, weights_id="hf-revision:abc")
    with pytest.raises(mi.IdentityError, match="weights-id"):
        mi.compatibility_fingerprint(m)


def test_fingerprint_sees_config_and_descriptor_changes():
    m = _fixture_model(None)
    base = mi.compatibility_fingerprint(m, weights_id="w")
    m2 = dict(m, config={"hidden_size": 3, "num_hidden_layers": 1})
    m3 = dict(m, desc={"arch": ":fixture", "flags": {"rope": ":dual"}})
    assert len({base, mi.compatibility_fingerprint(m2, weights_id="w"),
                mi.compatibility_fingerprint(m3, weights_id="w")}) == 3
    # key order does not matter (canonical maps)
    m4 = dict(m, config={"num_hidden_layers": 1, "hidden_size": 2})
    assert mi.compatibility_fingerprint(m4, weights_id="w") == base


def test_default_measurements_and_validation():
    """model_worker.clj:37-50, :93-99."""
    assert mw.default_measurements(":worker-a", 1024) == {
        "worker/node": "worker-a", "worker/queue-ms": 0.0, "worker/max-context": 1024,
        "worker/prefill-ms-per-token": 10.0, "worker/first-token-ms": 10.0,
        "worker/gpu-restore-bytes-per-ms": 1000000.0, "worker/tier-throughput-bytes-per-ms": {},
        "worker/object-store?": False}
    with pytest.raises(mw.WorkerError, match="compatibility fingerprint"):
        mw.open_worker("/nonexistent", None)


@pytest.mark.gpu
@pytest.mark.parametrize("prefill_T", [None, 8])
def test_worker_generates_like_the_oracle_on_the_checkpoint(tmp_path, prefill_T):
    print("case worker", prefill_T, flush=True)
    import oracle as O
    from rstr import loader
    from rstr import safetensors as st
    from rstr.page_pool import PagePool
    from rstr.paged_decoder import PagedDecoder
    from test_config1 import OracleStepDevice
    from test_gpu_loader import _write_checkpoint
    _write_checkpoint(str(tmp_path), "llama")
    hf = loader.load_hf(str(tmp_path))
    fp = mi.compatibility_fingerprint({"dir": str(tmp_path), "arch": "llama", "config": hf["config"],
                                       "desc": loader.DESCRIPTORS["llama"]["flags"]},
                                      execution_variant=":gpu-q4-paged")
    prompt = [int(x) for x in np.random.default_rng(1).integers(0, 1024, 21)]
    w = mw.open_worker(str(tmp_path), fp, max_position=64, page_size=16, prefill_T=prefill_T, split=16)
    try:
        assert w.worker_opts["worker/models"] == {fp} and w.worker_opts["worker/free-pages"] == 16
        got = w.generate("c", prompt, 9)
    finally:
        w.close()
        w.close()
    # the oracle decodes the same checkpoint: every tensor widened to f32
    # (safetensors.clj:39-78) and quantised by the oracle's block rules
    arch = loader.architecture(hf)
    cfg = loader.model_config(hf, arch)
    om = O.Model(cfg, seed=0)
    try:
        for layer, role, dtype, view in loader.raw_tensors(hf, arch):
            om.set_tensor(layer, role, st.to_f32(view, dtype))
        od = O.Decoder(om, 1, 16, 16, 4, 64, kv_f16=True, split=16)
        try:
            pool = PagePool(16, 16, cfg["n_layers"], cfg["n_kv"], cfg["head_dim"], "half", device=od)
            want = PagedDecoder(pool, OracleStepDevice(od), batch_size=1, maxpos=64,
                                pages_per_sequence=4).generate("c", prompt, 9)
        finally:
            od.close()
    finally:
        om.close()
    assert got == want and len(got) == 9
