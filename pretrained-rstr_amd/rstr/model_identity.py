"""Stable identities for attention-state compatibility
(``src/pretrained/model_identity.clj``).

``compatibility_fingerprint`` hashes a canonical manifest of the weights
identity (an explicit ``weights_id`` or the SHA-256 of ``model.safetensors``),
the execution variant, architecture, HF config, descriptor and attention-state
layout.  The reference serialises the manifest with the ``boring`` archival
encoding, which is not available here; this build serialises the same
manifest as canonical JSON (sorted keys, keywords as ":name" strings), so its
digests are stable and sensitive to the same inputs but are not byte-equal to
the reference's.
"""
from __future__ import annotations

import hashlib
import json
import os


class IdentityError(ValueError):
    pass


def _sha256_file(path: str) -> str:
    """model_identity.clj:9-19 (streamed in 1 MiB reads)."""
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 20), b""):
            h.update(block)
    return h.hexdigest()


def _canonical(v):
    """model_identity.clj:21-28: maps sorted by key, sets sorted, sequences kept."""
    if isinstance(v, dict):
        return ["map", [[_canonical(k), _canonical(v[k])] for k in sorted(v, key=repr)]]
    if isinstance(v, (set, frozenset)):
        return ["set", [_canonical(x) for x in sorted(v, key=repr)]]
    if isinstance(v, (list, tuple)):
        return [_canonical(x) for x in v]
    return v


def compatibility_fingerprint(model: dict, weights_id: str | None = None,
                              execution_variant: str = ":default") -> str:
    """model_identity.clj:30-63.  ``model`` carries ``dir``, ``arch`` (or
    ``desc["arch"]``), ``config``, ``desc`` and ``attention-state``."""
    ident = weights_id
    if ident is None:
        d = model.get("dir")
        f = os.path.join(str(d), "model.safetensors") if d is not None else None
        if f is None or not os.path.isfile(f):
            raise IdentityError("Model fingerprint requires :weights-id or model.safetensors")
        ident = "sha256:" + _sha256_file(f)
    manifest = _canonical({":format-version": 1, ":weights": ident, ":execution-variant": execution_variant,
                           ":architecture": model.get("arch") or (model.get("desc") or {}).get("arch"),
                           ":config": model.get("config"), ":descriptor": model.get("desc"),
                           ":attention-state": model.get("attention-state")})
    data = json.dumps(manifest, sort_keys=True, separators=(",", ":"), default=repr).encode("utf-8")
    return "sha256:" + hashlib.sha256(data).hexdigest()
