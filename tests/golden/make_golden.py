"""Write the decode-step golden fixtures (``tests/golden/decode_*.json``).

Each fixture records, for a seeded tiny model and a ragged lane schedule, the
greedy tokens of every step and SHA-256 digests of the active lanes' logits,
the resident next-input rows and every K/V page after the last step, as the CPU
oracle (``oracle/rstr_oracle.c``) computes them.  ``tests/test_golden.py``
checks that the oracle still reproduces them and the GPU tests check the HIP
decoder against the same digests.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "pretrained-rstr_amd"), os.path.dirname(HERE)]

import oracle as O  # noqa: E402
from lanes import Routes  # noqa: E402
from rstr import configs  # noqa: E402

CASES = {
    # name: (config, bits, lanes, prefix lengths, schedule of active lanes)
    "tiny_gemma_q4": ("tiny_gemma", 4, 5, [0, 9, 30, 2, 51],
                      [[0, 1, 2, 3, 4], [1, 2, 4], [0, 1, 2, 3, 4], [0, 2, 3], [0, 1, 2, 3, 4]]),
    "tiny_qwen_q8": ("tiny_qwen", 8, 4, [5, 0, 40, 17], [[0, 1, 2, 3]] * 3 + [[1, 3]] + [[0, 1, 2, 3]]),
    "tiny_llama_q4": ("tiny_llama", 4, 4, [12, 33, 0, 7], [[0, 1, 2, 3], [0, 2], [0, 1, 2, 3], [1, 2, 3]]),
}
GEOM = dict(ps=16, pages=40, pps=8, maxpos=128, split=16, seed=3, kv_seed=17)


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def schedule_descriptors(case):
    """The descriptors of every step (shared by the oracle and GPU runs)."""
    cfg_name, bits, B, prefix, sched = CASES[case]
    g = GEOM
    routes = Routes(B, g["ps"], g["pages"], g["pps"], seed=g["seed"])
    fills = []
    for b, n in enumerate(prefix):
        fills += routes.prefix(b, n)
    steps = [(sorted(a), routes.step(a)) for a in sched]
    return configs.with_bits(configs.MODELS[cfg_name], bits), B, fills, steps


def run_oracle(case):
    cfg, B, fills, steps = schedule_descriptors(case)
    g = GEOM
    om = O.Model(cfg, seed=g["seed"])
    od = O.Decoder(om, B, g["ps"], g["pages"], g["pps"], g["maxpos"], kv_f16=True, split=g["split"])
    try:
        for pg in fills:
            od.fill_synthetic(pg, g["kv_seed"])
        toks = (np.arange(B) * 37 + 5) % cfg["vocab"]
        od.prime_lanes(np.arange(B), toks)
        out = {"steps": []}
        for active, desc in steps:
            t = od.step_lanes(**desc)
            act = np.array(active)
            out["steps"].append({"active": active, "tokens": [int(x) for x in t[act]],
                                 "logits_sha256": sha(od.logits()[act])})
        out["rows_sha256"] = sha(od.r0())
        out["pages_sha256"] = [[sha(od.slab(s, l).view(np.uint16)) for s in (0, 1)]
                               for l in range(cfg["n_layers"])]
        return out
    finally:
        od.close()
        om.close()


def main():
    O.build()
    for case in CASES:
        cfg_name, bits, B, prefix, sched = CASES[case]
        rec = {"case": case, "config": cfg_name, "bits": bits, "lanes": B, "prefix": prefix,
               "schedule": sched, "geometry": GEOM, "first_tokens": "(lane*37+5) mod vocab",
               "oracle": run_oracle(case)}
        path = os.path.join(HERE, f"decode_{case}.json")
        with open(path, "w") as f:
            json.dump(rec, f, indent=1)
        print("wrote", path)


if __name__ == "__main__":
    main()
