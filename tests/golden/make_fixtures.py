"""Extract the reference's golden data for this path into small fixtures.

Run in a container where the mlx-bun reference is mounted:
    python tests/golden/make_fixtures.py [/root/reference]

Reads (data only, no code is executed or copied):
  goldens/rotating-kvq.{json,bin}      -- mechanics section: MLX's quantize
      outputs (8-bit, group 32, bf16) through a RotatingQuantizedKVCache
      driven by scripts/regen-rotating-kvq-goldens.ts:51-72
  tests/fixtures/batched-rotating-golden.json -- batched ring masks/keys

Writes:
  tests/golden/rotating_kvq_mechanics.npz
  tests/golden/batched_rotating.json
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

OUT = os.path.dirname(os.path.abspath(__file__))


def main(ref: str) -> None:
    man = json.load(open(os.path.join(ref, "goldens", "rotating-kvq.json")))
    blob = open(os.path.join(ref, "goldens", "rotating-kvq.bin"), "rb").read()

    def arr(t, dt):
        n = int(np.prod(t["shape"]))
        a = np.frombuffer(blob, dtype=dt, count=n, offset=t["offset"] * 4)
        return a.reshape(t["shape"]).copy()

    mech = man["mechanics"]
    out = {"config": np.array([mech["config"][k] for k in ("max_size", "heads", "dim", "group_size", "bits")],
                              dtype=np.int64)}
    out["step_sizes"] = np.array([s["S"] for s in mech["steps"]], dtype=np.int64)
    for i, s in enumerate(mech["steps"]):
        out[f"step{i}_k"] = arr(s["k"], np.float32)
        out[f"step{i}_v"] = arr(s["v"], np.float32)
    cps = sorted(int(c) for c in mech["checkpoints"])
    out["checkpoints"] = np.array(cps, dtype=np.int64)
    for c in cps:
        cp = mech["checkpoints"][str(c)]
        out[f"cp{c}_offset_idx"] = np.array([cp["offset"], cp["idx"]], dtype=np.int64)
        for name in ("k_packed", "v_packed"):
            out[f"cp{c}_{name}"] = arr(cp[name], np.uint32)
        for name in ("k_scales", "k_biases", "v_scales", "v_biases"):
            out[f"cp{c}_{name}"] = arr(cp[name], np.float32)
    np.savez_compressed(os.path.join(OUT, "rotating_kvq_mechanics.npz"), **out)

    br = json.load(open(os.path.join(ref, "tests", "fixtures", "batched-rotating-golden.json")))
    with open(os.path.join(OUT, "batched_rotating.json"), "w") as f:
        json.dump(br, f)
    print("wrote rotating_kvq_mechanics.npz and batched_rotating.json")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
