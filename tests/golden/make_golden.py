"""Writes tests/golden/moe_small.npz: seeded small layers, their routing, permutation,
per-(token, k) expert outputs and combined layer output, all computed by the oracle.

The reference's own tests hold no vectors for this path, and its expert-MLP sources need
Apple headers this image lacks, so these fixtures pin the oracle against drift
(tests/test_oracle.py::test_golden_fixture_reproduces) and give the GPU path a stored target
(tests/test_gpu_parity.py::test_stored_golden_fixture); the oracle itself is pinned by the
other tests in tests/test_oracle.py.
Only the layer's SHA-256 is stored, not the weights: the generator recreates them.

Run:  python -m tests.golden.make_golden
"""
from __future__ import annotations

import hashlib
import os

import numpy as np

from kandiga_amd import synth
from oracle import moe_oracle as O

CASES = {
    "h256_e16_i128_k4_3bit": (synth.LayerShape(256, 128, 16, 4, 3), 101, 5),
    "h256_e16_i128_k4_4bit": (synth.LayerShape(256, 128, 16, 4, 4), 102, 5),
    "h320_e12_i192_k3_3bit": (synth.LayerShape(320, 192, 12, 3, 3), 103, 9),
}


def layer_sha256(layer: dict) -> str:
    h = hashlib.sha256()
    for k in sorted(layer):
        h.update(k.encode())
        h.update(np.ascontiguousarray(layer[k]).tobytes())
    return h.hexdigest()


def build_case(name: str) -> dict:
    shape, seed, tokens = CASES[name]
    layer = synth.make_layer(shape, seed)
    x, logits = synth.make_inputs(shape, tokens, seed + 1)
    r = O.moe_layer(layer, x, logits, shape.top_k, shape.bits)
    return dict(layer_sha256=layer_sha256(layer), x=x, logits=logits, idx=r["idx"], w=r["w"],
                perm=O.permute(r["idx"], shape.num_experts)["perm"], y=r["y"], out=r["out"])


def main() -> None:
    out = {}
    for name in CASES:
        case = build_case(name)
        for k, v in case.items():
            out[f"{name}.{k}"] = np.asarray(v)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "moe_small.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
