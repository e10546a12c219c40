"""Writes tests/golden/tq3_quantize.npz: input/output vectors of the reference's TQ3 quantizer.

The quantizer (kandiga/tq3/quantize.py quantize_tensor, :390-463, with the scale search and
refinement of :190-236) is an optimisation procedure that no closed form pins, so its outputs are
taken from the reference itself: this script loads that one numpy-only file by path (not through
the kandiga package) in the build container and stores, for seeded input tensors, the 20-byte
blocks it writes and the weights its dequantize_tensor (:489-516) reads back.  The fixture holds
data only; the GPU box and the tests never read the reference.

    python tests/golden/make_tq3_golden.py      (in the build container)
"""
import importlib.util
import os

import numpy as np

REF = "/root/reference/kandiga/tq3/quantize.py"
HERE = os.path.dirname(os.path.abspath(__file__))


def inputs():
    rng = np.random.Generator(np.random.PCG64(2024))
    a = (rng.standard_normal((8, 64)) * 0.02).astype(np.float32)            # typical weights
    b = (rng.standard_normal((4, 96)) * 0.05).astype(np.float32)
    b[1] = 0.0                                                                # an all-zero row
    b[2, ::7] = 3.0                                                           # outliers
    c = np.full((2, 32), 0.125, np.float32)                                   # constant blocks
    d = (rng.standard_normal(50) * 0.01).astype(np.float32)                   # padded tail
    return {"a": a, "b": b, "c": c, "d": d}


def main():
    spec = importlib.util.spec_from_file_location("tq3_quantize_reference", REF)
    q = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(q)
    out = {}
    for name, w in inputs().items():
        data, shape, nblocks = q.quantize_tensor(w)
        out[f"{name}.input"] = w
        out[f"{name}.blocks"] = np.frombuffer(data, dtype=np.uint8).reshape(nblocks, 20)
        out[f"{name}.dequant"] = q.dequantize_tensor(data, shape, nblocks)
    np.savez(os.path.join(HERE, "tq3_quantize.npz"), **out)
    print("wrote", os.path.join(HERE, "tq3_quantize.npz"), sorted(out))


if __name__ == "__main__":
    main()
