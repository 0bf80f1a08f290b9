"""Writes tests/golden/ref_matvec.npz: matvec vectors computed by AIR's own
reference CPU code (ReferenceTensorReader::matvec, src/reference/
tensor_reader.cpp:369-394), compiled from the reference sources into
oracle/_ref by oracle/Makefile.

Each case stores the canonical GGUF bytes, the activations and the
reference output, so tests can pin the plain-C oracle (and through it the
GPU engine) to the real reference without the reference being present.
Run from the repository root after `make -C oracle`:
    python tests/golden/make_ref_matvec.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from air_amd import quant  # noqa: E402

CASES = [
    # (name, ggml type, K, N, M, weights: "quantized" N(0,0.02) or "random" bytes)
    ("q8_0_quantized", 8, 96, 24, 2, "quantized"),
    ("q8_0_random", 8, 64, 8, 1, "random"),
    ("q4_0_quantized", 2, 128, 16, 2, "quantized"),
    ("q4_0_random", 2, 64, 8, 1, "random"),
    ("q4_k_quantized", 12, 512, 8, 2, "quantized"),
    ("q4_k_random", 12, 256, 4, 1, "random"),
]
BLOCK = {2: (32, 18), 8: (32, 34), 12: (256, 144)}


def main():
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref/libairref.so is not built (needs the reference checkout)")
    rng = np.random.default_rng(0xA17)
    out = {}
    for name, t, k, n, m, kind in CASES:
        be, bb = BLOCK[t]
        if kind == "quantized":
            w = rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.02)
            data = quant.quantize(t, w).reshape(-1)
        else:
            data = rng.integers(0, 256, size=n * (k // be) * bb, dtype=np.uint8)
            blocks = data.reshape(-1, bb)
            nscale = 2 if t == 12 else 1
            for s in range(nscale):  # finite random f16 scales
                bits = rng.integers(0, 0x7800, size=blocks.shape[0], dtype=np.uint16)
                blocks[:, 2 * s:2 * s + 2] = bits.view(np.uint8).reshape(-1, 2)
            data = blocks.reshape(-1)
        x = rng.standard_normal((m, k)).astype(np.float32)
        y = oracle.ref_matvec(t, data, k, n, x)
        out[name + "_meta"] = np.array([t, k, n, m], dtype=np.int64)
        out[name + "_bytes"] = data
        out[name + "_x"] = x
        out[name + "_y"] = y
    path = os.path.join(ROOT, "tests", "golden", "ref_matvec.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
