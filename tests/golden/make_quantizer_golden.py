"""Writes tests/golden/quantizer_golden.npz: inputs and expected outputs of
the int8 block quantiser (BlockQuantizer.Quantize, Tensors/BlockQuantizer.cs:
34-101), computed with numpy alone — IEEE float16 rounding from numpy's
astype (round to nearest even) and np.rint (half to even) — so that the
oracle's bit-level C restatement and the library's quantisers are checked
against an independent implementation. The reference itself is C# and
cannot run here; its own test inputs (BlockQuantizerTests.cs:19-70) are
restated as cases: mixed-magnitude [4, 96] blocks, an all-zero block with a
1e-9 outlier (a zero half scale), exact ties at half a step, and values
large enough to clamp.

Run: python tests/golden/make_quantizer_golden.py
"""

from pathlib import Path

import numpy as np


def quantize(w: np.ndarray, block: int = 32):
    rows, cols = w.shape
    blocks = w.reshape(rows, cols // block, block).astype(np.float32)
    peak = np.abs(blocks).max(axis=2)
    scale16 = (peak / np.float32(127)).astype(np.float32).astype(np.float16)
    stored = scale16.astype(np.float32)
    inv = np.where(stored == 0, np.float32(0), np.float32(1) / np.where(stored == 0, np.float32(1), stored))
    q = np.rint(blocks * inv[:, :, None].astype(np.float32)).clip(-127, 127).astype(np.int8)
    q[stored == 0] = 0
    return q.reshape(rows, cols), scale16.view(np.uint16)


def cases():
    r = np.random.default_rng(1)
    mixed = (r.random((4, 96)) * 2 - 1) * np.where(r.integers(0, 4, (4, 96)) == 0, 8.0, 1.0)
    zero = np.zeros((2, 32))
    zero[1, 8] = 1e-9
    # Ties: a peak of 127 * 2^-4 gives an exact half scale of 2^-4; values at
    # odd multiples of half a step land exactly on .5 before rounding.
    ties = np.zeros((2, 32))
    ties[:, 0] = 127 / 16
    ties[0, 1:16] = (np.arange(1, 16) + 0.5) / 16
    ties[1, 1:16] = -(np.arange(1, 16) + 0.5) / 16
    big = (r.standard_normal((3, 64)) * 1000).astype(np.float32)
    small = (r.standard_normal((2, 64)) * 1e-4).astype(np.float32)
    return {"mixed": mixed, "zero": zero, "ties": ties, "big": big, "small": small}


def main():
    out = {}
    for name, w in cases().items():
        w = w.astype(np.float32)
        q, s = quantize(w)
        out[f"{name}_w"] = w
        out[f"{name}_q"] = q
        out[f"{name}_s"] = s
    path = Path(__file__).with_name("quantizer_golden.npz")
    np.savez(path, **out)
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
