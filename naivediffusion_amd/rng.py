"""The repository's seeded generator for synthetic inputs and weights.

Element i of a tensor with seed s is N(0, 1) by Box-Muller (cosine branch)
over two uniforms taken from splitmix64(s ^ splitmix64(2i)) and
splitmix64(s ^ splitmix64(2i + 1)), in double, then rounded to float32 —
the same counter-based rule the library's device fill uses
(ndx_tensor_fill_normal), so a tensor made on the host and one made on the
GPU agree up to last-ulp differences of the double log/cos. Per-tensor
seeds come from a base seed and the tensor's name (FNV-1a), so every
tensor of a synthetic model is reproducible on its own.
"""

from __future__ import annotations

import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix64(x: np.ndarray) -> np.ndarray:
    x = x + np.uint64(0x9E3779B97F4A7C15)
    x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return x ^ (x >> np.uint64(31))


def splitmix64(x: int) -> int:
    with np.errstate(over="ignore"):
        return int(_splitmix64(np.array([x & 0xFFFFFFFFFFFFFFFF], np.uint64))[0])


def tensor_seed(base: int, name: str) -> int:
    """The seed of one named tensor: splitmix64(base ^ FNV-1a-64(name))."""
    h = 0xCBF29CE484222325
    for b in name.encode():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return splitmix64((base ^ h) & 0xFFFFFFFFFFFFFFFF)


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """float32 N(mean, std) of the given shape."""
    n = int(np.prod(shape, dtype=np.int64))
    out = np.empty(n, np.float32)
    s = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
    chunk = 1 << 22
    with np.errstate(over="ignore"):
        for start in range(0, n, chunk):
            i = np.arange(start, min(n, start + chunk), dtype=np.uint64)
            h1 = _splitmix64(s ^ _splitmix64(np.uint64(2) * i))
            h2 = _splitmix64(s ^ _splitmix64(np.uint64(2) * i + np.uint64(1)))
            u1 = ((h1 >> np.uint64(11)) + np.uint64(1)).astype(np.float64) * (1.0 / 9007199254740992.0)
            u2 = (h2 >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
            z = np.sqrt(-2.0 * np.log(u1)) * np.cos(6.283185307179586 * u2)
            out[start:start + len(i)] = (np.float64(mean) + np.float64(std) * z).astype(np.float32)
    return out.reshape(shape)
