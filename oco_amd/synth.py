"""Seeded synthetic GGUF tensors and activations for the benchmark configs.

Counter-based splitmix64 streams (so any slice can be regenerated), uniform
variates from the top 53 bits, normals by Box-Muller.  Weight bytes follow the
exact GGUF block layouts (src/tensor.rs:24-38; decode rules of
shaders/matrix/weights.metal:40-85):

- Q8_0  : 32 int8 codes uniform in [-127, 127], f16 d = |N(0, 0.02)| / 127
- MXFP4 : 32 E2M1 codes uniform over all 16, E8M0 exponent uniform in 118..123
          (2^-9 .. 2^-4)
- Q4_K  : 6-bit scales and mins uniform, f16 d and dmin = |N(0, 0.01)|, codes uniform
- Q6_K  : 6-bit codes uniform, int8 sub-block scales uniform, f16 d = |N(0, 0.01)|
- Q4_0  : 4-bit codes uniform, f16 d = |N(0, 0.01)|
- Q4_1  : 4-bit codes uniform, f16 d = |N(0, 0.01)|, f16 m = N(0, 0.01)
- Q5_K  : as Q4_K plus uniform fifth bits (qh)
"""
from __future__ import annotations

import numpy as np

_G = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (np.arange(offset + 1, offset + n + 1, dtype=np.uint64) * _G) + np.uint64(seed * 0x632BE59BD9B4E019 & 0xFFFFFFFFFFFFFFFF)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int) -> np.ndarray:
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def normal(seed: int, n: int) -> np.ndarray:
    m = (n + 1) // 2
    u = uniform(seed, 2 * m)
    u1 = 1.0 - u[:m]  # (0, 1]
    u2 = u[m:]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])
    return z[:n]


def random_bytes(seed: int, n: int) -> np.ndarray:
    words = splitmix64(seed, (n + 7) // 8)
    return words.view(np.uint8)[:n].copy()


def activations(seed: int, n: int) -> np.ndarray:
    """f32 ~ N(0, 1)."""
    return normal(seed, n).astype(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def q8_0(rows: int, k: int, seed: int) -> np.ndarray:
    nb = rows * (k // 32)
    blocks = np.empty((nb, 34), np.uint8)
    codes = (splitmix64(seed, nb * 32) % np.uint64(255)).astype(np.int16) - 127
    blocks[:, 2:] = codes.astype(np.int8).view(np.uint8).reshape(nb, 32)
    d = (np.abs(normal(seed + 1, nb)) * 0.02 / 127.0).astype(np.float16)
    blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    return blocks.reshape(-1)


def mxfp4(rows: int, k: int, seed: int) -> np.ndarray:
    nb = rows * (k // 32)
    blocks = np.empty((nb, 17), np.uint8)
    blocks[:, 1:] = random_bytes(seed, nb * 16).reshape(nb, 16)
    blocks[:, 0] = (118 + splitmix64(seed + 1, nb) % np.uint64(6)).astype(np.uint8)
    return blocks.reshape(-1)


def q4_k(rows: int, k: int, seed: int) -> np.ndarray:
    nb = rows * (k // 256)
    blocks = random_bytes(seed, nb * 144).reshape(nb, 144)  # qs and 6-bit scales/mins uniform
    d = (np.abs(normal(seed + 1, nb)) * 0.01).astype(np.float16)
    dmin = (np.abs(normal(seed + 2, nb)) * 0.01).astype(np.float16)
    blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blocks[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    return blocks.reshape(-1)


def q6_k(rows: int, k: int, seed: int) -> np.ndarray:
    nb = rows * (k // 256)
    blocks = random_bytes(seed, nb * 210).reshape(nb, 210)  # codes and int8 scales uniform
    d = (np.abs(normal(seed + 1, nb)) * 0.01).astype(np.float16)
    blocks[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return blocks.reshape(-1)


def q4_0(rows: int, k: int, seed: int) -> np.ndarray:
    nb = rows * (k // 32)
    blocks = random_bytes(seed, nb * 18).reshape(nb, 18)
    d = (np.abs(normal(seed + 1, nb)) * 0.01).astype(np.float16)
    blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    return blocks.reshape(-1)


def q4_1(rows: int, k: int, seed: int) -> np.ndarray:
    nb = rows * (k // 32)
    blocks = random_bytes(seed, nb * 20).reshape(nb, 20)
    d = (np.abs(normal(seed + 1, nb)) * 0.01).astype(np.float16)
    m = (normal(seed + 2, nb) * 0.01).astype(np.float16)
    blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blocks[:, 2:4] = m.view(np.uint8).reshape(nb, 2)
    return blocks.reshape(-1)


def q5_k(rows: int, k: int, seed: int) -> np.ndarray:
    nb = rows * (k // 256)
    blocks = random_bytes(seed, nb * 176).reshape(nb, 176)
    d = (np.abs(normal(seed + 1, nb)) * 0.01).astype(np.float16)
    dmin = (np.abs(normal(seed + 2, nb)) * 0.01).astype(np.float16)
    blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blocks[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    return blocks.reshape(-1)


GENERATORS = {8: q8_0, 39: mxfp4, 12: q4_k, 14: q6_k, 2: q4_0, 3: q4_1, 13: q5_k}


def weights(fmt: int, rows: int, k: int, seed: int) -> np.ndarray:
    return GENERATORS[int(fmt)](rows, k, seed)
