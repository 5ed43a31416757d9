"""Independent GGUF packers restated from the reference's own dispatch tests.

These are the reference's fixtures: it stores no golden files, it generates
its vectors from a hash (``noise``) and packs GGUF bytes while recording every
coefficient exactly in fp64.  An encoder written from the codes up is an
independent statement of the block layout, so "decode(pack(codes)) equals the
recorded coefficients" pins the decoder (oracle and GPU) without the reference
running.

- ``noise``                 : src/weights/dispatch_tests.rs:15-20
- ``dense_weights``         : src/weights/dispatch_tests/matrix_precision.rs:145-287
- ``mxfp4_decode_weights``  : src/weights/dispatch_tests/mxfp4.rs:46-81
- ``mxfp4_expert_weights``  : src/weights/dispatch_tests/mxfp4.rs:283-307
- ``logits_selecting``      : src/weights/dispatch_tests/mxfp4.rs:38-44
- ``dense_input``           : matrix_precision.rs:45-47
"""
from __future__ import annotations

import numpy as np

F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q5_K, Q6_K, BF16, MXFP4 = 0, 1, 2, 3, 8, 12, 13, 14, 30, 39
WEIGHT_OFFSET = 7  # mxfp4.rs:16
M32 = 0xFFFFFFFF


def noise(index: int) -> int:
    value = index & M32
    value = ((value ^ (value >> 16)) * 0x7FEB352D) & M32
    value = ((value ^ (value >> 15)) * 0x846CA68B) & M32
    return value ^ (value >> 16)


def f16(value: float) -> float:
    """half::f16::from_f64 / from_f32 (round to nearest even), back to f64."""
    return float(np.float16(value))


def f16_bits(value: float) -> bytes:
    return np.float16(value).tobytes()


def bf16_bits(value: float) -> int:
    u = int(np.float32(value).view(np.uint32))
    if (u & 0x7FFFFFFF) > 0x7F800000:
        return (u >> 16) | 0x40
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF


def bf16_value(bits: int) -> float:
    return float(np.uint32(bits << 16).view(np.float32))


def dense_weights(fmt: int, n: int, k: int):
    """matrix_precision.rs:145-287: (GGUF bytes, [(coefficient, affine magnitude)])."""
    out = bytearray()
    coeffs: list[tuple[float, float]] = []
    for row in range(n):
        if fmt in (F32, F16, BF16):
            for column in range(k):
                v = (noise(row * k + column + 37) % 2001) - 1000
                v = float(np.float32(np.float32(v) * np.float32(0.000131)))
                if fmt == F32:
                    out += np.float32(v).tobytes()
                    val = v
                elif fmt == F16:
                    out += f16_bits(v)
                    val = f16(v)
                else:
                    b = bf16_bits(v)
                    out += int(b).to_bytes(2, "little")
                    val = bf16_value(b)
                coeffs.append((val, abs(val)))
            continue
        block = 32 if fmt in (Q4_0, Q4_1, Q8_0) else 256
        for start in range(0, k, block):
            seed = row * k + start
            scale = f16(float(np.float32(5 + noise(seed + 41) % 43) * np.float32(0.00031)))
            d = scale
            codes = [noise(seed + index + 113) & 0xFF for index in range(block)]
            if fmt in (Q4_0, Q4_1, Q8_0):
                out += f16_bits(scale)
                if fmt == Q8_0:
                    for code in codes:
                        value = d * float(np.int8(np.uint8(code)))
                        out.append(code)
                        coeffs.append((value, abs(value)))
                    continue
                if fmt == Q4_0:
                    offset = -8.0 * d
                else:
                    offset = f16(-7.5 * d)
                    out += f16_bits(offset)
                codes = [c & 15 for c in codes]
                for code in codes:
                    product = d * code
                    coeffs.append((product + offset, abs(product) + abs(offset)))
                for index in range(16):
                    out.append(codes[index] | (codes[index + 16] << 4))
            elif fmt in (Q4_K, Q5_K):
                minimum = f16(d * 0.9375)
                out += f16_bits(scale)
                out += f16_bits(minimum)
                scales = [1 + noise(seed + i + 223) % 63 for i in range(8)]
                minima = [noise(seed + i + 317) % 64 for i in range(8)]
                packed = [0] * 12
                for i in range(8):
                    if i < 4:
                        packed[i] = scales[i]
                        packed[i + 4] = minima[i]
                    else:
                        packed[i + 4] = (scales[i] & 15) | ((minima[i] & 15) << 4)
                        packed[i - 4] |= (scales[i] >> 4) << 6
                        packed[i] |= (minima[i] >> 4) << 6
                out += bytes(p & 0xFF for p in packed)
                high = [0] * 32
                mask = 31 if fmt == Q5_K else 15
                codes = [c & mask for c in codes]
                for index, code in enumerate(codes):
                    product = d * scales[index // 32] * code
                    offset = minimum * minima[index // 32]
                    coeffs.append((product - offset, abs(product) + abs(offset)))
                    high[index % 32] |= (code >> 4) << (index // 32)
                if fmt == Q5_K:
                    out += bytes(high)
                for c0 in range(0, 256, 64):
                    chunk = codes[c0:c0 + 64]
                    for index in range(32):
                        out.append((chunk[index] & 15) | ((chunk[index + 32] & 15) << 4))
            elif fmt == Q6_K:
                scales = [int(np.int8(np.uint8(noise(seed + i + 433) & 0xFF))) for i in range(16)]
                low = [0] * 128
                high = [0] * 64
                for index in range(256):
                    code = codes[index] & 63
                    value = d * scales[index // 16] * (code - 32)
                    coeffs.append((value, abs(value)))
                    half, quarter, lane = index // 128, index % 128 // 32, index % 32
                    low[half * 64 + quarter % 2 * 32 + lane] |= (code & 15) << (quarter // 2 * 4)
                    high[half * 32 + lane] |= (code >> 4) << (quarter * 2)
                out += bytes(low)
                out += bytes(high)
                out += bytes(s & 0xFF for s in scales)
                out += f16_bits(scale)
            else:
                raise ValueError(fmt)
    return bytes(out), coeffs


def dense_input(m: int, k: int) -> np.ndarray:
    """bf16 bits of (noise(i + 9173) % 251) / 127 - 1 (matrix_precision.rs:45-47)."""
    vals = [float(np.float32(noise(i + 9173) % 251) / np.float32(127.0) - np.float32(1.0))
            for i in range(m * k)]
    return np.array([bf16_bits(v) for v in vals], np.uint16).reshape(m, k)


HALVES = [0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12]


def mxfp4_decode_weights(k: int, n: int, experts: int = 4):
    """mxfp4.rs:46-81: bytes (after WEIGHT_OFFSET 0xa5 pad bytes) and f64 coefficients."""
    out = bytearray([0xA5] * WEIGHT_OFFSET)
    coeffs = []
    for expert in range(experts):
        for row in range(n):
            for block in range(k // 32):
                power = (noise(expert * n + row + block % (k // 64)) % 9) - 5
                scale = 2.0 ** power
                codes = [0] * 32
                for c in range(32):
                    column = block * 32 + c
                    source = column % (k // 2) if row % 3 == 0 else column
                    code = noise((expert * n + row) * k + source + 1327) % 16
                    if row % 3 == 0 and column >= k // 2:
                        code ^= 8
                    codes[c] = code
                    coeffs.append(HALVES[code] * 0.5 * scale)
                out.append(127 + power)
                for c in range(16):
                    out.append(codes[c] | (codes[c + 16] << 4))
    return bytes(out), np.array(coeffs, np.float64)


def mxfp4_decode_input(k: int) -> np.ndarray:
    """mxfp4.rs:86-92: four f32 input rows, the second half of each repeating the first."""
    vals = []
    for i in range(4 * k):
        index = i // k * k + i % (k // 2)
        vals.append(float(np.float32((noise(index + 8719) % 10007) - 5003) / np.float32(4093.0)))
    return np.array(vals, np.float32)


def mxfp4_expert_weights(k: int, n: int, salt: int, experts: int = 32):
    """mxfp4.rs:283-307 (with the WEIGHT_OFFSET pad)."""
    out = bytearray([0xA5] * WEIGHT_OFFSET)
    values = []
    for expert in range(experts):
        for row in range(n):
            for block in range(k // 32):
                power = ((expert + row + block + salt) % 5) - 3
                scale = 2.0 ** power
                codes = [((c * 13 + c // 16 * 5 + expert * 3 + row * 5 + block * 7 + salt) % 16)
                         for c in range(32)]
                values += [HALVES[c] * 0.5 * scale for c in codes]
                out.append(127 + power)
                for c in range(16):
                    out.append(codes[c] | (codes[c + 16] << 4))
    return bytes(out), np.array(values, np.float32)


def logits_selecting(ids) -> np.ndarray:
    logits = np.full(32, -10.0, np.float32)
    for rank, i in enumerate(ids):
        logits[i] = 4.0 - rank
    return logits


def expert_ids(batch: int) -> np.ndarray:
    """mxfp4.rs:345-347: expert 31 and 30 overfull, others sparse."""
    return np.array([[31, t % 15, 15 + t % 8, 30] for t in range(batch)], np.uint32).ravel()
