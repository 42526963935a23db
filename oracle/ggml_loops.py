"""A second restatement of the dequantizers, in the loop structure of ggml's C reference
(`dequantize_row_q8_0`, `dequantize_row_q4_K` with `get_scale_min_k4`, `dequantize_row_q6_K` in
ggml-quants.c, the functions leat/quant.py:14-231 restates with tensor ops and tests against
gguf-py at tests/test_quant.py:11-18). Test infrastructure only.

It walks bytes one weight at a time with Python ints, so it shares no indexing code with the
vectorised `leat_oracle.dequant_blocks`; agreement between the two on random blocks pins the
index arithmetic (a transposed nibble order or a swapped scale branch fails one of them). The
float steps are rounded to f32 after each operation, as C float arithmetic without contraction
does: d1 = d * sc, m1 = dmin * m, y = d1 * q - m1.
"""

from __future__ import annotations

import struct

import numpy as np


def _f32(v: float) -> float:
    return float(np.float32(v))


def _half(b: bytes, at: int) -> float:
    return float(np.frombuffer(b[at : at + 2], dtype=np.float16)[0])


def _scale_min_k4(j: int, q: bytes) -> tuple[int, int]:
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def row_q8_0(block: bytes) -> list[float]:
    d = _half(block, 0)
    return [_f32(d * struct.unpack_from("b", block, 2 + i)[0]) for i in range(32)]


def row_q4_k(block: bytes) -> list[float]:
    d, dmin, scales, q = _half(block, 0), _half(block, 2), block[4:16], block[16:144]
    y, is_, at = [], 0, 0
    for _ in range(0, 256, 64):
        sc, m = _scale_min_k4(is_, scales)
        d1, m1 = _f32(d * sc), _f32(dmin * m)
        sc, m = _scale_min_k4(is_ + 1, scales)
        d2, m2 = _f32(d * sc), _f32(dmin * m)
        y += [_f32(_f32(d1 * (q[at + l] & 0xF)) - m1) for l in range(32)]
        y += [_f32(_f32(d2 * (q[at + l] >> 4)) - m2) for l in range(32)]
        at += 32
        is_ += 2
    return y


def row_q6_k(block: bytes) -> list[float]:
    d = _half(block, 208)
    y = [0.0] * 256
    for n in range(2):
        ql, qh, sc, out = 64 * n, 128 + 32 * n, 192 + 8 * n, 128 * n
        for l in range(32):
            is_ = l // 16
            h = block[qh + l]
            q1 = ((block[ql + l] & 0xF) | (((h >> 0) & 3) << 4)) - 32
            q2 = ((block[ql + l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32
            q3 = ((block[ql + l] >> 4) | (((h >> 4) & 3) << 4)) - 32
            q4 = ((block[ql + l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32
            for k, qv in enumerate((q1, q2, q3, q4)):
                s = struct.unpack_from("b", block, sc + is_ + 2 * k)[0]
                y[out + l + 32 * k] = _f32(_f32(d * s) * qv)
    return y


ROWS = {8: row_q8_0, 12: row_q4_k, 14: row_q6_k}


def dequant_blocks(ggml_type: int, blocks: np.ndarray) -> np.ndarray:
    fn = ROWS[ggml_type]
    return np.array([fn(bytes(b)) for b in np.asarray(blocks, np.uint8)], dtype=np.float32)
