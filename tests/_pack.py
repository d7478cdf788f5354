"""Block ENCODERS for the GGUF formats, written from the published layout
(the inverse direction of every decoder under test).  Used to build blocks
whose dequantised values are known in closed form, so a decoder that reads a
nibble, a scale bit or a byte from the wrong place fails."""
from __future__ import annotations

import numpy as np


def f16_bits(v: float) -> int:
    return int(np.array([v], dtype=np.float16).view(np.uint16)[0])


def pack_q4_k(d: float, dmin: float, sc: list[int], m: list[int], q: np.ndarray) -> np.ndarray:
    """sc, m: 8 six-bit values (sub-blocks of 32 weights, in weight order); q: 256 values 0..15."""
    assert len(sc) == 8 and len(m) == 8 and q.shape == (256,)
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(f16_bits(d)).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(f16_bits(dmin)).tobytes(), np.uint8)
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4)
    b[4:16] = s
    qs = np.zeros(128, np.uint8)
    for i in range(4):          # pair i holds sub-blocks 2i (low nibbles) and 2i+1 (high)
        for l in range(32):
            qs[32 * i + l] = (q[64 * i + l] & 0xF) | ((q[64 * i + 32 + l] & 0xF) << 4)
    b[16:] = qs
    return b


def q4_k_values(d, dmin, sc, m, q) -> np.ndarray:
    """Exact real values d*sc_j*q - dmin*m_j (j = weight // 32), float64."""
    j = np.arange(256) // 32
    return d * np.array(sc, np.float64)[j] * q - dmin * np.array(m, np.float64)[j]


def pack_q5_k(d: float, dmin: float, sc: list[int], m: list[int], q: np.ndarray) -> np.ndarray:
    """Q5_K (176 B): the Q4_K header (d, dmin, 12 scale bytes), qh[32], qs[128].
    q: 256 values 0..31; weight 64i + 32h + l keeps its low 4 bits in nibble h of
    qs[32i + l] and its fifth bit in bit 2i + h of qh[l]."""
    assert q.shape == (256,) and int(q.max()) < 32
    hdr = pack_q4_k(d, dmin, sc, m, q & 0xF)
    b = np.zeros(176, np.uint8)
    b[0:16] = hdr[0:16]
    b[48:176] = hdr[16:144]
    qh = np.zeros(32, np.uint8)
    for i in range(4):
        for h in range(2):
            for l in range(32):
                qh[l] |= ((int(q[64 * i + 32 * h + l]) >> 4) & 1) << (2 * i + h)
    b[16:48] = qh
    return b


def pack_q6_k(d: float, sc: list[int], q: np.ndarray) -> np.ndarray:
    """sc: 16 int8 scales (sub-blocks of 16 weights in weight order); q: 256 values 0..63."""
    assert len(sc) == 16 and q.shape == (256,)
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for n in range(2):
        for l in range(32):
            q1, q2, q3, q4 = (int(q[128 * n + l + 32 * p]) for p in range(4))
            ql[64 * n + l] = (q1 & 0xF) | ((q3 & 0xF) << 4)
            ql[64 * n + l + 32] = (q2 & 0xF) | ((q4 & 0xF) << 4)
            qh[32 * n + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    b = np.zeros(210, np.uint8)
    b[0:128] = ql
    b[128:192] = qh
    b[192:208] = np.array(sc, np.int8).view(np.uint8)
    b[208:210] = np.frombuffer(np.uint16(f16_bits(d)).tobytes(), np.uint8)
    return b


def q6_k_values(d, sc, q) -> np.ndarray:
    j = np.arange(256) // 16
    return d * np.array(sc, np.float64)[j] * (q.astype(np.float64) - 32)


def pack_q8_0(d: float, qs: np.ndarray) -> np.ndarray:
    b = np.zeros(34, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(f16_bits(d)).tobytes(), np.uint8)
    b[2:] = qs.astype(np.int8).view(np.uint8)
    return b
