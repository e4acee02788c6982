"""GGML super-block packers and synthetic matrices for the CPU oracle tests
(block_q4_K: dtype.hpp:149; block_q6_K: dtype.hpp:152 of the reference).
Not a test module: imported by test_oracle_math and test_oracle_compose."""
import numpy as np

F16_ONE, F16_HALF, F16_QUARTER = 0x3C00, 0x3800, 0x3400
Q4K, Q6K, F32 = 12, 14, 0


def pack_q4k(d16, dmin16, sc, mn, q):
    """One Q4_K block from 8 6-bit scales, 8 6-bit mins and 256 4-bit values."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    qs = np.zeros(128, np.uint8)
    for c in range(4):                      # 64-weight chunk c: low nibbles, then high
        for l in range(32):
            qs[32 * c + l] = q[64 * c + l] | (q[64 * c + 32 + l] << 4)
    hdr = np.array([d16, dmin16], np.uint16).view(np.uint8)
    return np.concatenate([hdr, s, qs]).astype(np.uint8)


def pack_q6k(d16, sc, q):
    """One Q6_K block from 16 int8 scales and 256 6-bit values (0..63)."""
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for n in range(2):                      # 128-weight halves
        for l in range(32):
            q1, q2, q3, q4 = (q[128 * n + l + 32 * k] for k in range(4))
            ql[64 * n + l] = (q1 & 15) | ((q3 & 15) << 4)
            ql[64 * n + l + 32] = (q2 & 15) | ((q4 & 15) << 4)
            qh[32 * n + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    return np.concatenate([ql, qh, np.asarray(sc, np.int8).view(np.uint8),
                           np.array([d16], np.uint16).view(np.uint8)]).astype(np.uint8)


def q4k_identity(rows: int, cols: int, c: int = 1) -> np.ndarray:
    """Q4_K matrix with weight c (0..15) at (r, r) for r < min(rows, cols), 0
    elsewhere: d = 1, dmin = 0, every 6-bit scale 1, every min 0.  Rows past
    cols are all-zero blocks (d = dmin = 0)."""
    nb = cols // 256
    out = np.zeros((rows, nb, 144), np.uint8)
    for r in range(min(rows, cols)):
        q = np.zeros(256, np.int64)
        q[r % 256] = c
        out[r, r // 256] = pack_q4k(F16_ONE, 0, [1] * 8, [0] * 8, q)
    return out.reshape(-1)


def q4k_zero(rows: int, cols: int) -> np.ndarray:
    return np.zeros(rows * (cols // 256) * 144, np.uint8)


def q4k_random(rng, rows: int, cols: int, scale: float = 1e-4) -> np.ndarray:
    """Random Q4_K bytes with fp16 d, dmin in scale*[0.5, 1.5): weights ~ +-0.02."""
    nb = cols // 256
    b = rng.integers(0, 256, (rows, nb, 144), dtype=np.uint8)
    d = (rng.uniform(0.5, 1.5, (rows, nb, 2)) * scale).astype(np.float16)
    b[:, :, 0:4] = d.view(np.uint8).reshape(rows, nb, 4)
    return b.reshape(-1)


def q6k_random(rng, rows: int, cols: int, scale: float = 1e-5) -> np.ndarray:
    """Random Q6_K bytes (any int8 scales) with fp16 d in scale*[0.5, 1.5)."""
    nb = cols // 256
    b = rng.integers(0, 256, (rows, nb, 210), dtype=np.uint8)
    d = (rng.uniform(0.5, 1.5, (rows, nb)) * scale).astype(np.float16)
    b[:, :, 208:210] = d.view(np.uint8).reshape(rows, nb, 2)
    return b.reshape(-1)


def unpack_q8(b):
    b = np.asarray(b, np.uint8).reshape(-1, 36)
    d = b[:, :4].copy().view(np.float32).reshape(-1)
    q = b[:, 4:].view(np.int8).astype(np.int32)
    return d, q


def dequant_q8(b) -> np.ndarray:
    """d*q per element, one fp32 rounding (what an identity-weight GEMV returns)."""
    d, q = unpack_q8(b)
    return (d[:, None] * q.astype(np.float32)).astype(np.float32).reshape(-1)


Q8_0W, Q5_0W, F16W = 8, 6, 1  # GGUF type ids of the other weight types


def misc_identity(qtype: int, rows: int, cols: int, c: int = 1) -> np.ndarray:
    """Matrix with weight c at (r, r) for r < min(rows, cols), 0 elsewhere, in
    Q8_0 (d = 1, q = c), Q5_0 (d = 1, q5 = 16 + c: every other value 16, i.e. 0)
    or F16 layout (dtype.hpp:130-133 block sizes: 34, 22 bytes per 32; F16 2 per
    element)."""
    if qtype == F16W:
        w = np.zeros((rows, cols), np.float16)
        for r in range(min(rows, cols)):
            w[r, r] = c
        return w.reshape(-1).view(np.uint8)
    nb = cols // 32
    if qtype == Q8_0W:
        out = np.zeros((rows, nb, 34), np.uint8)
        out[:, :, 0:2] = np.array([F16_ONE], np.uint16).view(np.uint8)
        for r in range(min(rows, cols)):
            out[r, r // 32, 2 + r % 32] = c & 0xff
        return out.reshape(-1)
    assert qtype == Q5_0W and 0 <= c <= 15
    out = np.zeros((rows, nb, 22), np.uint8)
    out[:, :, 0:2] = np.array([F16_ONE], np.uint16).view(np.uint8)
    out[:, :, 2:6] = 0xFF                    # the fifth bit of every value: 16 + nibble
    for r in range(min(rows, cols)):
        e = r % 32                           # element e < 16: low nibble of qs[e], else high of qs[e-16]
        if e < 16:
            out[r, r // 32, 6 + e] |= c
        else:
            out[r, r // 32, 6 + e - 16] |= c << 4
    return out.reshape(-1)


def misc_random(rng, qtype: int, rows: int, cols: int, scale: float = 1e-3) -> np.ndarray:
    """Random blocks of the other types: any int8 / 5-bit values, fp16 d in
    scale*[0.5, 1.5); F16 weights N(0, 0.02)."""
    if qtype == F16W:
        return (rng.standard_normal((rows, cols)) * 0.02).astype(np.float16).reshape(-1).view(np.uint8)
    nb = cols // 32
    bb = 34 if qtype == Q8_0W else 22
    b = rng.integers(0, 256, (rows, nb, bb), dtype=np.uint8)
    d = (rng.uniform(0.5, 1.5, (rows, nb)) * scale).astype(np.float16)
    b[:, :, 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    return b.reshape(-1)
