"""Hand-built GGUF K-quant blocks for known-answer tests.

The builders below write blocks field by field from the GGUF block layouts
(crates/inferi/src/quantization.rs:42-45, 60-63, 87-91, 116-120, 147-152,
183-187, 217-222, 262-268, 335-340 in the reference, i.e. ggml's block_q8_0,
q4_0, q4_1, q5_0, q5_1, q8_K, q6_K, q5_K and q4_K), so
that a test can state the expected dequantized values in closed form.  They
share no code with the oracle.
"""

import numpy as np

F16_ONE = 0x3C00
F16_HALF = 0x3800
F16_QUARTER = 0x3400
F16_TWO = 0x4000


def pack_scales_bits(sc, mn) -> bytes:
    """Place eight 6-bit scales and mins into the 12-byte K-quant field.

    Bit placement (ggml-common.h, block_q4_K.scales):
      j < 4 : sc_j -> bits 0..5 of byte j;   m_j -> bits 0..5 of byte j+4
      j >= 4: sc_j bits 0..3 -> bits 0..3 of byte j+4, bits 4..5 -> bits 6..7 of byte j-4
              m_j  bits 0..3 -> bits 4..7 of byte j+4, bits 4..5 -> bits 6..7 of byte j
    """
    b = [0] * 12
    for j in range(8):
        s, m = int(sc[j]) & 63, int(mn[j]) & 63
        if j < 4:
            b[j] |= s
            b[j + 4] |= m
        else:
            b[j + 4] |= (s & 15) | ((m & 15) << 4)
            b[j - 4] |= (s >> 4) << 6
            b[j] |= (m >> 4) << 6
    return bytes(b)


def q4k_block(d16: int, dmin16: int, sc, mn, q) -> bytes:
    """q: 256 ints in 0..15 in element order."""
    q = np.asarray(q, dtype=np.int64)
    qs = bytearray(128)
    for g in range(4):
        for l in range(32):
            qs[32 * g + l] = int(q[64 * g + l]) | (int(q[64 * g + 32 + l]) << 4)
    return d16.to_bytes(2, "little") + dmin16.to_bytes(2, "little") + pack_scales_bits(sc, mn) + bytes(qs)


def q5k_block(d16: int, dmin16: int, sc, mn, q) -> bytes:
    """q: 256 ints in 0..31 in element order."""
    q = np.asarray(q, dtype=np.int64)
    qh = bytearray(32)
    qs = bytearray(128)
    for g in range(4):
        for l in range(32):
            a, b = int(q[64 * g + l]), int(q[64 * g + 32 + l])
            qs[32 * g + l] = (a & 15) | ((b & 15) << 4)
            qh[l] |= ((a >> 4) & 1) << (2 * g)
            qh[l] |= ((b >> 4) & 1) << (2 * g + 1)
    return d16.to_bytes(2, "little") + dmin16.to_bytes(2, "little") + pack_scales_bits(sc, mn) + bytes(qh) + bytes(qs)


def q6k_block(d16: int, sc, q) -> bytes:
    """sc: 16 ints in -128..127 (one per 16 elements); q: 256 ints in -32..31."""
    u = np.asarray(q, dtype=np.int64) + 32
    ql = bytearray(128)
    qh = bytearray(64)
    for i in range(2):
        for l in range(32):
            e = 128 * i + l
            a, b, c, dd = int(u[e]), int(u[e + 32]), int(u[e + 64]), int(u[e + 96])
            ql[64 * i + l] = (a & 15) | ((c & 15) << 4)
            ql[64 * i + l + 32] = (b & 15) | ((dd & 15) << 4)
            qh[32 * i + l] = (a >> 4) | ((b >> 4) << 2) | ((c >> 4) << 4) | ((dd >> 4) << 6)
    scb = bytes(int(s) & 0xFF for s in sc)
    return bytes(ql) + bytes(qh) + scb + d16.to_bytes(2, "little")


def q8_0_block(d16: int, q) -> bytes:
    return d16.to_bytes(2, "little") + bytes(int(v) & 0xFF for v in q)


def _nibbles16(u) -> bytes:
    """Byte j holds code j (low nibble) and code j+16 (high)."""
    return bytes((int(u[j]) & 15) | ((int(u[j + 16]) & 15) << 4) for j in range(16))


def _high32(u) -> bytes:
    """Bit j of the little-endian word is bit 4 of code j."""
    h = 0
    for j in range(32):
        h |= ((int(u[j]) >> 4) & 1) << j
    return h.to_bytes(4, "little")


def q4_0_block(d16: int, q) -> bytes:
    """q: 32 ints in -8..7 (stored +8); layout d@0 qs[16]@2 (ggml block_q4_0)."""
    u = [int(v) + 8 for v in q]
    return d16.to_bytes(2, "little") + _nibbles16(u)


def q4_1_block(d16: int, m16: int, q) -> bytes:
    """q: 32 ints in 0..15; layout d@0 m@2 qs[16]@4 (block_q4_1)."""
    return d16.to_bytes(2, "little") + m16.to_bytes(2, "little") + _nibbles16(q)


def q5_0_block(d16: int, q) -> bytes:
    """q: 32 ints in -16..15 (stored +16); layout d@0 qh[4]@2 qs[16]@6 (block_q5_0)."""
    u = [int(v) + 16 for v in q]
    return d16.to_bytes(2, "little") + _high32(u) + _nibbles16(u)


def q5_1_block(d16: int, m16: int, q) -> bytes:
    """q: 32 ints in 0..31; layout d@0 m@2 qh[4]@4 qs[16]@8 (block_q5_1)."""
    return d16.to_bytes(2, "little") + m16.to_bytes(2, "little") + _high32(q) + _nibbles16(q)


def q8_k_block(d: float, q, bsums=None) -> bytes:
    """q: 256 ints in -128..127; layout d:f32@0 qs[256]@4 bsums:i16[16]@260
    (block_q8_K; bsums default to the sums of q over 16 elements)."""
    q = [int(v) for v in q]
    if bsums is None:
        bsums = [sum(q[16 * j:16 * j + 16]) for j in range(16)]
    return (np.array([d], np.float32).tobytes() + bytes(v & 0xFF for v in q)
            + np.array(bsums, np.int16).astype("<i2").tobytes())


def f16_value(code: int) -> float:
    return float(np.array([code], np.uint16).view(np.float16)[0])


def random_valid_f16_scale(rng: np.random.Generator) -> int:
    """A finite f16 in [-1, 1], a quarter of them subnormal, as the reference's
    GEMV tests draw them (crates/inferi/src/ops/gemv_quant.rs:354-365)."""
    v = rng.random() * 2.0 - 1.0
    if rng.integers(0, 256) < 64:
        v *= 1e-5
    return int(np.array([v], np.float16).view(np.uint16)[0])


def random_blocks(dtype: int, n_blocks: int, rng: np.random.Generator) -> np.ndarray:
    """Raw random bits with valid (finite, often subnormal) f16 scales, the
    shape of the reference's rand_block_* test generators
    (gemv_quant.rs:367-430)."""
    from oracle import BLOCK_BYTES, Q4_0, Q4_1, Q4_K, Q5_0, Q5_1, Q5_K, Q6_K, Q8_0, Q8_K

    if dtype in (0, 1):  # F32 / F16: finite values, some tiny and some large
        v = rng.standard_normal(n_blocks)
        v[rng.integers(0, 256, size=n_blocks) < 16] *= 1e-5
        v[rng.integers(0, 256, size=n_blocks) < 4] *= 100.0
        return v.astype(np.float32 if dtype == 0 else np.float16).view(np.uint8)
    bb = BLOCK_BYTES[dtype]
    raw = rng.integers(0, 256, size=(n_blocks, bb), dtype=np.uint8)

    def scales(n):
        v = rng.random(n) * 2.0 - 1.0
        v[rng.integers(0, 256, size=n) < 64] *= 1e-5
        return v.astype(np.float16).view(np.uint8).reshape(n, 2)

    if dtype in (Q4_K, Q5_K):
        raw[:, 0:2] = scales(n_blocks)
        raw[:, 2:4] = scales(n_blocks)
    elif dtype == Q6_K:
        raw[:, 208:210] = scales(n_blocks)
    elif dtype in (Q8_0, Q4_0, Q5_0):
        raw[:, 0:2] = scales(n_blocks)
    elif dtype in (Q4_1, Q5_1):
        raw[:, 0:2] = scales(n_blocks)
        raw[:, 2:4] = scales(n_blocks)
    elif dtype == Q8_K:
        # d: f32 uniform in [-1, 1] (gemv_quant.rs:381-387)
        raw[:, 0:4] = (rng.random(n_blocks) * 2.0 - 1.0).astype(np.float32).view(np.uint8).reshape(n_blocks, 4)
    return raw.reshape(-1)
