"""Pins the oracle's f16 codec, scale unpacking, dequantizers and quantizers.

Reference behaviour: crates/inferi/src/quantization.rs (decode_f16 :405-422,
get_scale_min_k4 :394-402, Block*::dequantize :47-55, :66-82, :94-112,
:123-143, :155-177, :204-212, :224-257, :287-330, :358-392).  Every check compares against something the oracle does not share
code with: numpy's IEEE binary16 codec, hand-built blocks with closed-form
outputs (tests/kquant.py), one-hot blocks that fix the element order, or
round-trip error bounds.
"""

import numpy as np
import pytest

import oracle as O
from tests import kquant as K


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_decode_f16_exhaustive_vs_numpy(oracle_lib):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = O.decode_f16(codes)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(bits(ours)[~nan], bits(ref)[~nan])
    # The reference returns a canonical NaN (quantization.rs:415): payload dropped.
    assert np.all(bits(ours)[nan] & 0x7FFFFFFF == 0x7FC00000)


def test_encode_f16_rne_vs_numpy(oracle_lib):
    rng = np.random.default_rng(11)
    parts = [
        rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32),
        (rng.standard_normal(1 << 16) * 1e-6).astype(np.float32),  # subnormal half range
        (rng.standard_normal(1 << 16) * 6e4).astype(np.float32),  # overflow boundary
        # exact ties between adjacent halves, in the normal and subnormal ranges
        ((np.arange(1, 4096, dtype=np.float32) + 0.5) * np.float32(2.0**-24)),
        ((np.arange(1024, 2048, dtype=np.float32) + 0.5) * np.float32(2.0**-10)),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, np.inf, -np.inf, np.nan, 2.0**-25, 2.0**-24,
                  1.5 * 2.0**-25, 2.0**-14, 2.0**-14 - 2.0**-25], np.float32),
    ]
    x = np.concatenate(parts)
    ours = O.encode_f16(x)
    ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all((ours[nan] & 0x7C00) == 0x7C00) and np.all((ours[nan] & 0x3FF) != 0)


def test_get_scale_min_k4_round_trip(oracle_lib):
    rng = np.random.default_rng(3)
    for _ in range(500):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        packed = K.pack_scales_bits(sc, mn)
        for j in range(8):
            assert O.get_scale_min_k4(j, packed) == (sc[j], mn[j])


def _closed_q4k(d, dmin, sc, mn, q):
    y = np.empty(256, np.float32)
    for e in range(256):
        j = e // 32
        d1 = np.float32(d) * np.float32(sc[j])
        m1 = np.float32(dmin) * np.float32(mn[j])
        y[e] = np.float32(d1 * np.float32(q[e])) - m1
    return y


def test_dequant_q4_k_known_answer(oracle_lib):
    sc = [1, 2, 3, 4, 5, 6, 7, 8]
    mn = [0, 2, 4, 6, 8, 10, 12, 14]
    q = [(e * 7 + 3) % 16 for e in range(256)]
    blk = K.q4k_block(K.F16_ONE, K.F16_HALF, sc, mn, q)
    y = O.dequant(O.Q4_K, blk, 256)
    # closed form: y[e] = (e//32 + 1) * q[e] - 0.5 * 2 * (e//32), all exact
    expect = np.array([(e // 32 + 1) * q[e] - (e // 32) for e in range(256)], np.float32)
    assert np.array_equal(y, expect)


def test_dequant_q4_k_element_order_one_hot(oracle_lib):
    for e in [0, 1, 31, 32, 33, 63, 64, 100, 127, 128, 191, 200, 255]:
        q = [0] * 256
        q[e] = 1
        blk = K.q4k_block(K.F16_ONE, 0, [1] * 8, [0] * 8, q)
        y = O.dequant(O.Q4_K, blk, 256)
        hot = np.zeros(256, np.float32)
        hot[e] = 1.0
        assert np.array_equal(y, hot), e


def test_dequant_q4_k_subnormal_and_high_scales(oracle_lib):
    rng = np.random.default_rng(5)
    for d16, dmin16 in [(0x0001, 0x0003), (0x03FF, 0x0200), (0x7BFF, 0x3C00), (0x8400, 0x0001)]:
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        blk = K.q4k_block(d16, dmin16, sc, mn, q)
        y = O.dequant(O.Q4_K, blk, 256)
        expect = _closed_q4k(K.f16_value(d16), K.f16_value(dmin16), sc, mn, q)
        assert np.array_equal(bits(y), bits(expect))


def test_dequant_q5_k_known_answer_and_order(oracle_lib):
    rng = np.random.default_rng(6)
    sc = rng.integers(0, 64, 8)
    mn = rng.integers(0, 64, 8)
    q = rng.integers(0, 32, 256)
    for d16, dmin16 in [(K.F16_ONE, K.F16_HALF), (0x0005, 0x0001), (0x4800, 0x3555)]:
        blk = K.q5k_block(d16, dmin16, sc, mn, q)
        y = O.dequant(O.Q5_K, blk, 256)
        expect = _closed_q4k(K.f16_value(d16), K.f16_value(dmin16), sc, mn, q)
        assert np.array_equal(bits(y), bits(expect))
    for e in [0, 5, 31, 32, 63, 64, 95, 96, 130, 160, 224, 255]:
        qq = [0] * 256
        qq[e] = 16  # only the fifth (qh) bit set
        y = O.dequant(O.Q5_K, K.q5k_block(K.F16_ONE, 0, [1] * 8, [0] * 8, qq), 256)
        hot = np.zeros(256, np.float32)
        hot[e] = 16.0
        assert np.array_equal(y, hot), e


def test_dequant_q6_k_known_answer_and_order(oracle_lib):
    rng = np.random.default_rng(7)
    sc = rng.integers(-128, 128, 16)
    q = rng.integers(-32, 32, 256)
    for d16 in [K.F16_QUARTER, 0x0007, 0xC500]:
        blk = K.q6k_block(d16, sc, q)
        y = O.dequant(O.Q6_K, blk, 256)
        d = np.float32(K.f16_value(d16))
        expect = np.array([np.float32(d * np.float32(sc[e // 16])) * np.float32(q[e]) for e in range(256)], np.float32)
        assert np.array_equal(bits(y), bits(expect))
    for e in [0, 1, 15, 16, 31, 32, 48, 64, 80, 96, 127, 128, 160, 192, 224, 255]:
        qq = [0] * 256
        qq[e] = 5
        scales = list(range(1, 17))
        y = O.dequant(O.Q6_K, K.q6k_block(K.F16_ONE, scales, qq), 256)
        hot = np.zeros(256, np.float32)
        hot[e] = 5.0 * scales[e // 16]
        assert np.array_equal(y, hot), e


def test_dequant_q8_0_known_answer(oracle_lib):
    q = list(range(-16, 16))
    y = O.dequant(O.Q8_0, K.q8_0_block(K.F16_HALF, q), 32)
    assert np.array_equal(y, np.array(q, np.float32) * 0.5)
    q = [-128, 127] + [0] * 30
    y = O.dequant(O.Q8_0, K.q8_0_block(0x0001, q), 32)
    assert y[0] == -128 * 2.0**-24 and y[1] == 127 * 2.0**-24 and not y[2:].any()


def test_dequant_q4_0_order_and_offset(oracle_lib):
    """quantization.rs:66-82: byte j holds element j (low nibble) and j+16
    (high); stored code 8 is zero."""
    for e in range(32):
        q = [0] * 32
        q[e] = 5
        y = O.dequant(O.Q4_0, K.q4_0_block(K.F16_ONE, q), 32)
        hot = np.zeros(32, np.float32)
        hot[e] = 5.0
        assert np.array_equal(y, hot), e
    q = list(range(-8, 8)) * 2
    y = O.dequant(O.Q4_0, K.q4_0_block(K.F16_HALF, q), 32)
    assert np.array_equal(y, np.array(q, np.float32) * 0.5)


def test_dequant_q4_1_order_and_min(oracle_lib):
    """quantization.rs:94-112: y = q * d + m, two roundings (no FMA)."""
    for e in (0, 7, 15, 16, 31):
        q = [0] * 32
        q[e] = 7
        y = O.dequant(O.Q4_1, K.q4_1_block(K.F16_HALF, K.F16_QUARTER, q), 32)
        want = np.full(32, 0.25, np.float32)
        want[e] = 3.75
        assert np.array_equal(y, want), e
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, 32)
    d16, m16 = 0x2E66, 0xB4CD  # about 0.1 and -0.3: the products round
    y = O.dequant(O.Q4_1, K.q4_1_block(d16, m16, q), 32)
    d, m = np.float32(K.f16_value(d16)), np.float32(K.f16_value(m16))
    want = (q.astype(np.float32) * d).astype(np.float32) + m
    assert np.array_equal(y, want.astype(np.float32))


def test_dequant_q5_0_fifth_bit_placement(oracle_lib):
    """quantization.rs:123-143: bit j of qh is the fifth bit of element j and
    bit j+16 of element j+16 (xh_1 = (qh >> (j+12)) & 0x10); stored 16 is zero."""
    for e in range(32):
        q = [-16] * 32  # stored 0
        q[e] = 0  # stored 16: only the fifth bit
        y = O.dequant(O.Q5_0, K.q5_0_block(K.F16_ONE, q), 32)
        want = np.full(32, -16.0, np.float32)
        want[e] = 0.0
        assert np.array_equal(y, want), e
    q = list(range(-16, 16))
    y = O.dequant(O.Q5_0, K.q5_0_block(K.F16_QUARTER, q), 32)
    assert np.array_equal(y, np.array(q, np.float32) * 0.25)


def test_dequant_q5_1_fifth_bit_and_min(oracle_lib):
    """quantization.rs:155-177."""
    for e in (0, 3, 15, 16, 17, 31):
        q = [0] * 32
        q[e] = 16
        y = O.dequant(O.Q5_1, K.q5_1_block(K.F16_ONE, K.F16_HALF, q), 32)
        want = np.full(32, 0.5, np.float32)
        want[e] = 16.5
        assert np.array_equal(y, want), e
    q = np.arange(32)
    y = O.dequant(O.Q5_1, K.q5_1_block(K.F16_TWO, 0xBC00, q), 32)  # d 2, m -1
    assert np.array_equal(y, q.astype(np.float32) * 2 - 1)


def test_dequant_q8_k_known_answer(oracle_lib):
    """quantization.rs:204-212: y = d * q with d an f32; bsums are not read."""
    rng = np.random.default_rng(4)
    q = rng.integers(-128, 128, 256)
    for d in (0.5, 0.1, -3.0e-5):
        y = O.dequant(O.Q8_K, K.q8_k_block(d, q, bsums=rng.integers(-30000, 30000, 16)), 256)
        want = np.float32(d) * q.astype(np.float32)
        assert np.array_equal(y, want.astype(np.float32))


@pytest.mark.parametrize("dtype,tol", [(O.Q8_0, 0.012), (O.Q4_K, 0.13), (O.Q5_K, 0.065), (O.Q6_K, 0.045),
                                       (O.Q4_0, 0.13), (O.Q4_1, 0.1), (O.Q5_0, 0.065), (O.Q5_1, 0.05),
                                       (O.Q8_K, 0.012)])
def test_quantize_round_trip(oracle_lib, dtype, tol):
    rng = np.random.default_rng(100 + dtype)
    x = (rng.standard_normal(256 * 64) * 0.02).astype(np.float32)
    blocks = O.quantize(dtype, x)
    assert blocks.size == x.size // O.BLOCK_ELEMS[dtype] * O.BLOCK_BYTES[dtype]
    y = O.dequant(dtype, blocks, x.size)
    rel = np.sqrt(np.mean((y - x) ** 2)) / np.sqrt(np.mean(x**2))
    assert rel < tol, rel
    # every element lands within one quantization step of its input
    step = {O.Q8_0: 1 / 127, O.Q4_K: 1 / 15 * 2, O.Q5_K: 1 / 31 * 2, O.Q6_K: 1 / 31 * 2, O.Q4_0: 1 / 8,
            O.Q4_1: 2 / 15, O.Q5_0: 1 / 16, O.Q5_1: 2 / 31, O.Q8_K: 1 / 127}[dtype]
    qk = O.BLOCK_ELEMS[dtype]
    amax = np.abs(x).reshape(-1, qk).max(axis=1).repeat(qk)
    assert np.all(np.abs(y - x) <= step * amax * 1.05 + 1e-7)


def test_quantize_zero_and_constant_blocks(oracle_lib):
    for dtype in (O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K, O.Q4_0, O.Q4_1, O.Q5_0, O.Q5_1, O.Q8_K):
        z = np.zeros(256, np.float32)
        assert not O.dequant(dtype, O.quantize(dtype, z), 256).any()
    # a Q4_K sub-block of a constant negative value is represented exactly via the min
    x = np.full(256, -0.5, np.float32)
    y = O.dequant(O.Q4_K, O.quantize(O.Q4_K, x), 256)
    assert np.allclose(y, x, atol=1e-3)
