"""Pins the host-core restatement of the reference's GEMV and attention
shaders (oracle/ref_shaders.c), the CPU baseline bench.py times beside the
GPU's GEMV sweep and decode attention block.

- GEMV: x = e_k selects column k of the dequantized matrix exactly (one
  nonzero product), which fixes every lane's element mapping and each
  element's dequantization; random x agrees with the oracle's f64 GEMV
  within the f32 rounding bound.
- Attention: the first position alone gives v_0; equal keys give the mean of
  V; random caches agree with the oracle's attention, on both shader forms
  (fused_attention up to 2048 positions, flash_attention beyond).
"""

import numpy as np
import pytest

import oracle as O

FMTS = [("Q4_K", 256), ("Q5_K", 256), ("Q6_K", 512), ("Q8_0", 128)]


def _weights(dtype, rows, cols, rng):
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    q = O.quantize(dtype, w.ravel())
    return q, O.dequant(dtype, q, rows * cols).reshape(rows, cols)


@pytest.mark.parametrize("fmt,step", FMTS)
def test_ref_gemv_selects_columns_exactly(oracle_lib, fmt, step):
    dtype = getattr(O, fmt)
    rng = np.random.default_rng(dtype)
    rows, cols = 8, 2 * step
    q, deq = _weights(dtype, rows, cols, rng)
    for k in range(cols):
        x = np.zeros(cols, np.float32)
        x[k] = 1.0
        got = O.ref_gemv(dtype, q, rows, cols, x, 2)
        assert np.array_equal(got, deq[:, k]), f"{fmt}: column {k}"


@pytest.mark.parametrize("fmt,step", FMTS)
@pytest.mark.parametrize("rows,cols_steps", [(4, 1), (64, 4), (300, 16)])
def test_ref_gemv_matches_oracle(oracle_lib, fmt, step, rows, cols_steps):
    dtype = getattr(O, fmt)
    rng = np.random.default_rng(rows * 17 + cols_steps + dtype)
    cols = step * cols_steps
    q, deq = _weights(dtype, rows, cols, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    got = O.ref_gemv(dtype, q, rows, cols, x, 3).astype(np.float64)
    ref = O.gemv_quant(dtype, q, rows, cols, x)
    # f32 sums of at most cols / 4 + 40 terms along any path
    bound = (np.abs(deq.astype(np.float64)) @ np.abs(x.astype(np.float64))) * (cols / 4 + 40) * 2.0**-24
    assert np.all(np.abs(got - ref) <= bound + 1e-30)


def test_ref_gemv_rejects_shapes_the_shaders_do_not_take(oracle_lib):
    q = np.zeros(6 * O.row_bytes(O.Q4_K, 256), np.uint8)
    x = np.zeros(256, np.float32)
    with pytest.raises(ValueError):
        O.ref_gemv(O.Q4_K, q, 6, 256, x)  # rows % 4
    with pytest.raises(ValueError):
        O.ref_gemv(O.Q6_K, np.zeros(4 * 210, np.uint8), 4, 256, x)  # one Q6_K block: no pair


@pytest.mark.parametrize("L", [1, 700, 2048, 2049, 3000])
def test_ref_attention(oracle_lib, L):
    nh, nkv, hs = 8, 2, 64
    rng = np.random.default_rng(L)
    q = rng.standard_normal(nh * hs).astype(np.float32)
    kc = O.encode_f16(rng.standard_normal((L, nkv * hs)).astype(np.float32))
    vc = O.encode_f16(rng.standard_normal((L, nkv * hs)).astype(np.float32))
    got = O.ref_attention(q, kc, vc, nh, nkv, hs, L - 1, 4)
    ref = O.attention(q, kc, vc, nh, nkv, hs, L - 1, True)
    assert np.abs(got - ref).max() <= 2e-6 * max(1.0, np.abs(ref).max())
    if L == 1:  # one position: its value row, for every query head of the group
        v0 = O.decode_f16(vc[0]).reshape(nkv, hs)
        assert np.array_equal(got.reshape(nh, hs), np.repeat(v0, nh // nkv, axis=0))
    # equal keys: the mean of the value rows
    keq = np.repeat(kc[:1], L, axis=0)
    got = O.ref_attention(q, keq, vc, nh, nkv, hs, L - 1, 4)
    mean = O.decode_f16(vc).astype(np.float64).reshape(L, nkv, hs).mean(axis=0)
    assert np.abs(got.reshape(nh, hs) - np.repeat(mean, nh // nkv, axis=0)).max() <= 1e-5
