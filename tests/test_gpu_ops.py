"""GPU parity of every op kernel against the CPU oracle, through the C ABI.

Bars: dequantized weights bit-exact; GEMV/op outputs
within |a - e| <= 1e-3 * max(|e|, 1) with fp32 accumulation (the reference's
floor style, crates/inferi/src/ops/gemv_quant.rs:528-535, tightened from 1e-2);
integer work (quantizer bytes, argmax) exact.
"""

import numpy as np
import pytest

import oracle as O
from tests import kquant as K

pytestmark = pytest.mark.gpu

FMTS = [O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K, O.Q4_0, O.Q4_1, O.Q5_0, O.Q5_1, O.Q8_K]
FNAME = {O.Q8_0: "Q8_0", O.Q4_K: "Q4_K", O.Q5_K: "Q5_K", O.Q6_K: "Q6_K", O.Q4_0: "Q4_0", O.Q4_1: "Q4_1",
         O.Q5_0: "Q5_0", O.Q5_1: "Q5_1", O.Q8_K: "Q8_K"}
TOL = 1e-3


def assert_close(a, e, tol=TOL, what=""):
    a = np.asarray(a, np.float64)
    e = np.asarray(e, np.float64)
    err = np.abs(a - e) / np.maximum(np.abs(e), 1.0)
    assert np.all(np.isfinite(a)), f"{what}: non-finite output"
    assert err.max() <= tol, f"{what}: max scaled error {err.max():.3e} at {int(err.argmax())}"


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------- dequant --

@pytest.mark.parametrize("dtype", FMTS, ids=FNAME.get)
def test_dequant_bit_exact_random_blocks(ctx, oracle_lib, dtype):
    rng = np.random.default_rng(1000 + dtype)
    nblk = 4096 if O.BLOCK_ELEMS[dtype] == 32 else 512
    blocks = K.random_blocks(dtype, nblk, rng)
    n = nblk * O.BLOCK_ELEMS[dtype]
    db, dy = ctx.upload(blocks), ctx.alloc(n * 4)
    ctx.dequant(dy, db, dtype, n)
    got = dy.download(np.float32, n)
    ref = O.dequant(dtype, blocks, n)
    assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("dtype", FMTS, ids=FNAME.get)
def test_dequant_bit_exact_known_answer_blocks(ctx, oracle_lib, dtype):
    """Hand-built blocks with closed-form values, including subnormal and
    extreme scales, plus an all-0xFF block (NaN scales: NaN-ness must match)."""
    rng = np.random.default_rng(7)
    blks = []
    for d16 in (0x3C00, 0x0001, 0x03FF, 0x7BFF, 0x8400):
        if dtype == O.Q4_K:
            blks.append(K.q4k_block(d16, 0x0200, rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 16, 256)))
        elif dtype == O.Q5_K:
            blks.append(K.q5k_block(d16, 0x0003, rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 32, 256)))
        elif dtype == O.Q6_K:
            blks.append(K.q6k_block(d16, rng.integers(-128, 128, 16), rng.integers(-32, 32, 256)))
        elif dtype == O.Q4_0:
            blks.extend(K.q4_0_block(d16, rng.integers(-8, 8, 32)) for _ in range(8))
        elif dtype == O.Q4_1:
            blks.extend(K.q4_1_block(d16, 0x8001, rng.integers(0, 16, 32)) for _ in range(8))
        elif dtype == O.Q5_0:
            blks.extend(K.q5_0_block(d16, rng.integers(-16, 16, 32)) for _ in range(8))
        elif dtype == O.Q5_1:
            blks.extend(K.q5_1_block(d16, 0x3555, rng.integers(0, 32, 32)) for _ in range(8))
        elif dtype == O.Q8_K:
            d = float(np.array([d16], np.uint16).view(np.float16)[0])
            blks.append(K.q8_k_block(d, rng.integers(-128, 128, 256)))
        else:
            blks.extend(K.q8_0_block(d16, rng.integers(-128, 128, 32)) for _ in range(8))
    blks.append(b"\xff" * O.BLOCK_BYTES[dtype])
    data = np.frombuffer(b"".join(blks), np.uint8)
    n = len(blks) * O.BLOCK_ELEMS[dtype]
    db, dy = ctx.upload(data), ctx.alloc(n * 4)
    ctx.dequant(dy, db, dtype, n)
    got, ref = dy.download(np.float32, n), O.dequant(dtype, data, n)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got)[~nan], bits(ref)[~nan])


# ------------------------------------------------------------ quantize --

@pytest.mark.parametrize("dtype", FMTS, ids=FNAME.get)
def test_quantize_bytes_match_oracle(ctx, oracle_lib, dtype):
    rng = np.random.default_rng(2000 + dtype)
    parts = [
        rng.standard_normal(256 * 512) * 0.02,
        rng.uniform(-3, 3, 256 * 64),
        np.abs(rng.standard_normal(256 * 16)),  # all-positive blocks (min 0)
        -np.abs(rng.standard_normal(256 * 16)),
        np.zeros(256 * 4),
        np.full(256 * 4, -0.5),
        rng.standard_normal(256 * 16) * 1e-6,
    ]
    x = np.concatenate(parts).astype(np.float32)
    dx, db = ctx.upload(x), ctx.alloc(x.size // O.BLOCK_ELEMS[dtype] * O.BLOCK_BYTES[dtype])
    ctx.quantize(db, dx, dtype, x.size)
    got = db.download(np.uint8, db.nbytes)
    ref = O.quantize(dtype, x)
    assert np.array_equal(got, ref), f"first differing byte {int(np.argmax(got != ref))}"


def test_fill_normal_statistics_and_determinism(ctx):
    n = 1 << 22
    a, b, c = ctx.alloc(n * 4), ctx.alloc(n * 4), ctx.alloc(n * 4)
    ctx.fill_normal(a, n, 42, 3, 0.0, 0.02)
    ctx.fill_normal(b, n, 42, 3, 0.0, 0.02)
    ctx.fill_normal(c, n, 42, 4, 0.0, 0.02)
    va, vb, vc = a.download(), b.download(), c.download()
    assert np.array_equal(va, vb)
    assert not np.array_equal(va, vc)
    assert abs(va.mean()) < 5e-5 and abs(va.std() - 0.02) < 1e-4
    # tails of a normal: P(|z| > 3) = 0.0027
    frac = np.mean(np.abs(va) > 3 * 0.02)
    assert 0.0022 < frac < 0.0032


# ---------------------------------------------------------------- GEMV --

def _gemv_case(ctx, dtype, rows, cols, w, x):
    dw, dx, dy = ctx.upload(w), ctx.upload(x), ctx.alloc(rows * 4)
    ctx.matmul_quant_assign(dy, dw, dtype, rows, cols, dx)
    return dy.download(np.float32, rows)


@pytest.fixture(params=[False, True], ids=["int", "exact"])
def gemv_path(request, ctx):
    """Runs a test on the integer GEMV path (default) and on the exact fp32 one."""
    ctx.set_option("gemv_exact", int(request.param))
    yield request.param
    ctx.set_option("gemv_exact", 0)


def test_activation_quantization_bounds(ctx):
    """x -> 16-value groups of 22-bit fixed point (three int8 digits):
    |x~ - x| <= max|x|_group / (2 * (2^21 - 1)) (+ the f32 rounding of the
    group scale), XSUM = sum of x~ per group, partial sums of x^2 per 256."""
    import inferi_amd as I

    rng = np.random.default_rng(12)
    n = 4096
    x = rng.standard_normal(n).astype(np.float32)
    x[::97] *= 300.0  # outliers
    x[1024:1040] = 0.0  # an all-zero group
    x[2048:2064] = -1e-30  # a denormal-scale group
    g = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    dx, dg = ctx.upload(x), ctx.upload(g)
    xq = ctx.alloc(I.LlmContext.activation_bytes(n))
    ss = ctx.alloc((n // 256) * 4)
    ctx.quantize_activation(xq, dx, n, gamma=dg, ss_out=ss)
    raw = xq.download(np.uint8, 3 * n + n // 2)
    da = raw[:n].view(np.int8).astype(np.float64)
    db = raw[n:2 * n].view(np.int8).astype(np.float64)
    dc = raw[2 * n:3 * n].view(np.int8).astype(np.float64)
    xs = raw[3 * n:3 * n + n // 4].view(np.float32).astype(np.float64)
    xsum = raw[3 * n + n // 4:].view(np.float32).astype(np.float64)
    xg = (x * g).astype(np.float64)
    rec = np.repeat(xs, 16) * (65536 * da + 256 * db + dc)
    amax = np.abs(xg).reshape(-1, 16).max(1).repeat(16)
    # half a code step, plus the f32 roundings of the scale and its inverse
    assert np.all(np.abs(rec - xg) <= amax / (2 * 2097151) + 4e-7 * amax + 1e-37)
    assert np.allclose(xsum, rec.reshape(-1, 16).sum(1), rtol=1e-6, atol=1e-30)
    assert np.all(np.abs(da) <= 32) and np.all(np.abs(db) <= 128) and np.all(np.abs(dc) <= 128)
    assert np.all(np.abs(65536 * da + 256 * db + dc) <= 2097151)
    assert np.allclose(ss.download(np.float32, n // 256), (x.astype(np.float64) ** 2).reshape(-1, 256).sum(1), rtol=1e-5)


@pytest.mark.parametrize("dtype", FMTS, ids=FNAME.get)
@pytest.mark.parametrize("rows,cols", [(1, 256), (7, 512), (33, 1024), (64, 2048), (100, 5632), (20, 14336)])
def test_gemv_random_blocks(ctx, oracle_lib, gemv_path, dtype, rows, cols):
    """Raw random block bits with a quarter of the f16 scales subnormal, as the
    reference's GEMV tests draw them (gemv_quant.rs:354-430); odd row counts
    exercise the tile tail, cols 5632 a block count that is not a multiple of
    the per-step block group."""
    rng = np.random.default_rng(rows * 7 + cols + dtype)
    w = K.random_blocks(dtype, rows * cols // O.BLOCK_ELEMS[dtype], rng)
    x = (rng.random(cols) * 2 - 1).astype(np.float32)
    got = _gemv_case(ctx, dtype, rows, cols, w, x)
    assert_close(got, O.gemv_quant(dtype, w, rows, cols, x), what=f"{FNAME[dtype]} {rows}x{cols}")


@pytest.mark.parametrize("dtype", FMTS, ids=FNAME.get)
def test_gemv_selects_columns(ctx, oracle_lib, gemv_path, dtype):
    """x = e_k picks column k of the dequantized matrix (exactly on the fp32
    path; to the activation rounding, here exact too, on the integer path)."""
    rows, cols = 48, 1024
    rng = np.random.default_rng(dtype)
    w = O.quantize(dtype, (rng.standard_normal(rows * cols) * 0.02).astype(np.float32))
    deq = O.dequant(dtype, w, rows * cols).reshape(rows, cols)
    for k in (0, 1, 31, 255, 256, 700, 1023):
        e = np.zeros(cols, np.float32)
        e[k] = 1.0
        got = _gemv_case(ctx, dtype, rows, cols, w, e)
        # the block affine map d1*q - m1 is applied as d1*sum(q x) - m1*sum(x):
        # its cancellation is bounded by the matrix magnitude, not the output
        np.testing.assert_allclose(got, deq[:, k], rtol=2e-6, atol=1e-6 * np.abs(deq).max())


@pytest.mark.parametrize("dtype", [O.F16, O.F32], ids=["F16", "F32"])
@pytest.mark.parametrize("rows,cols", [(1, 32), (33, 1024), (100, 5632), (4096, 4096), (64, 14336)])
def test_gemv_unquantized(ctx, oracle_lib, gemv_path, dtype, rows, cols):
    """F32 matrices (GpuQuantTensor::F32 -> Gemm, gemv_quant.rs:203-208) and
    F16 ones (converted to F32 at load by the reference, gguf.rs:113-128):
    N(0, 0.02) values with a sprinkling of f16 subnormals and of large
    magnitudes, against the oracle's f64 product of the same values."""
    rng = np.random.default_rng(rows + cols + dtype)
    wf = rng.standard_normal(rows * cols) * 0.02
    wf[rng.integers(0, rows * cols, rows * cols // 50)] *= 1e-4  # f16 subnormal range
    wf[rng.integers(0, rows * cols, rows * cols // 200)] *= 300.0
    w = wf.astype(np.float16 if dtype == O.F16 else np.float32).view(np.uint8)
    x = rng.standard_normal(cols).astype(np.float32)
    got = _gemv_case(ctx, dtype, rows, cols, w, x)
    assert_close(got, O.gemv_quant(dtype, w, rows, cols, x), what=f"{rows}x{cols}")


def test_gemv_c1_q4k_4096(ctx, oracle_lib, gemv_path):
    """W 4096x4096 ~ N(0, 0.02) quantized to Q4_K, x ~ N(0, 1).
    Dequant bit-exact and y within 1e-3."""
    rows = cols = 4096
    rng = np.random.default_rng(1)
    wf = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    x = np.random.default_rng(2).standard_normal(cols).astype(np.float32)
    w = O.quantize(O.Q4_K, wf)
    dw = ctx.upload(w)
    dd = ctx.alloc(rows * cols * 4)
    ctx.dequant(dd, dw, O.Q4_K, rows * cols)
    assert np.array_equal(bits(dd.download()), bits(O.dequant(O.Q4_K, w, rows * cols)))
    got = _gemv_case(ctx, O.Q4_K, rows, cols, w, x)
    assert_close(got, O.gemv_quant(O.Q4_K, w, rows, cols, x), what="C1")


@pytest.mark.parametrize("dtype", FMTS, ids=FNAME.get)
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
def test_gemv_c2_sweep_shapes(ctx, oracle_lib, gemv_path, dtype, rows, cols):
    """BASELINE config 2 shapes; weights generated and quantized on the device
    (N(0, 0.02)), checked against the oracle on the same bytes."""
    n = rows * cols
    tmp = ctx.alloc(n * 4)
    ctx.fill_normal(tmp, n, 100 + 4 * dtype, rows + cols, 0.0, 0.02)
    dw = ctx.alloc(rows * cols // O.BLOCK_ELEMS[dtype] * O.BLOCK_BYTES[dtype])
    ctx.quantize(dw, tmp, dtype, n)
    tmp.free()
    x = np.random.default_rng(rows ^ cols).standard_normal(cols).astype(np.float32)
    dx, dy = ctx.upload(x), ctx.alloc(rows * 4)
    ctx.matmul_quant_assign(dy, dw, dtype, rows, cols, dx)
    got = dy.download(np.float32, rows)
    w = dw.download(np.uint8, dw.nbytes)
    dw.free()
    assert_close(got, O.gemv_quant(dtype, w, rows, cols, x), what=f"{FNAME[dtype]} {rows}x{cols}")


def test_gemv_rejects_bad_shapes(ctx):
    import inferi_amd as I

    w, x, y = ctx.alloc(1 << 16), ctx.alloc(1 << 16), ctx.alloc(1 << 16)
    with pytest.raises(I.HipError) as e:
        ctx.matmul_quant_assign(y, w, I.Q4_K, 4, 300, x)  # cols not a multiple of 256
    assert e.value.status == 1
    with pytest.raises(I.HipError) as e:
        ctx.matmul_quant_assign(y, w.at(8), I.Q4_K, 4, 256, x)  # misaligned weights
    assert e.value.status == 1
    with pytest.raises(I.HipError) as e:
        ctx.matmul_quant_assign(y, w.at(4), I.F32, 4, 256, x)  # f32 rows must be 16-byte aligned
    assert e.value.status == 1
    with pytest.raises(I.HipError) as e:
        ctx.matmul_quant_assign(y, w, 5, 4, 256, x)  # no GGUF type 5
    assert e.value.status in (1, 2)


# ------------------------------------------------------- elementwise ops --

def test_rms_norm_matches_oracle(ctx, oracle_lib):
    import inferi_amd as I

    rng = np.random.default_rng(3)
    for n, eps in ((4096, 1e-5), (2048, 1e-6), (1000, 1e-5), (14336, 1e-5)):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        g = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        cfg = ctx.upload(np.frombuffer(bytes(I.RmsNormConfig(eps)), np.uint8))
        dx, dg, do = ctx.upload(x), ctx.upload(g), ctx.alloc(n * 4)
        ctx.rms_norm_assign(cfg, do, dx, dg, n)
        assert_close(do.download(np.float32, n), O.rms_norm(x, g, eps), tol=1e-5, what=f"rms n={n}")


@pytest.mark.parametrize("neox", [False, True])
def test_rope_matches_oracle(ctx, oracle_lib, neox):
    import inferi_amd as I

    rng = np.random.default_rng(4)
    for hs, nq, nkv, theta, pos in ((128, 32, 8, 500000.0, 0), (128, 32, 8, 500000.0, 4095),
                                    (128, 32, 8, 500000.0, 8191), (64, 32, 4, 10000.0, 77),
                                    (64, 16, 16, 10000.0, 1)):
        q = rng.standard_normal(nq * hs).astype(np.float32)
        k = rng.standard_normal(nkv * hs).astype(np.float32)
        cfg = ctx.upload(np.frombuffer(bytes(I.RoPEConfig(hs, nkv * hs, pos, theta)), np.uint8))
        dq, dk = ctx.upload(q), ctx.upload(k)
        ctx.rope(I.ROPE_NEOX if neox else I.ROPE_ORIGINAL, cfg, dq, q.size, dk, k.size)
        eq, ek = O.rope(q, k, hs, pos, theta, neox)
        assert_close(dq.download(np.float32, q.size), eq, tol=1e-5, what="rope q")
        assert_close(dk.download(np.float32, k.size), ek, tol=1e-5, what="rope k")


def test_silu_and_add(ctx, oracle_lib):
    rng = np.random.default_rng(5)
    n = 14336
    h1 = (rng.standard_normal(n) * 4).astype(np.float32)
    h2 = rng.standard_normal(n).astype(np.float32)
    d1, d2 = ctx.upload(h1), ctx.upload(h2)
    ctx.silu(d1, d2, n)
    assert_close(d1.download(np.float32, n), O.silu_mul(h1, h2), tol=1e-6, what="silu")
    # known answer of the reference's add test (tests/onnx_ops.rs:155-178)
    a, b = ctx.upload(np.array([1, 2, 3, 4], np.float32)), ctx.upload(np.array([5, 6, 7, 8], np.float32))
    ctx.add_assign(a, b, 4)
    assert a.download(np.float32, 4).tolist() == [6.0, 8.0, 10.0, 12.0]


def test_argmax_ties_and_sizes(ctx, oracle_lib):
    out = ctx.alloc(4)
    rng = np.random.default_rng(6)
    for v in (np.array([1.0, 3.0, -2.0, 3.0, 3.0], np.float32), np.full(1000, -5.0, np.float32),
              rng.standard_normal(128256).astype(np.float32), rng.standard_normal(32000).astype(np.float32),
              -np.abs(rng.standard_normal(513)).astype(np.float32)):
        v = v.copy()
        if v.size == 128256:
            v[[5, 90000, 128255]] = v.max() + 1.0  # three-way tie far apart
        dv = ctx.upload(v)
        ctx.argmax(dv, v.size, out)
        assert int(out.download(np.uint32, 1)[0]) == O.argmax(v)


# ------------------------------------------------------------ attention --

def _attn_case(ctx, nh, nkv, hs, seq_len, pos, kv_f16, rng):
    import inferi_amd as I

    kv_dim = nkv * hs
    q = rng.standard_normal(nh * hs).astype(np.float32)
    kc = rng.standard_normal((seq_len, kv_dim)).astype(np.float32)
    vc = rng.standard_normal((seq_len, kv_dim)).astype(np.float32)
    if kv_f16:
        kc, vc = O.encode_f16(kc), O.encode_f16(vc)
    p = I.AttentionParams(seq_len, kv_dim, nh // nkv, nh, hs, pos)
    dp = ctx.upload(np.frombuffer(bytes(p), np.uint8))
    dq, dk, dv, do = ctx.upload(q), ctx.upload(kc), ctx.upload(vc), ctx.alloc(nh * hs * 4)
    I.BatchedMultiqueryAttention.launch(ctx, p, dp, dq, dk, dv, I.F16 if kv_f16 else I.F32, do)
    got = do.download(np.float32, nh * hs)
    ref = O.attention(q, kc, vc, nh, nkv, hs, pos, kv_f16)
    return got, ref


@pytest.mark.parametrize("kv_f16", [True, False], ids=["f16", "f32"])
@pytest.mark.parametrize("nh,nkv,hs", [(32, 8, 128), (32, 4, 64), (8, 8, 64), (16, 8, 128), (16, 2, 128)])
def test_attention_matches_oracle(ctx, oracle_lib, kv_f16, nh, nkv, hs):
    rng = np.random.default_rng(nh + nkv + hs)
    for pos in (0, 1, 63, 64, 300, 1023):
        got, ref = _attn_case(ctx, nh, nkv, hs, 1024, pos, kv_f16, rng)
        assert_close(got, ref, what=f"pos={pos}")


@pytest.mark.parametrize("L", [512, 2048, 8192])
def test_attention_c3_lengths(ctx, oracle_lib, L):
    """32 q heads, 8 KV heads, head_dim 128, f16 cache of
    length L filled with N(0, 1), attending at pos = L - 1."""
    rng = np.random.default_rng(L)
    got, ref = _attn_case(ctx, 32, 8, 128, L, L - 1, True, rng)
    assert_close(got, ref, what=f"L={L}")


def test_attention_equal_keys_gives_mean_of_values(ctx, oracle_lib):
    import inferi_amd as I

    nh, nkv, hs, L, pos = 32, 8, 128, 600, 599
    rng = np.random.default_rng(9)
    kv_dim = nkv * hs
    kc = np.tile(rng.standard_normal((1, kv_dim)).astype(np.float32), (L, 1))
    vc = rng.standard_normal((L, kv_dim)).astype(np.float32)
    q = rng.standard_normal(nh * hs).astype(np.float32)
    p = I.AttentionParams(L, kv_dim, nh // nkv, nh, hs, pos)
    dp = ctx.upload(np.frombuffer(bytes(p), np.uint8))
    do = ctx.alloc(nh * hs * 4)
    I.BatchedMultiqueryAttention.launch(ctx, p, dp, ctx.upload(q), ctx.upload(kc), ctx.upload(vc), I.F32, do)
    got = do.download(np.float32, nh * hs).reshape(nh, hs)
    mean = vc[: pos + 1].astype(np.float64).mean(0).reshape(nkv, hs)
    for h in range(nh):
        assert_close(got[h], mean[h // (nh // nkv)], tol=1e-5)
