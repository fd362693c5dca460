"""GPU check that every GEMV form the gemv_grp option selects gives the
default decode step's results bit for bit (same arithmetic, same reduction
orders): logits, tokens, KV-cache rows and the residual stream."""

import numpy as np
import pytest

from tests.test_gpu_model import run_steps

pytestmark = pytest.mark.gpu


def decode(ctx, cfg, w, prompt, n, mode="graph"):
    import inferi_amd as I

    s = I.Llama2State(ctx, cfg)
    try:
        logits, toks = run_steps(ctx, s, w, prompt, n, mode)
        kv = {}
        for layer in range(cfg.n_layers):
            for name in ("key_cache", "value_cache"):
                dt = np.uint16 if cfg.kv_dtype == I.F16 else np.float32
                kv[name, layer] = s.read(name, dt, layer).reshape(cfg.max_pos, cfg.kv_dim)[:n]
        x = s.read("x")
    finally:
        s.close()
    return np.array(logits), toks, kv, x


def assert_same(a, b, what):
    a, b = np.asarray(a), np.asarray(b)
    if not np.array_equal(a.view(np.uint8), b.view(np.uint8)):
        d = np.abs(a.astype(np.float64) - b.astype(np.float64))
        raise AssertionError(f"{what}: not bit-identical (max |diff| {d.max():.3e} at {np.unravel_index(d.argmax(), d.shape)})")


@pytest.mark.parametrize("grp", [0, 2, 4, 12, 16, 31, 33, 63, 64, 97, 128, 160, 225, 256, 481])
def test_gemv_forms_same_results(ctx, grp):
    """The looping body, the one-item forms of O, down, gate/up and the
    head, the head's 256-VGPR form, the four-row one-item forms of gate/up
    (bit 7) and of the plain and QKV GEMVs (bit 8), on the C4 shape."""
    import inferi_amd as I

    cfg = I.Llama2Config(n_layers=4, hidden=2048, ffn=5632, n_heads=32, n_kv_heads=4, vocab=32000, max_pos=32,
                         rope_theta=10000.0, rms_eps=1e-5, kv_dtype=I.F16)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=1000)
    try:
        prompt = [5, 31999, 7, 1234]
        ref = decode(ctx, cfg, w, prompt, 12)
        ctx.set_option("gemv_grp", grp)
        try:
            got = decode(ctx, cfg, w, prompt, 12)
        finally:
            ctx.set_option("gemv_grp", 225)
        assert_same(got[0], ref[0], "logits")
        assert np.array_equal(got[1], ref[1]), "tokens"
        for k in ref[2]:
            assert_same(got[2][k], ref[2][k], f"{k[0]} layer {k[1]}")
        assert_same(got[3], ref[3], "residual x")
    finally:
        w.close()


@pytest.mark.parametrize("dtype_name,rows,cols", [("Q4_K", 4096, 4096), ("Q4_K", 300, 1024), ("Q6_K", 512, 2048)])
def test_matmul_quant_four_row_form(ctx, dtype_name, rows, cols):
    """ifr_matmul_quant with gemv_grp bit 8 (the four-rows-per-wave one-item
    kernel where the format has one) against the default form, bit for bit,
    and against the oracle's f64 GEMV at 1e-3."""
    import inferi_amd as I
    import oracle as O

    dtype = getattr(I, dtype_name)
    rng = np.random.default_rng(rows + cols)
    w = O.quantize(dtype, (rng.standard_normal(rows * cols) * 0.02).astype(np.float32))
    x = rng.standard_normal(cols).astype(np.float32)
    dw, dx, y = ctx.upload(w), ctx.upload(x), ctx.alloc(rows * 4)
    try:
        ctx.matmul_quant_assign(y, dw, dtype, rows, cols, dx)
        ref = y.download(np.float32, rows)
        ctx.set_option("gemv_grp", 225 | 256)
        try:
            ctx.matmul_quant_assign(y, dw, dtype, rows, cols, dx)
        finally:
            ctx.set_option("gemv_grp", 225)
        got = y.download(np.float32, rows)
        assert_same(got, ref, f"{dtype_name} {rows}x{cols}")
        e = O.gemv_quant(dtype, w, rows, cols, x)
        assert np.all(np.abs(got - e) <= 1e-3 * np.maximum(np.abs(e), 1.0))
    finally:
        for b in (dw, dx, y):
            b.free()
