"""ifr_matmul_quant_noalloc (the entry point that allocates nothing) against
ifr_matmul_quant, through the C ABI: the same kernels, so the outputs are
identical; two calls in a row, the second smaller, share the fixed scratch."""

import numpy as np
import pytest


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["int", "exact"])
def test_noalloc_matches_matmul_quant(ctx, path):
    import inferi_amd as I
    import oracle as O

    ctx.set_option("gemv_exact", int(path == "exact"))
    try:
        rng = np.random.default_rng(7)
        for rows, cols, dtype in ((4096, 14336, I.Q4_K), (300, 1024, I.Q6_K)):  # second call smaller
            w = O.quantize(dtype, (rng.standard_normal(rows * cols) * 0.02).astype(np.float32))
            x = rng.standard_normal(cols).astype(np.float32)
            dw, dx = ctx.upload(w), ctx.upload(x)
            y1, y2 = ctx.alloc(rows * 4), ctx.alloc(rows * 4)
            ctx.matmul_quant_assign(y1, dw, dtype, rows, cols, dx)
            ctx.matmul_quant_noalloc(y2, dw, dtype, rows, cols, dx)
            a, b = y1.download(np.float32, rows), y2.download(np.float32, rows)
            print(f"{path} {rows}x{cols} dtype {dtype}: max |diff| {np.abs(a - b).max():.3e}", flush=True)
            assert np.array_equal(a, b), "noalloc output differs from ifr_matmul_quant"
            e = O.gemv_quant(dtype, w, rows, cols, x)
            assert np.all(np.abs(b - e) <= 1e-3 * np.maximum(np.abs(e), 1.0))
            for buf in (dw, dx, y1, y2):
                buf.free()
    finally:
        ctx.set_option("gemv_exact", 0)


@pytest.mark.gpu
def test_noalloc_rejects_inputs_beyond_the_scratch(ctx):
    import inferi_amd as I

    cols = 18944  # 3 * cols + cols / 2 = 66304 bytes > 65536
    dw, dx, dy = ctx.alloc(16 * I.row_bytes(I.Q4_K, cols)), ctx.alloc(cols * 4), ctx.alloc(64)
    try:
        with pytest.raises(I.HipError) as e:
            ctx.matmul_quant_noalloc(dy, dw, I.Q4_K, 16, cols, dx)
        assert e.value.status == 1
    finally:
        for buf in (dw, dx, dy):
            buf.free()
