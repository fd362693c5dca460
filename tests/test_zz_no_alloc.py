"""ifr_matmul_quant_noalloc (the entry point that allocates nothing) against
ifr_matmul_quant, through the C ABI: the same kernels, so the outputs are
identical; two calls in a row, the second smaller, share the fixed scratch;
the device's free memory (hipMemGetInfo) is the same before and after the
calls."""

import ctypes

import numpy as np
import pytest


def _free_bytes(ctx):
    """Free device memory as the HIP runtime reports it, after draining the
    context's stream."""
    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime the library is linked against
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    ctx.sync()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


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
            ctx.matmul_quant_noalloc(y2, dw, dtype, rows, cols, dx)  # warm-up: modules loaded
            before = _free_bytes(ctx)
            for _ in range(3):
                ctx.matmul_quant_noalloc(y2, dw, dtype, rows, cols, dx)
            after = _free_bytes(ctx)
            assert after == before, f"device free memory changed by {before - after} bytes across the calls"
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
