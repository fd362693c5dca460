"""GPU checks of the strided-view forms of RMSNorm, RoPE, SiLU and the
residual add (ifr_*_view), through the C ABI.  The reference's op shaders
index every operand through its tensor layout (rms_norm.rs:118-119,
rope.rs:81-87 and 129-132, silu.rs:46-47); here a view is (offset, stride)
in elements.  Each case gathers the views' elements on the host, runs the
oracle's contiguous op on them and scatters the result back, so the
expected buffer also checks that no element outside the output view moved.
RoPE follows the reference's pair rule: the pair's second element lies 1
(Original) or head_size / 2 (NeoX) elements after its first in memory."""

import numpy as np
import pytest

import oracle as O
from tests.test_gpu_model import assert_close

pytestmark = pytest.mark.gpu

VIEWS = [(0, 1), (5, 1), (3, 2), (7, 3), (2, 5)]


def _idx(view, n):
    off, st = view
    return off + st * np.arange(n, dtype=np.int64)


@pytest.mark.parametrize("ov", VIEWS)
def test_rms_norm_view(ctx, oracle_lib, ov):
    import inferi_amd as I

    rng = np.random.default_rng(ov[0] * 10 + ov[1])
    n, eps = 1000, 1e-5
    vv, wv = (ov[1] + 1, 2), (3, ov[1])
    size = 8 * n + 64
    v = (rng.standard_normal(size) * 3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(size)).astype(np.float32)
    out = np.full(size, -7.0, np.float32)
    cfg = ctx.upload(np.frombuffer(bytes(I.RmsNormConfig(eps)), np.uint8))
    dv, dw, do = ctx.upload(v), ctx.upload(w), ctx.upload(out)
    ctx.rms_norm_view(cfg, do, ov, dv, vv, dw, wv, n)
    exp = out.copy()
    exp[_idx(ov, n)] = O.rms_norm(v[_idx(vv, n)], w[_idx(wv, n)], eps)
    got = do.download(np.float32, size)
    assert_close(got, exp, tol=1e-5, what=f"rms_norm view {ov}")
    assert np.array_equal(np.delete(got, _idx(ov, n)), np.delete(exp, _idx(ov, n))), "elements outside the view"


@pytest.mark.parametrize("av", VIEWS)
def test_add_and_silu_views(ctx, oracle_lib, av):
    rng = np.random.default_rng(av[0] * 7 + av[1])
    n = 777
    bv = (1, av[1] + 1)
    size = 8 * n + 64
    a = rng.standard_normal(size).astype(np.float32) * 4
    b = rng.standard_normal(size).astype(np.float32)
    da, db = ctx.upload(a), ctx.upload(b)
    ctx.add_view(da, av, db, bv, n)
    exp = a.copy()
    exp[_idx(av, n)] = a[_idx(av, n)] + b[_idx(bv, n)]
    assert np.array_equal(da.download(np.float32, size), exp), f"add view {av}"
    ctx.silu_view(da, av, db, bv, n)
    exp2 = exp.copy()
    exp2[_idx(av, n)] = O.silu_mul(exp[_idx(av, n)], b[_idx(bv, n)])
    assert_close(da.download(np.float32, size), exp2, tol=1e-6, what=f"silu view {av}")


@pytest.mark.parametrize("neox", [False, True])
@pytest.mark.parametrize("qv,kv", [((0, 1), (0, 1)), ((4, 1), (9, 1)), ((3, 3), (1, 3)), ((2, 5), (6, 7))])
def test_rope_view(ctx, oracle_lib, neox, qv, kv):
    import inferi_amd as I

    hs, nq, nk, pos, theta = 128, 4 * 128, 2 * 128, 4095, 500000.0
    rng = np.random.default_rng(qv[1] * 100 + kv[1] + neox)
    size = 8 * nq + 256
    q = rng.standard_normal(size).astype(np.float32)
    k = rng.standard_normal(size).astype(np.float32)
    cfg = ctx.upload(np.frombuffer(bytes(I.RoPEConfig(hs, nk, pos, theta)), np.uint8))
    dq, dk = ctx.upload(q), ctx.upload(k)
    ctx.rope_view(I.ROPE_NEOX if neox else I.ROPE_ORIGINAL, cfg, dq, qv, nq, dk, kv, nk)

    def pairs(view, n):
        # memory slots of the logical vector's elements under the pair rule
        off, st = view
        slots = np.empty(n, np.int64)
        for i in range(n // 2):
            if neox:
                e0 = i + (2 * i) // hs * hs // 2
                shift = hs // 2
            else:
                e0, shift = 2 * i, 1
            slots[e0] = off + e0 * st
            slots[e0 + shift] = slots[e0] + shift
        assert len(set(slots.tolist())) == n, "the view's pairs overlap"
        return slots

    sq, sk = pairs(qv, nq), pairs(kv, nk)
    eq, ek = O.rope(q[sq], k[sk], hs, pos, theta, neox)
    expq, expk = q.copy(), k.copy()
    expq[sq], expk[sk] = eq, ek
    assert_close(dq.download(np.float32, size), expq, tol=1e-5, what=f"rope q view {qv}")
    assert_close(dk.download(np.float32, size), expk, tol=1e-5, what=f"rope k view {kv}")
