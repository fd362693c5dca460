"""GPU parity of the persistent layer tail (device/pk.h): the decode step
with O, gate/up, down and the next QKV in one launch per layer equals the
fused kernels' step bit for bit (logits, KV-cache rows, tokens), with the
graph and without, across steps (the barrier epoch carries over), and
against the oracle; no barrier gives up (the error word stays 0)."""

import numpy as np
import pytest

import oracle as O
from tests.test_gpu_model import check_steps_vs_oracle, run_steps, tiny_cfg

pytestmark = pytest.mark.gpu


def pk_err(state):
    return int(state.read("pk_err", np.uint32)[0])


def decode(ctx, cfg, w, prompt, n, persistent, mode="graph"):
    import inferi_amd as I

    ctx.set_option("persistent", int(persistent))
    s = I.Llama2State(ctx, cfg)
    try:
        logits, toks = run_steps(ctx, s, w, prompt, n, mode)
        kv = {}
        for layer in range(cfg.n_layers):
            for name in ("key_cache", "value_cache"):
                dt = np.uint16 if cfg.kv_dtype == I.F16 else np.float32
                kv[name, layer] = s.read(name, dt, layer).reshape(cfg.max_pos, cfg.kv_dim)[:n]
        x = s.read("x")
        err = pk_err(s)
    finally:
        s.close()
        ctx.set_option("persistent", 0)
    return np.array(logits), toks, kv, x, err


def assert_same(a, b, what):
    a, b = np.asarray(a), np.asarray(b)
    if not np.array_equal(a.view(np.uint8), b.view(np.uint8)):
        d = np.abs(a.astype(np.float64) - b.astype(np.float64))
        raise AssertionError(f"{what}: not bit-identical (max |diff| {d.max():.3e} at {np.unravel_index(d.argmax(), d.shape)})")


def check_same_as_fused(ctx, cfg, w, prompt, n, mode="graph"):
    ref = decode(ctx, cfg, w, prompt, n, persistent=False, mode=mode)
    got = decode(ctx, cfg, w, prompt, n, persistent=True, mode=mode)
    assert got[4] == 0, "a grid barrier gave up"
    assert_same(got[0], ref[0], "logits")
    assert np.array_equal(got[1], ref[1]), "tokens"
    for k in ref[2]:
        assert_same(got[2][k], ref[2][k], f"{k[0]} layer {k[1]}")
    assert_same(got[3], ref[3], "residual x")


@pytest.mark.parametrize("mode", ["graph", "fused"])
def test_tiny_same_as_fused(ctx, mode):
    import inferi_amd as I

    cfg = tiny_cfg(n_layers=3, max_pos=64)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=5, std=0.05)
    try:
        check_same_as_fused(ctx, cfg, w, [1, 2, 3], 30, mode)
    finally:
        w.close()


def test_tiny_against_oracle(ctx, oracle_lib):
    import inferi_amd as I

    cfg = tiny_cfg()
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=11, std=0.05)
    ctx.set_option("persistent", 1)
    try:
        check_steps_vs_oracle(ctx, cfg, w, "graph")
    finally:
        ctx.set_option("persistent", 0)
        w.close()


def test_continuation_and_f32_cache(ctx):
    """N steps then M more equal N+M steps (the barrier epoch advances across
    launches and graph replays); an f32 KV cache takes the same path."""
    import inferi_amd as I

    cfg = tiny_cfg(n_layers=2, max_pos=64, kv_dtype=I.F32)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=9, std=0.05)
    s = I.Llama2State(ctx, cfg)
    try:
        ref = decode(ctx, cfg, w, [4, 5], 40, persistent=False)
        ctx.set_option("persistent", 1)
        s.reset([4, 5], 0)
        I.Llama2.generate(ctx, s, w, 13, use_graph=True)
        for _ in range(4):
            I.Llama2.launch(ctx, s, w)
        I.Llama2.generate(ctx, s, w, 23, use_graph=True)
        assert np.array_equal(s.tokens(0, 41), ref[1])
        assert pk_err(s) == 0
    finally:
        ctx.set_option("persistent", 0)
        s.close()
        w.close()


@pytest.mark.timeout(600)
def test_c4_shape_same_as_fused(ctx):
    """BASELINE config 4 shape (22 layers, hidden 2048, FFN 5632, 32/4 heads)."""
    import inferi_amd as I

    cfg = I.Llama2Config(n_layers=22, hidden=2048, ffn=5632, n_heads=32, n_kv_heads=4, vocab=32000, max_pos=64,
                         rope_theta=10000.0, rms_eps=1e-5, kv_dtype=I.F16)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=1000)
    try:
        prompt = np.random.default_rng(7).integers(0, cfg.vocab, 8).tolist()
        check_same_as_fused(ctx, cfg, w, prompt, 24)
    finally:
        w.close()


@pytest.mark.timeout(900)
def test_c5_shape_same_as_fused(ctx):
    """BASELINE config 5 shape (32 layers, hidden 4096, FFN 14336, 32/8 heads,
    vocab 128256) at full size."""
    import inferi_amd as I

    cfg = I.Llama2Config(n_layers=32, hidden=4096, ffn=14336, n_heads=32, n_kv_heads=8, vocab=128256, max_pos=16,
                         rope_theta=500000.0, rms_eps=1e-5, kv_dtype=I.F16)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=2000)
    try:
        check_same_as_fused(ctx, cfg, w, [17, 128255, 0, 4242], 8)
    finally:
        w.close()


@pytest.mark.parametrize("grp", [0, 2, 4, 12, 16, 31, 33, 63, 64, 97])
def test_gemv_forms_same_results(ctx, grp):
    """Every GEMV form the gemv_grp option selects (the looping body, the
    one-item forms of O, down, gate/up and the head, the head's 256-VGPR
    form) gives the default path's logits, tokens and KV rows bit for bit
    (same arithmetic, same reduction orders), on the C4 shape."""
    import inferi_amd as I

    cfg = I.Llama2Config(n_layers=4, hidden=2048, ffn=5632, n_heads=32, n_kv_heads=4, vocab=32000, max_pos=32,
                         rope_theta=10000.0, rms_eps=1e-5, kv_dtype=I.F16)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=1000)
    try:
        prompt = [5, 31999, 7, 1234]
        ref = decode(ctx, cfg, w, prompt, 12, persistent=False)
        ctx.set_option("gemv_grp", grp)
        try:
            got = decode(ctx, cfg, w, prompt, 12, persistent=False)
        finally:
            ctx.set_option("gemv_grp", 97)
        assert_same(got[0], ref[0], "logits")
        assert np.array_equal(got[1], ref[1]), "tokens"
        for k in ref[2]:
            assert_same(got[2][k], ref[2][k], f"{k[0]} layer {k[1]}")
        assert_same(got[3], ref[3], "residual x")
    finally:
        w.close()
