"""GPU parity of the matrix-core attention split kernel (device/attention.h
attn2_body: q.k with v_mfma_f32_32x32x16_f16 on a hi/lo f16 split of the
query, softmax and P.V in f32), selected by the attn_mfma option for f16
caches of head size 128 with 1, 2 or 4 query heads per KV head.

The decode's logits at every step are checked against the oracle's forward
(reference transformer.rs attention: f32 scores, softmax, weighted V sum)
within the decode bar 1e-3 * max(|e|, 1), over enough positions that several
splits, a ragged last block and (max_pos 40000) splits of two 128-position
blocks are in use; greedy ids must equal the oracle's argmax wherever its
top-2 gap exceeds the tolerance."""

import numpy as np
import pytest

import oracle as O
from tests.test_gpu_model import assert_close, oracle_model
from tests.test_gpu_ops import _attn_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nh,nkv", [(4, 4), (8, 4), (16, 4), (32, 8)])
def test_attention_op_against_oracle(ctx, oracle_lib, nh, nkv):
    """The attention operator (ifr_attention) on the matrix-core kernel:
    f16 cache of N(0, 1) rows, positions inside one block, across blocks
    and splits, and at a ragged end."""
    rng = np.random.default_rng(nh * 7 + nkv)
    ctx.set_option("attn_mfma", 1)
    try:
        for pos in (0, 1, 31, 32, 127, 128, 300, 1023, 4095):
            got, ref = _attn_case(ctx, nh, nkv, 128, 4096, pos, True, rng)
            assert_close(got, ref, what=f"pos={pos}")
    finally:
        ctx.set_option("attn_mfma", 0)


def cfg_hs128(kv_mul, max_pos):
    import inferi_amd as I

    return I.Llama2Config(n_layers=2, hidden=512, ffn=512, n_heads=4, n_kv_heads=4 // kv_mul, vocab=1000,
                          max_pos=max_pos, rope_theta=10000.0, rms_eps=1e-5, kv_dtype=I.F16)


def decode_vs_oracle(ctx, cfg, w, prompt, n):
    import inferi_amd as I

    s = I.Llama2State(ctx, cfg)
    try:
        s.reset(prompt, 0)
        logits = []
        for _ in range(n):
            I.Llama2.generate(ctx, s, w, 1, use_graph=True)
            logits.append(s.read("logits"))
        toks = s.tokens(0, n + 1)
    finally:
        s.close()
    m = oracle_model(cfg, w)
    for pos in range(n):
        ref = m.forward(int(toks[pos]), pos)
        assert_close(logits[pos], ref, what=f"pos {pos}")
        if pos + 1 >= len(prompt):
            top = np.sort(ref)[-2:]
            if top[1] - top[0] > 1e-2:
                assert int(toks[pos + 1]) == O.argmax(ref), f"token at {pos + 1}"
        else:
            assert int(toks[pos + 1]) == prompt[pos + 1]
    return toks


@pytest.mark.parametrize("kv_mul", [1, 2, 4])
@pytest.mark.parametrize("max_pos", [400, 40000])
@pytest.mark.parametrize("mfma", [1, 0])
def test_decode_against_oracle(ctx, oracle_lib, kv_mul, max_pos, mfma):
    """mfma 0: the default split kernel on the same shapes, for comparison."""
    import inferi_amd as I

    cfg = cfg_hs128(kv_mul, max_pos)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=21 + kv_mul, std=0.05)
    ctx.set_option("attn_mfma", mfma)
    try:
        decode_vs_oracle(ctx, cfg, w, [3, 999, 41, 0, 512], 300)
    finally:
        ctx.set_option("attn_mfma", 0)
        w.close()


def test_after_prefill_matches_default_kernel(ctx):
    """After a 700-token prefill the matrix-core split and the default split
    kernel give logits within the decode bar of each other, step by step."""
    import inferi_amd as I

    cfg = cfg_hs128(4, 1000)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=5, std=0.05)
    prompt = np.random.default_rng(3).integers(0, cfg.vocab, 700).astype(np.uint32)
    out = {}
    try:
        for mf in (0, 1):
            ctx.set_option("attn_mfma", mf)
            s = I.Llama2State(ctx, cfg)
            try:
                s.reset(prompt, 0)
                I.Llama2.prefill(ctx, s, w, 699)
                lg = []
                for _ in range(40):
                    I.Llama2.generate(ctx, s, w, 1, use_graph=True)
                    lg.append(s.read("logits"))
                out[mf] = lg
            finally:
                s.close()
    finally:
        ctx.set_option("attn_mfma", 0)
        w.close()
    for i, (a, b) in enumerate(zip(out[1], out[0])):
        assert_close(a, b, what=f"step {i}")
