"""GPU parity at the benchmark configurations' full shapes (BASELINE configs 4
and 5), prompt path included, against the oracle's forward (the restatement
of crates/inferi/src/models/llama2/cpu.rs:384-451 with the GPU path's eps and
theta) on the same weight bytes.

Two numerics are involved.  Decode steps keep activations at 22 bits and
accumulate in f32: their logits must be within 1e-3 of the oracle's and their
greedy ids identical.  The prompt path (ifr_llama2_prefill) multiplies on the
matrix cores with both operands rounded to binary16, as north_star asks for
the prefill GEMM; for its layer-0 K/V rows the test states the rounding bound
exactly (2^-11 relative per operand, summed over |w x|), and for the deeper
layers and the logits that follow it reports the distance and holds it to
2e-2 (the tolerance of the f16 path), with greedy ids compared wherever the
oracle's top-2 margin exceeds twice that step's error.
"""

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

C4 = dict(n_layers=22, hidden=2048, ffn=5632, n_heads=32, n_kv_heads=4, vocab=32000, rope_theta=10000.0,
          rms_eps=1e-5)
C5 = dict(n_layers=32, hidden=4096, ffn=14336, n_heads=32, n_kv_heads=8, vocab=128256, rope_theta=500000.0,
          rms_eps=1e-5)
U16 = 2.0 ** -11  # binary16 unit roundoff


def scaled(a, e):
    a, e = np.asarray(a, np.float64), np.asarray(e, np.float64)
    return np.abs(a - e) / np.maximum(np.abs(e), 1.0)


def oracle_model(cfg, w):
    from tests.test_gpu_model import oracle_model as om

    return om(cfg, w)


def kv_rows(state, cfg, layer, which, n):
    """The first n rows of a layer's f16 cache as f32."""
    raw = state.read(which, np.uint16, layer).reshape(cfg.max_pos, cfg.hidden // cfg.n_heads * cfg.n_kv_heads)
    return O.decode_f16(raw[:n]).astype(np.float64)


def layer0_kv_reference(cfg, w, tokens):
    """Layer-0 K (after RoPE) and V rows of `tokens` at positions 0.. from the
    exact arithmetic (f64 products of the f32 RMSNorm output and the
    bit-exact dequantized weights), and the bound on a device row formed from
    binary16 operands: per output i, b_i = (2u + u^2 + K 2^-24) sum_j |w_ij x_j|
    (u = 2^-11), rotated pairs bounded by the pair's norm."""
    import inferi_amd as I

    H, hs = cfg.hidden, cfg.hidden // cfg.n_heads
    dt, emb, _, cols = w.download("token_embd.weight")
    rb = I.row_bytes(dt, cols)
    x = np.stack([O.dequant(dt, emb[t * rb:(t + 1) * rb], H) for t in tokens])
    gamma = w.download("blk.0.attn_norm.weight")[1]
    xt = np.stack([O.rms_norm(r, gamma, cfg.rms_eps) for r in x]).astype(np.float64)
    out = {}
    for name, key in (("attn_k", "k"), ("attn_v", "v")):
        dtw, data, rows, c = w.download(f"blk.0.{name}.weight")
        W = O.dequant(dtw, data, rows * c).reshape(rows, c).astype(np.float64)
        pre = xt @ W.T
        A = (np.abs(xt).astype(np.float32) @ np.abs(W).T.astype(np.float32)).astype(np.float64) * 1.001
        b = (2 * U16 + U16 * U16 + c * 2.0 ** -24) * A
        if key == "k":
            rot = np.empty_like(pre)
            for p in range(len(tokens)):
                rot[p] = O.rope(pre[p].astype(np.float32), None, hs, p, cfg.rope_theta)[0]
            pair = np.sqrt(b[:, 0::2] ** 2 + b[:, 1::2] ** 2)
            b = np.repeat(pair, 2, axis=1) * 1.0001 + 1e-6 * np.abs(rot)  # + the f32 RoPE's own rounding
            pre = rot
        out[key] = (pre, b)
    return out


def check_layer0_bound(state, cfg, w, tokens):
    ref = layer0_kv_reference(cfg, w, tokens)
    worst = 0.0
    for key, which in (("k", "key_cache"), ("v", "value_cache")):
        e, b = ref[key]
        got = kv_rows(state, cfg, 0, which, len(tokens))
        # both sides are stored rounded to binary16
        lim = b + U16 * (np.abs(got) + np.abs(e)) + 1e-7
        excess = np.abs(got - e) - lim
        worst = max(worst, float(np.max(np.abs(got - e) / lim)))
        assert np.all(excess <= 0), f"layer 0 {which}: row {int(np.argmax(excess)) // e.shape[1]} beyond the f16 bound"
    return worst


@pytest.mark.timeout(900)
def test_c4_prefill_128_then_256_greedy_vs_oracle(ctx, oracle_lib):
    """Config 4 as the benchmark states it: a 128-token uniform random prompt
    (seed 7), then 256 greedy tokens.
    A: the prompt decoded token by token, then the greedy loop (the decode
       path alone): logits within 1e-3 of the oracle at every generated step,
       and every greedy id the oracle's argmax.
    B: the same 383 tokens with the first 127 through ifr_llama2_prefill
       (causal attention kernel pf_attn_f16_h64_g8: 32 query heads over 4 KV
       heads of size 64), then 256 decode steps: layer-0 K/V rows within the
       f16 rounding bound, every layer's rows and every step's logits within
       2e-2, ids where the margin allows."""
    import inferi_amd as I

    P, N = 128, 256
    cfg = I.Llama2Config(max_pos=P + N + 8, kv_dtype=I.F16, **C4)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=1000)
    sa, sb = I.Llama2State(ctx, cfg), I.Llama2State(ctx, cfg)
    try:
        prompt = np.random.default_rng(7).integers(0, cfg.vocab, P).tolist()
        # A
        sa.reset(prompt, 0)
        I.Llama2.generate(ctx, sa, w, P - 1, use_graph=True)
        la = []
        for _ in range(N):
            I.Llama2.generate(ctx, sa, w, 1, use_graph=True)
            la.append(sa.read("logits").copy())
        toks = sa.tokens(0, P + N)
        # B: teacher-forced on A's sequence
        sb.reset(toks[: P + N - 1], 0)
        I.Llama2.prefill(ctx, sb, w, P - 1)
        lb = []
        for _ in range(N):
            I.Llama2.generate(ctx, sb, w, 1, use_graph=True)
            lb.append(sb.read("logits").copy())
        # the oracle over the same sequence
        m = oracle_model(cfg, w)
        refs = []
        for pos in range(P + N - 1):
            r = m.forward(int(toks[pos]), pos)
            if pos >= P - 1:
                refs.append(r)
        worst_a, margins, checked_b, worst_b = 0.0, [], 0, 0.0
        for i, ref in enumerate(refs):
            ea = scaled(la[i], ref).max()
            worst_a = max(worst_a, float(ea))
            assert ea <= 1e-3, f"A step {i}: logits {ea:.3e} from the oracle"
            top2 = np.partition(ref, -2)[-2:]
            margins.append(float(top2[1] - top2[0]))
            assert int(toks[P + i]) == O.argmax(ref), f"A token {P + i} (margin {margins[-1]:.2e})"
            eb = scaled(lb[i], ref).max()
            worst_b = max(worst_b, float(eb))
            assert eb <= 2e-2, f"B step {i}: logits {eb:.3e} from the oracle"
            if top2[1] - top2[0] > 2 * np.abs(lb[i].astype(np.float64) - ref).max():
                assert O.argmax(lb[i]) == O.argmax(ref), f"B step {i}: greedy id"
                checked_b += 1
        bound_use = check_layer0_bound(sb, cfg, w, [int(t) for t in toks[: P - 1]])
        kv_err = []
        for layer in range(cfg.n_layers):
            for which, key in (("key_cache", "k"), ("value_cache", "v")):
                e = O.decode_f16(m.kv_cache(layer, key)[: P + N - 1]).astype(np.float64)
                ga, gb = kv_rows(sa, cfg, layer, which, P + N - 1), kv_rows(sb, cfg, layer, which, P + N - 1)
                # A: within 1e-3 of max(|e|, 1) plus the binary16 step of
                # the stored value (both sides round to f16)
                ea = float(np.max(np.abs(ga - e) / (1e-3 * np.maximum(np.abs(e), 1.0) + 2 * U16 * np.abs(e))))
                eb = float(np.abs(gb - e).max() / np.abs(e).max())
                assert ea <= 1.0, f"A layer {layer} {which}: {ea:.3f} of the bar"
                assert eb <= 2e-2, f"B layer {layer} {which}: normwise {eb:.3e}"
                kv_err.append(eb)
        print(f"c4 A (decode path): {N} greedy ids identical, logits within {worst_a:.2e}, smallest margin "
              f"{min(margins):.3e}; B (prefill 127 + {N} steps): logits within {worst_b:.2e}, {checked_b}/{N} ids "
              f"compared and equal, layer-0 K/V at {bound_use:.2f} of the f16 bound, KV rows normwise <= "
              f"{max(kv_err):.2e}", flush=True)
        assert checked_b >= N // 2
    finally:
        sa.close()
        sb.close()
        w.close()


@pytest.mark.timeout(900)
def test_c5_prefill_4095_tokens(ctx, oracle_lib):
    """Config 5 shape: the benchmark's 4095-token prefill in one pass (the
    default pass length) at the 8B shape.  Layer-0 K/V rows at every position
    against the exact arithmetic within the f16 rounding bound; every layer's
    rows (2e-2 normwise) and the next step's logits (5e-2 scaled: 32 layers of
    f16-operand products) against sequential decode of the same prompt on the
    device; and passes of 512 tokens (128 x 128 GEMM tiles, where the
    4095-token pass takes 256 x 256 tiles) give the same rows and logits bit
    for bit."""
    import inferi_amd as I

    P = 4096
    cfg = I.Llama2Config(max_pos=P + 8, kv_dtype=I.F16, **C5)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=2000)
    prompt = np.random.default_rng(8).integers(0, cfg.vocab, P).tolist()
    sa = I.Llama2State(ctx, cfg)
    try:
        sa.reset(prompt, 0)
        I.Llama2.prefill(ctx, sa, w, P - 1)
        I.Llama2.generate(ctx, sa, w, 1, use_graph=True)
        la = sa.read("logits").copy()
        bound_use = check_layer0_bound(sa, cfg, w, prompt[: P - 1])
        # passes of 512 tokens
        ctx.set_option("pf_chunk", 512)
        sc = I.Llama2State(ctx, cfg)
        try:
            sc.reset(prompt, 0)
            I.Llama2.prefill(ctx, sc, w, P - 1)
            I.Llama2.generate(ctx, sc, w, 1, use_graph=True)
            e512 = float(scaled(sc.read("logits"), la).max())
            kv512 = 0.0
            for layer in range(cfg.n_layers):
                for which in ("key_cache", "value_cache"):
                    ga, gc = kv_rows(sa, cfg, layer, which, P), kv_rows(sc, cfg, layer, which, P)
                    kv512 = max(kv512, float(np.abs(gc - ga).max() / np.abs(ga).max()))
            assert kv512 == 0.0, f"KV rows, passes of 512: normwise {kv512:.3e}"
            assert e512 == 0.0, f"logits, passes of 512: {e512:.3e}"
        finally:
            ctx.set_option("pf_chunk", 0)
            sc.close()
        # sequential decode of the same prompt
        sb = I.Llama2State(ctx, cfg)
        try:
            sb.reset(prompt, 0)
            I.Llama2.generate(ctx, sb, w, P, use_graph=True)
            lb = sb.read("logits").copy()
            el = float(scaled(la, lb).max())
            worst = 0.0
            for layer in range(cfg.n_layers):
                for which in ("key_cache", "value_cache"):
                    ga, gb = kv_rows(sa, cfg, layer, which, P), kv_rows(sb, cfg, layer, which, P)
                    e = float(np.abs(ga - gb).max() / np.abs(gb).max())
                    worst = max(worst, e)
                    assert e <= 2e-2, f"{which} layer {layer}: normwise {e:.3e} from sequential decode"
            top2 = np.partition(lb, -2)[-2:]
            same_id = O.argmax(la) == O.argmax(lb)
            print(f"c5 prefill of {P - 1} tokens: layer-0 K/V at {bound_use:.2f} of the f16 bound; all layers' rows "
                  f"within {worst:.2e} (normwise) of sequential decode; next logits within {el:.2e} (scaled); greedy "
                  f"id {'equal' if same_id else 'differs'} (margin {top2[1] - top2[0]:.3e}); passes of 512: rows within "
                  f"{kv512:.2e}, logits within {e512:.2e}",
                  flush=True)
            # 32 layers of f16-operand products: the KV rows stay within 2e-2
            # normwise; the logits that read all of them within 5e-2
            assert el <= 5e-2, f"next-step logits {el:.3e} from sequential decode"
            if top2[1] - top2[0] > 2 * np.abs(la.astype(np.float64) - lb).max():
                assert same_id, "greedy id after the prefill"

        finally:
            sb.close()
    finally:
        sa.close()
        w.close()
