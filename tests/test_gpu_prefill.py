"""GPU parity of the prompt (prefill) path.

ifr_gemm_quant multiplies f16 activations by weights of any quantized GGUF
type dequantized to f16 tiles on the matrix cores, in 256 x 256 or 128 x 128
tiles (option pf_tile): both forms are checked against an f64 product of the
same f16-rounded operands (only the f32 accumulation order may differ) and
against each other (bit for bit).

ifr_llama2_prefill runs a prompt through every layer in chunks; the state it
leaves (KV-cache rows, position) must continue exactly like a state that
decoded the prompt token by token.  Its products take f16 inputs where the
decode path keeps 22-bit activations, so KV rows and logits are compared
within 2e-2 of max(|e|, 1) (the tolerance is a property of the f16 path),
and the continuation's greedy ids are compared where the sequential path's
top-2 logit margin exceeds that tolerance.
"""

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def synthetic_q(ctx, rows, cols, seed, dtype):
    import inferi_amd as I

    n = rows * cols
    tmp = ctx.alloc(n * 4)
    ctx.fill_normal(tmp, n, seed, 0, 0.0, 0.02)
    w = ctx.alloc(rows * I.row_bytes(dtype, cols))
    ctx.quantize(w, tmp, dtype, n)
    tmp.free()
    return w


# (pf_tile, pf_ws): the 128 x 128 form, the 256 x 256 eight-wave form and
# the 256 x 256 warp-specialized form (Q4_K only; other types ignore pf_ws)
TILE_FORMS = ((128, 0), (256, 0), (256, 1))


def _gemm_case(ctx, dtype, rows, cols, m, w, rng, forms=TILE_FORMS):
    """y = x . deq(W)^T in each tile form against the f64 product of the same
    f16-rounded operands (bound 2e-5 * sum |x w|), then the accumulating form;
    the tile forms agree bit for bit."""
    import inferi_amd as I

    outs = []
    ws0 = ctx.get_option("pf_ws")
    for tile, ws in forms:
        ctx.set_option("pf_tile", tile)
        ctx.set_option("pf_ws", ws)
        try:
            outs.append(_gemm_case1(ctx, dtype, rows, cols, m, w, np.random.default_rng(rows + cols + m)))
        finally:
            ctx.set_option("pf_tile", 0)
            ctx.set_option("pf_ws", ws0)
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), "tile forms differ"


def _gemm_case1(ctx, dtype, rows, cols, m, w, rng):
    import inferi_amd as I

    rb = I.row_bytes(dtype, cols)
    deq = O.dequant(dtype, w.download(np.uint8, rows * rb), rows * cols).reshape(rows, cols)
    wh = deq.astype(np.float16).astype(np.float64)
    x = rng.standard_normal((m, cols)).astype(np.float16)
    dx = ctx.upload(x)
    y = ctx.alloc(m * rows * 4)
    ctx.gemm_quant(y, w, dtype, rows, cols, dx, m)
    got = y.download(np.float32, m * rows).reshape(m, rows).astype(np.float64)
    xd = x.astype(np.float64)
    ref = xd @ wh.T
    bound = 2e-5 * (np.abs(xd) @ np.abs(wh).T) + 1e-30
    assert np.all(np.abs(got - ref) <= bound), f"max excess {np.max(np.abs(got - ref) - bound):.3e}"
    ctx.gemm_quant(y, w, dtype, rows, cols, dx, m, accumulate=True)
    got2 = y.download(np.float32, m * rows).reshape(m, rows).astype(np.float64)
    assert np.all(np.abs(got2 - 2 * ref) <= 2 * bound)
    for b in (dx, y):
        b.free()
    return got.astype(np.float32)


@pytest.mark.parametrize("rows,cols,m", [(128, 256, 128), (300, 512, 70), (1000, 1024, 257), (4096, 4096, 128),
                                         (64, 14336, 33), (4096, 4096, 512), (512, 14336, 300), (1024, 4096, 4095),
                                         (6144, 4096, 4095)])
def test_gemm_quant_matches_f64(ctx, oracle_lib, rows, cols, m):
    """Q4_K at shapes whose 256 x 256 tile counts cover the warp-specialized
    form's cases: fewer than 128 tiles (every tile in two halves), and 384
    tiles (the 8B Q/K/V shape: 256 whole tiles, then 128 in halves)."""
    import inferi_amd as I

    rng = np.random.default_rng(rows * 7 + cols + m)
    w = synthetic_q(ctx, rows, cols, rows + m, I.Q4_K)
    _gemm_case(ctx, I.Q4_K, rows, cols, m, w, rng)
    w.free()


FMTS = ["Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q8_0", "Q4_K", "Q5_K", "Q6_K", "Q8_K", "F16", "F32"]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("rows,cols,m", [(300, 512, 70), (130, 2048, 129), (300, 512, 300), (130, 2048, 260)])
def test_gemm_quant_every_format(ctx, oracle_lib, fmt, rows, cols, m):
    """Each GGUF type's tile loader in both tile forms: quantized synthetic
    weights and raw random blocks with a quarter of the scales subnormal (the
    reference's GEMV test generator, gemv_quant.rs:354-430)."""
    import inferi_amd as I
    from tests import kquant as K

    dtype = getattr(I, fmt)
    rng = np.random.default_rng(rows + cols + dtype)
    w = synthetic_q(ctx, rows, cols, rows * 3 + dtype, dtype)
    _gemm_case(ctx, dtype, rows, cols, m, w, rng)
    w.free()
    raw = K.random_blocks(dtype, rows * cols // O.BLOCK_ELEMS[dtype], rng)
    w = ctx.upload(raw)
    _gemm_case(ctx, dtype, rows, cols, m, w, rng)
    w.free()


def test_gemm_quant_rejects_bad_input(ctx):
    import inferi_amd as I

    buf = ctx.alloc(1 << 16)
    with pytest.raises(I.HipError):
        ctx.gemm_quant(buf, buf, 5, 16, 256, buf, 4)  # no GGUF type 5
    with pytest.raises(I.HipError):
        ctx.gemm_quant(buf, buf, I.Q4_K, 16, 100, buf, 4)  # cols % 256
    with pytest.raises(I.HipError):
        ctx.gemm_quant(buf, buf, I.Q8_0, 16, 96, buf, 4)  # cols % 64
    with pytest.raises(I.HipError):
        ctx.gemm_quant(buf, buf.at(4), I.Q4_K, 16, 256, buf, 4)  # K-quant rows 16-byte aligned
    buf.free()


def _prefill_vs_decode(ctx, cfg, w, prompt, n_gen, tol=2e-2):
    import inferi_amd as I

    P = len(prompt)
    sa, sb = I.Llama2State(ctx, cfg), I.Llama2State(ctx, cfg)
    try:
        # A: the prompt token by token, then n_gen greedy steps, logits kept
        sa.reset(prompt, 0)
        I.Llama2.generate(ctx, sa, w, P - 1, use_graph=True)
        logits_a = []
        for _ in range(n_gen):
            I.Llama2.generate(ctx, sa, w, 1, use_graph=True)
            logits_a.append(sa.read("logits"))
        # B: prefill of the first P-1 tokens, then the same decode steps
        sb.reset(prompt, 0)
        I.Llama2.prefill(ctx, sb, w, P - 1)
        assert int(sb.read("pos", np.uint32)[0]) == P - 1
        logits_b = []
        for _ in range(n_gen):
            I.Llama2.generate(ctx, sb, w, 1, use_graph=True)
            logits_b.append(sb.read("logits"))
        f16 = cfg.kv_dtype == I.F16
        for layer in range(cfg.n_layers):
            for which in ("key_cache", "value_cache"):
                ga = sa.read(which, np.uint16 if f16 else np.float32, layer).reshape(cfg.max_pos, cfg.kv_dim)[: P - 1]
                gb = sb.read(which, np.uint16 if f16 else np.float32, layer).reshape(cfg.max_pos, cfg.kv_dim)[: P - 1]
                if f16:
                    ga, gb = O.decode_f16(ga), O.decode_f16(gb)
                err = np.abs(gb.astype(np.float64) - ga) / np.maximum(np.abs(ga), 1.0)
                assert err.max() <= tol, f"{which} layer {layer}: {err.max():.3e} at row {int(err.argmax()) // cfg.kv_dim}"
        toks_a, toks_b = sa.tokens(0, P + n_gen), sb.tokens(0, P + n_gen)
        compared = 0
        for i in range(n_gen):
            la, lb = logits_a[i].astype(np.float64), logits_b[i].astype(np.float64)
            if not np.array_equal(toks_a[: P + i], toks_b[: P + i]):
                break  # the sequences diverged earlier: later steps see different inputs
            err = np.abs(lb - la) / np.maximum(np.abs(la), 1.0)
            assert err.max() <= tol, f"logits of step {i}: {err.max():.3e}"
            top2 = np.partition(la, -2)[-2:]
            if top2[1] - top2[0] > 2 * tol * max(abs(top2[1]), 1.0):
                assert toks_b[P + i] == toks_a[P + i], f"token {P + i}"
                compared += 1
        return compared
    finally:
        sa.close()
        sb.close()


def test_prefill_matches_sequential_decode_hs64(ctx, oracle_lib):
    import inferi_amd as I

    cfg = I.Llama2Config(n_layers=3, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, vocab=1000, max_pos=200,
                         rope_theta=10000.0, rms_eps=1e-5, kv_dtype=I.F16)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=31, std=0.05)
    try:
        prompt = np.random.default_rng(3).integers(0, cfg.vocab, 150).tolist()
        assert _prefill_vs_decode(ctx, cfg, w, prompt, 12) > 0
    finally:
        w.close()


@pytest.mark.parametrize("hs", [32, 64, 96])
def test_prefill_f32_cache_small_heads(ctx, oracle_lib, hs):
    """An f32 cache with head sizes staged on the 64-wide attention tile (two
    keys per staging thread; 32: half its dims past the head) and on the
    128-wide one with dims past the head (96), across 300 prompt tokens."""
    import inferi_amd as I

    cfg = I.Llama2Config(n_layers=2, hidden=8 * hs, ffn=512, n_heads=8, n_kv_heads=2, vocab=512, max_pos=330,
                         rope_theta=10000.0, rms_eps=1e-5, kv_dtype=I.F32)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=hs, std=0.05)
    try:
        prompt = np.random.default_rng(hs).integers(0, cfg.vocab, 301).tolist()
        assert _prefill_vs_decode(ctx, cfg, w, prompt, 6) > 0
    finally:
        w.close()


@pytest.mark.parametrize("chunk", [512, 0])
def test_prefill_chunks_and_gqa4_hs128(ctx, oracle_lib, chunk):
    """Two prefill passes (512 + rest) or one (the default pass length),
    head size 128, 4 query heads per KV head, f32 cache."""
    import inferi_amd as I

    cfg = I.Llama2Config(n_layers=2, hidden=512, ffn=1024, n_heads=4, n_kv_heads=1, vocab=512, max_pos=700,
                         rope_theta=500000.0, rms_eps=1e-5, kv_dtype=I.F32)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=41, std=0.05)
    ctx.set_option("pf_chunk", chunk)
    try:
        prompt = np.random.default_rng(4).integers(0, cfg.vocab, 600).tolist()
        assert _prefill_vs_decode(ctx, cfg, w, prompt, 8) > 0
    finally:
        ctx.set_option("pf_chunk", 0)
        w.close()


def _prefill_run(ctx, cfg, w, prompt, n_prefill, n_gen):
    """Prefill then n_gen graph steps on a fresh state: (logits bits, tokens, KV rows)."""
    import inferi_amd as I

    s = I.Llama2State(ctx, cfg)
    try:
        s.reset(prompt, 0)
        I.Llama2.prefill(ctx, s, w, n_prefill)
        I.Llama2.generate(ctx, s, w, n_gen, use_graph=True)
        kv = [s.read(n, np.uint16, layer).copy() for layer in range(cfg.n_layers) for n in ("key_cache", "value_cache")]
        return s.read("logits").view(np.uint32).copy(), s.tokens(0, n_prefill + n_gen + 1), kv
    finally:
        s.close()


def _same(a, b, what):
    assert np.array_equal(a[0], b[0]), f"logits: {what}"
    assert np.array_equal(a[1], b[1]), f"tokens: {what}"
    for x, y in zip(a[2], b[2]):
        assert np.array_equal(x, y), f"KV cache: {what}"


def test_prefill_pass_length_and_tile_give_same_results(ctx):
    """The prompt in passes of 64, 192 or all its 299 tokens at once, with the
    GEMMs in 128 x 128 or 256 x 256 tiles: the same KV cache rows, logits and
    tokens bit for bit, since each output row's GEMM sum (k in the same order
    in every tile form) and each query's attention are computed the same way
    in any pass."""
    import inferi_amd as I

    cfg = I.Llama2Config(n_layers=2, hidden=512, ffn=1024, n_heads=8, n_kv_heads=2, vocab=700, max_pos=400,
                         rope_theta=10000.0, rms_eps=1e-5, kv_dtype=I.F16)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=43, std=0.05)
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, 300).astype(np.uint32)
    out = {}
    ws0 = ctx.get_option("pf_ws")
    try:
        for tile, ws in TILE_FORMS:
            ctx.set_option("pf_tile", tile)
            ctx.set_option("pf_ws", ws)
            for chunk in (64, 192, 0):
                ctx.set_option("pf_chunk", chunk)
                out[tile, ws, chunk] = _prefill_run(ctx, cfg, w, prompt, 299, 6)
    finally:
        ctx.set_option("pf_chunk", 0)
        ctx.set_option("pf_tile", 0)
        ctx.set_option("pf_ws", ws0)
        w.close()
    ref = out[256, 0, 0]
    for key, got in out.items():
        _same(got, ref, f"tile {key[0]}{' warp-specialized' if key[1] else ''}, passes of {key[2] or 299}")


@pytest.mark.timeout(300)
@pytest.mark.parametrize("kv,bias", [("F16", False), ("F32", True)])
def test_prefill_fused_rope_same_results(ctx, kv, bias):
    """The Q/K/V product's epilogue with RoPE and the KV-cache store fused
    (option pf_rope_fuse, warp-specialized form) against the plain store
    epilogue followed by pf_rope_kv_k: the same KV cache rows, logits and
    tokens bit for bit, at the 8B widths (Q/K/V 6144 columns: a 4095-token
    pass has 256 whole tiles and 128 in halves), with f16 and f32 caches and
    with QKV biases on the (2i, 2i + 1) pairs."""
    import inferi_amd as I

    cfg = I.Llama2Config(n_layers=2, hidden=4096, ffn=1024, n_heads=32, n_kv_heads=8, vocab=1000, max_pos=4104,
                         rope_theta=500000.0, rms_eps=1e-5, kv_dtype=getattr(I, kv))
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=7, qkv_bias=bias)
    prompt = np.random.default_rng(17).integers(0, cfg.vocab, 4096).astype(np.uint32)
    fuse0 = ctx.get_option("pf_rope_fuse")
    out = {}
    try:
        for fuse in (0, 1):
            ctx.set_option("pf_rope_fuse", fuse)
            out[fuse] = _prefill_run(ctx, cfg, w, prompt, 4095, 3)
    finally:
        ctx.set_option("pf_rope_fuse", fuse0)
        w.close()
    _same(out[1], out[0], "fused RoPE epilogue")


def test_prefill_uses_weights_rewritten_in_place(ctx):
    """The prefill kernels read the bound GGUF blocks themselves: new bytes
    written into a bound tensor's buffer (no ifr_llama2_weights_set call) are
    what the next prefill multiplies, the same as binding a fresh buffer that
    holds them."""
    import inferi_amd as I

    cfg = I.Llama2Config(n_layers=2, hidden=512, ffn=1024, n_heads=8, n_kv_heads=2, vocab=700, max_pos=400,
                         rope_theta=10000.0, rms_eps=1e-5, kv_dtype=I.F16)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=47, std=0.05)
    prompt = np.random.default_rng(9).integers(0, cfg.vocab, 300).astype(np.uint32)
    rows, cols = cfg.hidden, cfg.ffn
    nbytes = rows * I.row_bytes(I.Q4_K, cols)
    tmp = ctx.alloc(rows * cols * 4)
    down = ctx.alloc(nbytes)
    try:
        before = _prefill_run(ctx, cfg, w, prompt, 299, 4)
        # another ffn_down for layer 0, quantized on the device
        ctx.fill_normal(tmp, rows * cols, 1234, 0, 0.0, 0.05)
        ctx.quantize(down, tmp, I.Q4_K, rows * cols)
        new_bytes = down.download(np.uint8, nbytes)
        bound = w.buffers["blk.0.ffn_down.weight"][1]
        ctx._check(I.lib().ifr_upload(ctx.h, bound.ptr, new_bytes.ctypes.data, nbytes))
        in_place = _prefill_run(ctx, cfg, w, prompt, 299, 4)
        w.set("blk.0.ffn_down.weight", I.Q4_K, down, rows, cols)
        bound.free()
        rebound = _prefill_run(ctx, cfg, w, prompt, 299, 4)
        _same(in_place, rebound, "bytes rewritten in place vs the same bytes bound anew")
        assert not np.array_equal(in_place[2][2], before[2][2]), "layer 1's K rows ignore the new matrix"
    finally:
        tmp.free()
        w.close()


def test_prefill_gate_up_of_different_types(ctx, oracle_lib):
    """A layer whose gate and up matrices differ in GGUF type takes separate
    gate and up products and the SiLU pass instead of the SwiGLU epilogue
    (the other layers keep it); against sequential decode."""
    import inferi_amd as I

    cfg = I.Llama2Config(n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, vocab=700, max_pos=160,
                         rope_theta=10000.0, rms_eps=1e-5, kv_dtype=I.F16)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=53, std=0.05, overrides={"blk.1.ffn_up.weight": I.Q6_K,
                                                                           "attn_v": I.Q8_0})
    try:
        prompt = np.random.default_rng(12).integers(0, cfg.vocab, 120).tolist()
        assert _prefill_vs_decode(ctx, cfg, w, prompt, 8) > 0
    finally:
        w.close()


def test_prefill_qwen2_style(ctx, oracle_lib):
    """NeoX RoPE pairs and QKV biases (Qwen2) in the prefill's RoPE/KV kernel."""
    import inferi_amd as I

    cfg = I.Llama2Config(n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, vocab=600, max_pos=160,
                         rope_theta=1000000.0, rms_eps=1e-6, kv_dtype=I.F16, rope_variant=I.ROPE_NEOX)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=43, std=0.05, qkv_bias=True)
    try:
        prompt = np.random.default_rng(5).integers(0, cfg.vocab, 130).tolist()
        assert _prefill_vs_decode(ctx, cfg, w, prompt, 8) > 0
    finally:
        w.close()


@pytest.mark.parametrize("mat,head", [("Q8_0", "Q8_0"), ("Q5_K", "Q6_K"), ("Q6_K", "Q4_K"), ("Q4_0", "Q8_K"),
                                      ("Q5_1", "Q4_1"), ("Q8_K", "Q5_0"), ("F16", "F16"), ("F32", "Q6_K")])
def test_prefill_other_formats(ctx, oracle_lib, mat, head):
    """Prefill with every layer matrix of another GGUF type."""
    import inferi_amd as I

    cfg = I.Llama2Config(n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, vocab=700, max_pos=128,
                         rope_theta=10000.0, rms_eps=1e-5, kv_dtype=I.F16)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=47, std=0.05, mat_dtype=getattr(I, mat), head_dtype=getattr(I, head),
                                  embd_dtype=getattr(I, mat))
    try:
        prompt = np.random.default_rng(6).integers(0, cfg.vocab, 100).tolist()
        assert _prefill_vs_decode(ctx, cfg, w, prompt, 8) > 0
    finally:
        w.close()


def test_prefill_rejects_unsupported(ctx):
    import inferi_amd as I

    cfg = I.Llama2Config(n_layers=1, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, vocab=300, max_pos=64,
                         rope_theta=10000.0, rms_eps=1e-5, kv_dtype=I.F16)
    s = I.Llama2State(ctx, cfg)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=5)
    try:
        s.reset([1, 2, 3], 0)
        with pytest.raises(I.HipError):
            I.Llama2.prefill(ctx, s, w, 5)  # only 3 prompt tokens
    finally:
        w.close()
        s.close()
        w.close()
