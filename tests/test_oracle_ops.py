"""Pins the oracle's GEMV, RMSNorm, RoPE, SiLU-mul, attention, argmax and
model forward against closed forms, invariants and independent numpy/scipy
computations.

Reference behaviour: crates/inferi/src/ops/gemv_quant.rs:444-456 (f64 GEMV
oracle), inferi-shaders/src/{rms_norm.rs:112-120, rope.rs:51-141,
silu.rs:24-53, fused_attention.rs:66-241}, models/sampler.rs:54-56 and
models/llama2/transformer.rs:409-481.
"""

import numpy as np
import pytest
from scipy.special import expit, softmax

import oracle as O
from tests import kquant as K


@pytest.mark.parametrize("dtype", [O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K])
def test_gemv_quant_selects_columns(oracle_lib, dtype):
    rows, cols = 8, 512
    rng = np.random.default_rng(dtype)
    w = K.random_blocks(dtype, rows * cols // O.BLOCK_ELEMS[dtype], rng)
    deq = O.dequant(dtype, w, rows * cols).reshape(rows, cols)
    for k in [0, 1, 255, 256, 511]:
        e = np.zeros(cols, np.float32)
        e[k] = 1.0
        y = O.gemv_quant(dtype, w, rows, cols, e)
        assert np.array_equal(y, deq[:, k])
    assert not O.gemv_quant(dtype, w, rows, cols, np.zeros(cols, np.float32)).any()


@pytest.mark.parametrize("dtype", [O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K])
def test_gemv_quant_vs_numpy(oracle_lib, dtype):
    rows, cols = 64, 1024
    rng = np.random.default_rng(20 + dtype)
    w = K.random_blocks(dtype, rows * cols // O.BLOCK_ELEMS[dtype], rng)
    x = (rng.random(cols) * 2 - 1).astype(np.float32)
    deq = O.dequant(dtype, w, rows * cols).reshape(rows, cols)
    ref = (deq.astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
    for nt in (1, 3, 0):
        y = O.gemv_quant(dtype, w, rows, cols, x, nthreads=nt)
        assert np.allclose(y, ref, rtol=1e-6, atol=1e-30)
    assert np.allclose(O.gemv_f64(deq, x), ref, rtol=1e-6, atol=1e-30)


@pytest.mark.parametrize("dtype", [O.Q8_0, O.Q4_K], ids=["Q8_0", "Q4_K"])
def test_gemv_f32_accumulation_mode(oracle_lib, dtype):
    """The f32-accumulation mode is the left-to-right f32 dot (each product
    and sum rounded) bit for bit, the f64 mode is restored after the block,
    and the two differ by no more than the f32 rounding bound."""
    rng = np.random.default_rng(11)
    rows, cols = 6, 512
    blocks = K.random_blocks(dtype, rows * cols // O.BLOCK_ELEMS[dtype], rng)
    x = rng.standard_normal(cols).astype(np.float32)
    wd = O.dequant(dtype, blocks, rows * cols).reshape(rows, cols)
    with O.f32_accumulation():
        y32 = O.gemv_quant(dtype, blocks, rows, cols, x)
    y64 = O.gemv_quant(dtype, blocks, rows, cols, x)
    seq = np.array([np.add.accumulate((wd[r] * x).astype(np.float32), dtype=np.float32)[-1] for r in range(rows)])
    assert np.array_equal(y32.view(np.uint32), seq.view(np.uint32))
    assert np.array_equal(y64, (wd.astype(np.float64) @ x.astype(np.float64)).astype(np.float32))
    bound = cols * np.finfo(np.float32).eps * (np.abs(wd).astype(np.float64) @ np.abs(x).astype(np.float64))
    assert np.all(np.abs(y32.astype(np.float64) - y64) <= bound + np.abs(y64) * 1e-7)


def test_rms_norm_closed_forms(oracle_lib):
    n = 4096
    w = np.linspace(0.5, 1.5, n).astype(np.float32)
    for c, eps in [(2.0, 1e-5), (-0.25, 1e-6), (3e-3, 1e-5)]:
        x = np.full(n, c, np.float32)
        out = O.rms_norm(x, w, eps)
        expect = (c / np.sqrt(c * c + eps)) * w.astype(np.float64)
        assert np.allclose(out, expect, rtol=2e-7)
    rng = np.random.default_rng(1)
    x = rng.standard_normal(n).astype(np.float32)
    a = O.rms_norm(x, w, 0.0)
    b = O.rms_norm(x * np.float32(8.0), w, 0.0)  # scale invariance with eps = 0
    assert np.allclose(a, b, rtol=1e-6)
    assert abs(np.sqrt(np.mean((a / w) ** 2)) - 1.0) < 1e-5


def test_rope_identity_norms_and_closed_form(oracle_lib):
    rng = np.random.default_rng(2)
    hs, nq, nkv = 128, 32, 8
    q = rng.standard_normal(nq * hs).astype(np.float32)
    k = rng.standard_normal(nkv * hs).astype(np.float32)
    q0, k0 = O.rope(q, k, hs, 0, 500000.0)
    assert np.array_equal(q0, q) and np.array_equal(k0, k)
    for pos in (1, 7, 4095):
        q1, k1 = O.rope(q, k, hs, pos, 500000.0)
        pn = lambda v: np.hypot(v[0::2].astype(np.float64), v[1::2].astype(np.float64))
        assert np.allclose(pn(q1), pn(q), rtol=1e-6)
        assert np.allclose(pn(k1), pn(k), rtol=1e-6)
        # pair 0 of every head has theta = base^0 = 1, so its angle is pos radians
        for h in range(nq):
            a, b = float(q[h * hs]), float(q[h * hs + 1])
            assert np.isclose(q1[h * hs], np.cos(pos) * a - np.sin(pos) * b, rtol=1e-5, atol=1e-6)
            assert np.isclose(q1[h * hs + 1], np.sin(pos) * a + np.cos(pos) * b, rtol=1e-5, atol=1e-6)
    # the key vector is shorter than q: only its kv_dim entries rotate
    assert O.rope(q, k, hs, 3, 1e4)[1].size == k.size


def test_rope_composition_and_neox_pairs(oracle_lib):
    rng = np.random.default_rng(4)
    hs = 64
    q = rng.standard_normal(4 * hs).astype(np.float32)
    for neox in (False, True):
        a, _ = O.rope(q, None, hs, 5, 10000.0, neox)
        ab, _ = O.rope(a, None, hs, 9, 10000.0, neox)
        c, _ = O.rope(q, None, hs, 14, 10000.0, neox)
        assert np.allclose(ab, c, atol=2e-5)  # rotations by 5 and then 9 compose to 14
    # NeoX rotates (i, i + hs/2): a vector supported on one such pair stays there
    v = np.zeros(hs, np.float32)
    v[3] = 1.0
    r, _ = O.rope(v, None, hs, 2, 10000.0, True)
    nz = np.nonzero(r)[0].tolist()
    assert set(nz) <= {3, 3 + hs // 2} and np.isclose(np.hypot(r[3], r[3 + hs // 2]), 1.0)
    r, _ = O.rope(v, None, hs, 2, 10000.0, False)
    assert set(np.nonzero(r)[0].tolist()) <= {2, 3}


def test_silu_mul_vs_expit(oracle_lib):
    rng = np.random.default_rng(8)
    h1 = (rng.standard_normal(14336) * 4).astype(np.float32)
    h2 = rng.standard_normal(14336).astype(np.float32)
    out = O.silu_mul(h1, h2)
    expect = h2.astype(np.float64) * h1.astype(np.float64) * expit(h1.astype(np.float64))
    assert np.allclose(out, expect, rtol=1e-6, atol=1e-30)


def _attn_numpy(q, kc, vc, nh, nkv, hs, pos):
    out = np.zeros(nh * hs)
    for h in range(nh):
        g = h // (nh // nkv)
        K_ = kc[: pos + 1, g * hs:(g + 1) * hs].astype(np.float64)
        V_ = vc[: pos + 1, g * hs:(g + 1) * hs].astype(np.float64)
        p = softmax(K_ @ q[h * hs:(h + 1) * hs].astype(np.float64) / np.sqrt(hs))
        out[h * hs:(h + 1) * hs] = p @ V_
    return out


@pytest.mark.parametrize("kv_f16", [False, True])
def test_attention_closed_forms_and_brute_force(oracle_lib, kv_f16):
    rng = np.random.default_rng(9)
    nh, nkv, hs, max_pos = 8, 2, 32, 40
    kv_dim = nkv * hs
    kc = rng.standard_normal((max_pos, kv_dim)).astype(np.float32)
    vc = rng.standard_normal((max_pos, kv_dim)).astype(np.float32)
    if kv_f16:
        kc = kc.astype(np.float16).astype(np.float32)
        vc = vc.astype(np.float16).astype(np.float32)
    enc = (lambda a: a.astype(np.float16).view(np.uint16)) if kv_f16 else (lambda a: a)
    q = rng.standard_normal(nh * hs).astype(np.float32)
    # pos 0: a single key, so out_h = v_0 of its kv head
    out = O.attention(q, enc(kc), enc(vc), nh, nkv, hs, 0, kv_f16)
    for h in range(nh):
        g = h // (nh // nkv)
        assert np.allclose(out[h * hs:(h + 1) * hs], vc[0, g * hs:(g + 1) * hs], rtol=1e-6)
    # identical keys: uniform weights, out = mean of V rows 0..pos
    kk = np.tile(kc[:1], (max_pos, 1))
    out = O.attention(q, enc(kk), enc(vc), nh, nkv, hs, 9, kv_f16)
    for h in range(nh):
        g = h // (nh // nkv)
        assert np.allclose(out[h * hs:(h + 1) * hs], vc[:10, g * hs:(g + 1) * hs].mean(0), rtol=1e-5, atol=1e-6)
    for pos in (5, 39):
        out = O.attention(q, enc(kc), enc(vc), nh, nkv, hs, pos, kv_f16)
        assert np.allclose(out, _attn_numpy(q, kc, vc, nh, nkv, hs, pos), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("nh,nkv,hs", [(14, 2, 64), (24, 8, 128), (24, 2, 32), (20, 2, 80), (6, 3, 40), (4, 4, 8)])
def test_attention_any_group_and_head_size(oracle_lib, nh, nkv, hs):
    """The group sizes (7, 3, 12, 10, 2, 1) and head sizes the device kernels
    take, against numpy in f64, including a position past 65,536."""
    rng = np.random.default_rng(nh * 100 + hs)
    L = 70001 if hs == 8 else 300
    kv_dim = nkv * hs
    kc = rng.standard_normal((L, kv_dim)).astype(np.float32)
    vc = rng.standard_normal((L, kv_dim)).astype(np.float32)
    q = rng.standard_normal(nh * hs).astype(np.float32)
    for pos in (0, 17, L - 1):
        out = O.attention(q, kc, vc, nh, nkv, hs, pos, False)
        assert np.allclose(out, _attn_numpy(q, kc, vc, nh, nkv, hs, pos), rtol=1e-5, atol=1e-6)


def test_argmax_ties_lowest_index(oracle_lib):
    v = np.array([1.0, 3.0, -2.0, 3.0, 3.0], np.float32)
    assert O.argmax(v) == 1
    v = np.full(1000, -5.0, np.float32)
    assert O.argmax(v) == 0
    v[777] = 0.0
    assert O.argmax(v) == 777


# --------------------------------------------------------------- forward --

def tiny_config(**kw):
    c = dict(hidden=64, ffn=128, n_layers=2, n_heads=4, n_kv_heads=2, vocab=50, max_pos=16,
             rope_theta=10000.0, rms_eps=1e-5, kv_f16=1)
    c.update(kw)
    return c


def random_weights(c, rng, mat_dtype=O.Q8_0, head_dtype=O.Q8_0, embd_dtype=O.Q8_0, zero_layers=False, bias=False):
    """Random model in GGUF block form.  Hidden 64 only fits 32-element blocks.
    bias: Qwen2's attn_{q,k,v}.bias vectors."""
    hd, kv = c["hidden"], c["hidden"] * c["n_kv_heads"] // c["n_heads"]
    shapes = {"attn_q": (hd, hd), "attn_k": (kv, hd), "attn_v": (kv, hd), "attn_output": (hd, hd),
              "ffn_gate": (c["ffn"], hd), "ffn_up": (c["ffn"], hd), "ffn_down": (hd, c["ffn"])}
    w = {}

    def qt(dt, rows, cols, scale=0.2, zero=False):
        x = (rng.standard_normal(rows * cols) * scale).astype(np.float32)
        if zero:
            x[:] = 0
        return (dt, O.quantize(dt, x), rows, cols)

    for l in range(c["n_layers"]):
        for m, (r, cc) in shapes.items():
            w[f"blk.{l}.{m}.weight"] = qt(mat_dtype, r, cc, zero=zero_layers)
        w[f"blk.{l}.attn_norm.weight"] = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
        w[f"blk.{l}.ffn_norm.weight"] = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
        if bias:
            for b, n in (("q", hd), ("k", kv), ("v", kv)):
                w[f"blk.{l}.attn_{b}.bias"] = (0.5 * rng.standard_normal(n)).astype(np.float32)
    w["token_embd.weight"] = qt(embd_dtype, c["vocab"], hd, 1.0)
    w["output.weight"] = qt(head_dtype, c["vocab"], hd)
    w["output_norm.weight"] = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    return w


def numpy_forward(c, w, tokens):
    """f64 re-derivation of the decode loop from the reference's description
    (transformer.rs:409-481), using only numpy/scipy and the dequantizer."""
    hd, nh, nkv = c["hidden"], c["n_heads"], c["n_kv_heads"]
    hs, kv = hd // nh, hd * nkv // nh
    deq = {}
    for name, v in w.items():
        if isinstance(v, tuple):
            dt, data, r, cc = v
            deq[name] = O.dequant(dt, data, r * cc).reshape(r, cc).astype(np.float64)
        else:
            deq[name] = v.astype(np.float64)
    kc = np.zeros((c["n_layers"], c["max_pos"], kv))
    vc = np.zeros((c["n_layers"], c["max_pos"], kv))

    def rms(x, g):
        return x / np.sqrt(np.mean(x * x) + c["rms_eps"]) * g

    def rope(v, pos):
        # original: pairs (2j, 2j+1); NeoX (rope.rs:97-141): pairs (j, j + hs/2)
        # within each head; both rotate by pos * base^(-2j/hs)
        v = v.copy()
        for h in range(v.size // hs):
            for j in range(hs // 2):
                th = np.float32(c["rope_theta"]) ** (-np.float32(2 * j) / np.float32(hs))
                a = np.float64(np.float32(pos) * np.float32(th))
                i0, i1 = (h * hs + j, h * hs + j + hs // 2) if c.get("rope_neox") else (h * hs + 2 * j, h * hs + 2 * j + 1)
                x0, x1 = v[i0], v[i1]
                v[i0], v[i1] = np.cos(a) * x0 - np.sin(a) * x1, np.sin(a) * x0 + np.cos(a) * x1
        return v

    all_logits = []
    for pos, tok in enumerate(tokens):
        x = deq["token_embd.weight"][tok].copy()
        for l in range(c["n_layers"]):
            g = lambda m: deq[f"blk.{l}.{m}.weight"]
            xb = rms(x, g("attn_norm"))
            bq, bk, bv = (deq.get(f"blk.{l}.attn_{b}.bias", 0.0) for b in "qkv")
            q = rope(g("attn_q") @ xb + bq, pos)
            k = rope(g("attn_k") @ xb + bk, pos)
            v = g("attn_v") @ xb + bv
            f = (lambda a: a.astype(np.float16).astype(np.float64)) if c["kv_f16"] else (lambda a: a)
            kc[l, pos], vc[l, pos] = f(k), f(v)
            att = np.zeros(hd)
            for h in range(nh):
                gk = h // (nh // nkv)
                s = kc[l, :pos + 1, gk * hs:(gk + 1) * hs] @ q[h * hs:(h + 1) * hs] / np.sqrt(hs)
                att[h * hs:(h + 1) * hs] = softmax(s) @ vc[l, :pos + 1, gk * hs:(gk + 1) * hs]
            x = x + g("attn_output") @ att
            xb = rms(x, g("ffn_norm"))
            hg, hu = g("ffn_gate") @ xb, g("ffn_up") @ xb
            x = x + g("ffn_down") @ (hu * hg * expit(hg))
        all_logits.append(deq["output.weight"] @ rms(x, deq["output_norm.weight"]))
    return all_logits


@pytest.mark.parametrize("kv_f16,qwen2", [(1, 0), (0, 0), (1, 1)], ids=["f16", "f32", "qwen2"])
def test_forward_vs_numpy_rederivation(oracle_lib, kv_f16, qwen2):
    """qwen2: QKV biases added before RoPE (transformer.rs:434-442) and the
    NeoX RoPE pairing (models/llama2/mod.rs:25-30)."""
    c = tiny_config(kv_f16=kv_f16, rope_neox=qwen2)
    rng = np.random.default_rng(1234)
    w = random_weights(c, rng, bias=bool(qwen2))
    m = O.Model(c, w)
    tokens = [3, 17, 42, 0, 49, 8, 8, 21]
    ref = numpy_forward(c, w, tokens)
    for pos, tok in enumerate(tokens):
        logits = m.forward(tok, pos)
        assert np.allclose(logits, ref[pos], rtol=1e-4, atol=1e-4), pos


def test_forward_zero_layers_reduces_to_head(oracle_lib):
    """With all layer matrices zero every residual branch adds 0, so the logits
    are output @ rmsnorm(embedding row): no attention, FFN or RoPE involved."""
    c = tiny_config()
    rng = np.random.default_rng(77)
    w = random_weights(c, rng, zero_layers=True)
    m = O.Model(c, w)
    emb = O.dequant(*w["token_embd.weight"][:2], c["vocab"] * c["hidden"]).reshape(c["vocab"], c["hidden"])
    head = O.dequant(*w["output.weight"][:2], c["vocab"] * c["hidden"]).reshape(c["vocab"], c["hidden"])
    for pos, tok in enumerate([5, 6, 7]):
        x = emb[tok].astype(np.float64)
        xn = x / np.sqrt(np.mean(x * x) + c["rms_eps"]) * w["output_norm.weight"]
        assert np.allclose(m.forward(tok, pos), head @ xn, rtol=1e-5, atol=1e-6)


def test_generate_forces_prompt_then_greedy(oracle_lib):
    c = tiny_config()
    w = random_weights(c, np.random.default_rng(5))
    prompt = [1, 2, 3, 4]
    m = O.Model(c, w)
    margins = []
    gen = m.generate(prompt, 5, margins=margins)
    assert len(gen) == 5 and len(margins) == 5 and all(mg >= 0 for mg in margins)
    # replay: forced prompt, then feed back each generated token
    m2 = O.Model(c, w)
    seq = prompt + gen
    for pos in range(len(seq) - 1):
        lg = m2.forward(seq[pos], pos)
        if pos >= len(prompt) - 1:
            assert O.argmax(lg) == seq[pos + 1]
