"""GGUF model loading on the device (ifr_llama2_config_from_gguf,
ifr_llama2_weights_from_gguf; Llama2Config::from_gguf cpu.rs:74-107,
Llama2Weights::from_gguf transformer.rs:294-393): a model written to a GGUF
file and read back decodes bit-identically to the same bytes bound directly,
and a file without output.weight uses token_embd.weight as the head
(transformer.rs:376-382)."""

import numpy as np
import pytest

import inferi_amd as I

pytestmark = pytest.mark.gpu


def tiny_cfg():
    return I.Llama2Config(n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, vocab=512, max_pos=32,
                          rope_theta=10000.0, rms_eps=1e-5, kv_dtype=I.F16)


def decode(ctx, cfg, w, prompt, n):
    s = I.Llama2State(ctx, cfg)
    try:
        s.reset(prompt, 0)
        logits = []
        for _ in range(n):
            I.Llama2.launch(ctx, s, w)
            logits.append(s.read("logits"))
        return np.stack(logits), s.tokens(0, n + 1)
    finally:
        s.close()


@pytest.mark.parametrize("mat,head,embd", [(I.Q4_K, I.Q6_K, I.Q8_0), (I.Q4_0, I.Q8_K, I.Q5_1), (I.Q5_0, I.Q4_1, I.Q4_0),
                                           (I.Q4_K, I.F16, I.F16), (I.F16, I.F32, I.F16)],
                         ids=["k_quants", "q4_0_q8_k_q5_1", "q5_0_q4_1_q4_0", "f16_head", "f16_matrices"])
def test_model_round_trips_through_gguf(ctx, tmp_path, mat, head, embd):
    cfg = tiny_cfg()
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=11, mat_dtype=mat, head_dtype=head, embd_dtype=embd)
    path = str(tmp_path / "tiny.gguf")
    w.to_gguf(path)
    g = I.Gguf(path)
    c2 = I.Llama2Config.from_gguf(g)
    assert (c2.n_layers, c2.hidden, c2.ffn, c2.n_heads, c2.n_kv_heads, c2.vocab, c2.max_pos) == \
        (cfg.n_layers, cfg.hidden, cfg.ffn, cfg.n_heads, cfg.n_kv_heads, cfg.vocab, cfg.max_pos)
    assert c2.rope_theta == cfg.rope_theta and c2.rms_eps == np.float32(cfg.rms_eps)
    assert c2.kv_dtype == I.F32  # the reference's cache; choose the f16 cache of the bound model below
    c2.kv_dtype = I.F16
    w2 = I.Llama2Weights.from_gguf(ctx, g, c2)
    g.close()  # the weights own device copies; the mapping can go
    try:
        a, ta = decode(ctx, cfg, w, [3, 7], 6)
        b, tb = decode(ctx, c2, w2, [3, 7], 6)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert np.array_equal(ta, tb)
    finally:
        w2.close()
        w.close()


def test_tied_embeddings_and_bad_files(ctx, tmp_path):
    cfg = tiny_cfg()
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=12, mat_dtype=I.Q4_K, head_dtype=I.Q4_K, embd_dtype=I.Q4_K)
    wr = I.GgufWriter()
    wr.set("general.architecture", I.GGUF_STRING, "llama")
    for key, ty, val in cfg.gguf_metadata():
        wr.set(key, ty, val)
    wr.set_array("tokenizer.ggml.tokens", I.GGUF_STRING, [str(i) for i in range(cfg.vocab)])
    for name in w.buffers:
        if name == "output.weight":
            continue
        dtype, arr, rows, cols = w.download(name)
        wr.add_tensor(name, dtype, [cols] if name.endswith("norm.weight") else [rows, cols], arr)
    path = str(tmp_path / "tied.gguf")
    wr.save(path)
    wr.close()
    # the same bytes bound directly, with token_embd as the head
    tied = I.Llama2Weights(ctx, cfg)
    for name, (dtype, buf, rows, cols) in w.buffers.items():
        tied.ctx._check(I.lib().ifr_llama2_weights_set(tied.h, name.encode(), dtype, buf.ptr, rows, cols))
    emb = w.buffers["token_embd.weight"]
    tied.ctx._check(I.lib().ifr_llama2_weights_set(tied.h, b"output.weight", emb[0], emb[1].ptr, emb[2], emb[3]))
    g = I.Gguf(path)
    c2 = I.Llama2Config.from_gguf(g)
    c2.kv_dtype = I.F16
    w2 = I.Llama2Weights.from_gguf(ctx, g, c2)
    try:
        a, _ = decode(ctx, cfg, tied, [5], 4)
        b, _ = decode(ctx, c2, w2, [5], 4)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        # a file whose tensor shapes disagree with its metadata is refused
        bad = I.Llama2Config.from_gguf(g)
        bad.ffn = 1024
        with pytest.raises(I.HipError):
            I.Llama2Weights.from_gguf(ctx, g, bad)
    finally:
        g.close()
        w2.close()
        lib_destroy = I.lib().ifr_llama2_weights_destroy
        lib_destroy(tied.h)
        tied.h = None
        w.close()


def test_qwen2_model_round_trips_through_gguf(ctx, tmp_path):
    """A Qwen2-style model (NeoX RoPE, QKV biases) written under
    general.architecture = qwen2 reads back with the qwen2.* keys, the NeoX
    variant and its biases, and decodes bit-identically."""
    cfg = I.Llama2Config(n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, vocab=512, max_pos=32,
                         rope_theta=1000000.0, rms_eps=1e-6, kv_dtype=I.F16, rope_variant=I.ROPE_NEOX)
    w = I.Llama2Weights.synthetic(ctx, cfg, seed=17, qkv_bias=True, std=0.05)
    path = str(tmp_path / "qwen.gguf")
    w.to_gguf(path)
    g = I.Gguf(path)
    assert g.get("general.architecture") == "qwen2" and "qwen2.block_count" in g.keys()
    assert "blk.1.attn_k.bias" in g.tensor_names()
    c2 = I.Llama2Config.from_gguf(g)
    assert c2.rope_variant == I.ROPE_NEOX
    c2.kv_dtype = I.F16
    w2 = I.Llama2Weights.from_gguf(ctx, g, c2)
    try:
        a, ta = decode(ctx, cfg, w, [9, 4], 5)
        b, tb = decode(ctx, c2, w2, [9, 4], 5)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)) and np.array_equal(ta, tb)
    finally:
        g.close()
        w2.close()
        w.close()
