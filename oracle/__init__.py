"""ctypes wrapper around the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY.  This is the checker the HIP path is compared
against.  Only tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg may import it; the product package ``inferi_amd`` never
does, and has no CPU fallback built on it.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 8, 12, 13, 14
Q4_0, Q4_1, Q5_0, Q5_1, Q8_K = 2, 3, 6, 7, 15
BLOCK_ELEMS = {F32: 1, F16: 1, Q4_0: 32, Q4_1: 32, Q5_0: 32, Q5_1: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256,
               Q8_K: 256}
BLOCK_BYTES = {F32: 4, F16: 2, Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210,
               Q8_K: 292}
NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q4_1: "Q4_1", Q5_0: "Q5_0", Q5_1: "Q5_1", Q8_0: "Q8_0",
         Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", Q8_K: "Q8_K"}


def build() -> None:
    """Compile liboracle.so from oracle.c (gcc only)."""
    subprocess.run(["make", "-s", "-C", HERE, "-B"], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        L = C.CDLL(LIB_PATH)
        vp, i, f, sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t
        L.ifo_decode_f16.restype = f
        L.ifo_decode_f16.argtypes = [C.c_uint16]
        L.ifo_encode_f16.restype = C.c_uint16
        L.ifo_encode_f16.argtypes = [f]
        L.ifo_decode_f16_array.argtypes = [vp, vp, sz]
        L.ifo_encode_f16_array.argtypes = [vp, vp, sz]
        L.ifo_get_scale_min_k4.argtypes = [i, vp, vp, vp]
        L.ifo_dequant.argtypes = [i, vp, sz, vp]
        L.ifo_dequant.restype = i
        L.ifo_quantize.argtypes = [i, vp, sz, vp]
        L.ifo_quantize.restype = i
        L.ifo_gemv_f64.argtypes = [vp, i, i, vp, vp]
        L.ifo_gemv_quant.argtypes = [i, vp, i, i, vp, vp, i]
        L.ifo_gemv_quant.restype = i
        u32 = C.c_uint32
        L.ifo_ref_gemv.argtypes = [C.c_int32, u32, u32, vp, vp, vp, i]
        L.ifo_ref_gemv.restype = i
        L.ifo_ref_attention.argtypes = [vp, vp, vp, u32, u32, u32, u32, vp, i]
        L.ifo_ref_attention.restype = i
        L.ifo_rms_norm.argtypes = [vp, vp, vp, i, f]
        L.ifo_rope.argtypes = [i, vp, i, vp, i, i, i, f]
        L.ifo_silu_mul.argtypes = [vp, vp, i]
        L.ifo_add.argtypes = [vp, vp, i]
        L.ifo_attention.argtypes = [vp, vp, vp, vp, i, vp]
        L.ifo_argmax.argtypes = [vp, i]
        L.ifo_argmax.restype = i
        L.ifo_set_f32_accum.argtypes = [i]
        L.ifo_softmax.argtypes = [vp, i]
        L.ifo_sample_mult.argtypes = [vp, i, f]
        L.ifo_sample_mult.restype = i
        L.ifo_sample_topp.argtypes = [vp, i, f, f, vp, vp]
        L.ifo_sample_topp.restype = i
        L.ifo_sample.argtypes = [vp, i, f, f, f]
        L.ifo_sample.restype = i
        L.ifo_state_new.argtypes = [vp]
        L.ifo_state_new.restype = vp
        L.ifo_state_free.argtypes = [vp]
        L.ifo_forward.argtypes = [vp, vp, i, i, vp, i]
        L.ifo_forward.restype = i
        L.ifo_state_buffer.argtypes = [vp, i, i]
        L.ifo_state_buffer.restype = vp
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def decode_f16(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().ifo_decode_f16_array(_p(h), _p(out), h.size)
    return out


def encode_f16(f) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().ifo_encode_f16_array(_p(f), _p(out), f.size)
    return out


def get_scale_min_k4(j: int, q: bytes) -> tuple[int, int]:
    qa = np.frombuffer(bytes(q), dtype=np.uint8).copy()
    d = np.zeros(1, np.uint8)
    m = np.zeros(1, np.uint8)
    lib().ifo_get_scale_min_k4(j, _p(qa), _p(d), _p(m))
    return int(d[0]), int(m[0])


def row_bytes(dtype: int, cols: int) -> int:
    return cols // BLOCK_ELEMS[dtype] * BLOCK_BYTES[dtype]


def dequant(dtype: int, data, n_elems: int) -> np.ndarray:
    buf = np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8) if isinstance(data, (bytes, bytearray)) else data).view(np.uint8)
    if buf.size < n_elems // BLOCK_ELEMS[dtype] * BLOCK_BYTES[dtype]:
        raise ValueError("dequant: buffer too small")
    out = np.empty(n_elems, np.float32)
    if lib().ifo_dequant(dtype, _p(buf), n_elems, _p(out)) != 0:
        raise ValueError("dequant: bad dtype or size")
    return out


def quantize(dtype: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(x.size // BLOCK_ELEMS[dtype] * BLOCK_BYTES[dtype], np.uint8)
    if lib().ifo_quantize(dtype, _p(x), x.size, _p(out)) != 0:
        raise ValueError("quantize: bad dtype or size")
    return out


def gemv_f64(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(w.shape[0], np.float32)
    lib().ifo_gemv_f64(_p(w), w.shape[0], w.shape[1], _p(x), _p(y))
    return y


def gemv_quant(dtype: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray, nthreads: int = 0) -> np.ndarray:
    w = np.ascontiguousarray(w).view(np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    assert w.size >= rows * row_bytes(dtype, cols) and x.size == cols
    y = np.empty(rows, np.float32)
    if lib().ifo_gemv_quant(dtype, _p(w), rows, cols, _p(x), _p(y), nthreads) != 0:
        raise ValueError("gemv_quant: bad shape")
    return y


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().ifo_rms_norm(_p(out), _p(x), _p(w), x.size, eps)
    return out


def rope(q: np.ndarray, k: np.ndarray | None, head_size: int, pos: int, base: float, neox: bool = False):
    q = np.array(q, np.float32, copy=True)
    kk = np.array(k if k is not None else np.zeros(0), np.float32, copy=True)
    lib().ifo_rope(int(neox), _p(q), q.size, _p(kk) if kk.size else None, kk.size, head_size, pos, base)
    return q, kk


def silu_mul(h1: np.ndarray, h2: np.ndarray) -> np.ndarray:
    h = np.array(h1, np.float32, copy=True)
    h2 = np.ascontiguousarray(h2, np.float32)
    lib().ifo_silu_mul(_p(h), _p(h2), h.size)
    return h


class AttnParams(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("seq_len", "kv_dim", "kv_mul", "n_heads", "head_size", "pos")]


def attention(q, k_cache, v_cache, n_heads: int, n_kv_heads: int, head_size: int, pos: int, kv_f16: bool) -> np.ndarray:
    """k_cache/v_cache: [max_pos, kv_dim] as float32, or uint16 binary16 codes when kv_f16."""
    q = np.ascontiguousarray(q, np.float32)
    kt = np.uint16 if kv_f16 else np.float32
    k_cache = np.ascontiguousarray(k_cache, kt)
    v_cache = np.ascontiguousarray(v_cache, kt)
    kv_dim = n_kv_heads * head_size
    p = AttnParams(k_cache.shape[0], kv_dim, n_heads // n_kv_heads, n_heads, head_size, pos)
    out = np.empty(n_heads * head_size, np.float32)
    lib().ifo_attention(C.byref(p), _p(q), _p(k_cache), _p(v_cache), int(kv_f16), _p(out))
    return out


def ref_gemv(dtype: int, w, rows: int, cols: int, x: np.ndarray, nthreads: int = 1) -> np.ndarray:
    """The reference GEMV shader's decomposition on host threads
    (oracle/ref_shaders.c): the CPU baseline of the GEMV configs."""
    w = np.ascontiguousarray(w).view(np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    assert w.size >= rows * row_bytes(dtype, cols) and x.size == cols
    y = np.empty(rows, np.float32)
    if lib().ifo_ref_gemv(dtype, rows, cols, _p(w), _p(x), _p(y), nthreads) != 0:
        raise ValueError("ref_gemv: a shape the reference shader does not take")
    return y


def ref_attention(q, k_cache, v_cache, n_heads: int, n_kv_heads: int, head_size: int, pos: int,
                  nthreads: int = 1) -> np.ndarray:
    """The reference attention shaders' decomposition on host threads over
    f16 caches (uint16 codes, [>= pos + 1, kv_dim]): fused_attention up to
    2048 positions, flash_attention beyond."""
    q = np.ascontiguousarray(q, np.float32)
    k_cache = np.ascontiguousarray(k_cache, np.uint16)
    v_cache = np.ascontiguousarray(v_cache, np.uint16)
    out = np.empty(n_heads * head_size, np.float32)
    if lib().ifo_ref_attention(_p(q), _p(k_cache), _p(v_cache), n_heads, n_kv_heads, head_size, pos, _p(out),
                               nthreads) != 0:
        raise ValueError("ref_attention: bad shape")
    return out


class f32_accumulation:
    """Within the block the quantized GEMVs (and so Model.forward) accumulate
    in f32 left to right, as the reference's CPU path does, instead of f64:
    the spread between the two is the noise floor of f32 arithmetic."""

    def __enter__(self):
        lib().ifo_set_f32_accum(1)
        return self

    def __exit__(self, *exc):
        lib().ifo_set_f32_accum(0)
        return False


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return lib().ifo_argmax(_p(v), v.size)


# --------------------------------------------------------------- sampler --
# Reference restatement in C (f32 running sums, models/sampler.rs:32-131) and
# the same algorithm with exact running sums over probabilities truncated to
# multiples of 2^-40, which is what the device sampler computes.

def softmax(v: np.ndarray) -> np.ndarray:
    """SoftMax::run_cpu (ops/softmax.rs:130-143) on a copy."""
    out = np.array(v, np.float32, copy=True)
    lib().ifo_softmax(_p(out), out.size)
    return out


def sample_mult(p: np.ndarray, coin: float) -> int:
    p = np.ascontiguousarray(p, np.float32)
    return lib().ifo_sample_mult(_p(p), p.size, float(coin))


def sample_topp(p: np.ndarray, topp: float, coin: float) -> tuple[int, int, float]:
    """(index, truncation position, cumulative probability); index -1 where
    the reference has no candidate."""
    p = np.ascontiguousarray(p, np.float32)
    last, cum = C.c_int(-1), C.c_float(0.0)
    idx = lib().ifo_sample_topp(_p(p), p.size, float(topp), float(coin), C.byref(last), C.byref(cum))
    return idx, last.value, cum.value


def sample(logits: np.ndarray, temperature: float, topp: float, coin: float) -> tuple[int, np.ndarray]:
    """Sampler::sample (models/sampler.rs:32-52) with the coin given: (index,
    the logits as the reference leaves them, i.e. the probabilities)."""
    v = np.array(logits, np.float32, copy=True)
    idx = lib().ifo_sample(_p(v), v.size, float(temperature), float(topp), float(coin))
    return idx, v


FX_ONE = 2 ** 40


def prob_fx(p) -> np.ndarray:
    """floor(p * 2^40) of non-negative f32 values, as uint64 (exact)."""
    p = np.asarray(p, np.float32).astype(np.float64)
    return np.floor(np.maximum(p, 0.0) * FX_ONE).astype(np.uint64)


def clamp_coin(coin: float) -> np.float32:
    c = np.float32(coin)
    if not c >= 0:
        return np.float32(0.0)
    return min(c, np.float32(np.nextafter(np.float32(1.0), np.float32(0.0))))


def sample_mult_exact(p: np.ndarray, coin: float) -> int:
    """sample_mult with exact running sums: the first index whose summed
    2^-40 units exceed floor(coin * 2^40), n - 1 if none does."""
    c = prob_fx(clamp_coin(coin))
    cdf = np.cumsum(prob_fx(p), dtype=np.uint64)
    i = int(np.searchsorted(cdf, c, side="right"))
    return min(i, p.size - 1)


def sample_topp_exact(p: np.ndarray, topp: float, coin: float, fallback: int) -> int:
    """sample_topp with exact running sums.  The candidates (p >= cutoff,
    f32 as the reference computes it) in order of probability descending,
    index ascending; truncated at the first whose running sum exceeds
    floor(topp * 2^40) (else all); then the first whose running sum exceeds
    floor(coin * cum) with the product in f64.  `fallback` is returned when
    there is no candidate."""
    p = np.asarray(p, np.float32)
    n = p.size
    with np.errstate(divide="ignore", invalid="ignore"):  # n == 1: cutoff inf, no candidate
        cutoff = np.float32(np.float32(np.float32(1.0) - np.float32(topp)) / np.float32(np.float32(n) - np.float32(1.0)))
        cand = np.nonzero(p >= cutoff)[0]
    if cand.size == 0:
        return int(fallback)
    order = cand[np.lexsort((cand, -p[cand]))]
    cum = np.cumsum(prob_fx(p[order]), dtype=np.uint64)
    t = prob_fx(np.float32(topp))
    hit = np.nonzero(cum > t)[0]
    last = int(hit[0]) if hit.size else order.size - 1
    cum_last = cum[last]
    r = np.uint64(np.floor(np.float64(clamp_coin(coin)) * np.float64(cum_last)))
    j = int(np.searchsorted(cum[: last + 1], r, side="right"))
    return int(order[min(j, last)])


def seeded_coin(seed: int, pos: int) -> np.float32:
    """The decode step's coin for position `pos`: 24 bits of the splitmix64
    finaliser of seed + pos * 0x9E3779B97F4A7C15 (mod 2^64)."""
    m = (1 << 64) - 1
    z = (seed + pos * 0x9E3779B97F4A7C15) & m
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    z ^= z >> 31
    return np.float32((z >> 40) / 16777216.0)


# ------------------------------------------------------------------ model --

class _Config(C.Structure):
    _fields_ = [("hidden", C.c_int), ("ffn", C.c_int), ("n_layers", C.c_int), ("n_heads", C.c_int),
                ("n_kv_heads", C.c_int), ("vocab", C.c_int), ("max_pos", C.c_int),
                ("rope_theta", C.c_float), ("rms_eps", C.c_float), ("kv_f16", C.c_int), ("rope_neox", C.c_int)]


class _Tensor(C.Structure):
    _fields_ = [("dtype", C.c_int), ("data", C.c_void_p), ("rows", C.c_int), ("cols", C.c_int)]


class _Layer(C.Structure):
    _fields_ = [(n, _Tensor) for n in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")] + [
        ("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p), ("q_bias", C.c_void_p), ("k_bias", C.c_void_p),
        ("v_bias", C.c_void_p)]


class _Model(C.Structure):
    _fields_ = [("cfg", _Config), ("token_embd", _Tensor), ("output", _Tensor),
                ("output_norm", C.c_void_p), ("layers", C.c_void_p)]


LAYER_MATS = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")


class Model:
    """Oracle forward over host-resident GGUF blocks.

    ``weights`` maps GGUF tensor names (``blk.N.attn_q.weight`` ...,
    ``token_embd.weight``, ``output.weight``, ``output_norm.weight``) to
    ``(dtype, uint8/float32 ndarray, rows, cols)``; norms are float32 arrays.
    Qwen2-style models add ``blk.N.attn_{q,k,v}.bias`` (float32 arrays) and
    ``cfg["rope_neox"] = 1``.
    """

    def __init__(self, cfg: dict, weights: dict):
        self.cfg = dict(cfg)
        self._keep = []
        c = cfg
        self._ccfg = _Config(c["hidden"], c["ffn"], c["n_layers"], c["n_heads"], c["n_kv_heads"], c["vocab"],
                             c["max_pos"], c["rope_theta"], c["rms_eps"], int(c.get("kv_f16", 1)),
                             int(c.get("rope_neox", 0)))

        def tens(name):
            dt, arr, rows, cols = weights[name]
            arr = np.ascontiguousarray(arr)
            self._keep.append(arr)
            return _Tensor(dt, arr.ctypes.data, rows, cols)

        def vec(name):
            arr = np.ascontiguousarray(weights[name], np.float32)
            self._keep.append(arr)
            return arr.ctypes.data

        layers = (_Layer * c["n_layers"])()
        for l in range(c["n_layers"]):
            for m in LAYER_MATS:
                setattr(layers[l], m, tens(f"blk.{l}.{m}.weight"))
            layers[l].attn_norm = vec(f"blk.{l}.attn_norm.weight")
            layers[l].ffn_norm = vec(f"blk.{l}.ffn_norm.weight")
            for b in ("q", "k", "v"):
                if f"blk.{l}.attn_{b}.bias" in weights:
                    setattr(layers[l], f"{b}_bias", vec(f"blk.{l}.attn_{b}.bias"))
        self._layers = layers
        self._m = _Model(self._ccfg, tens("token_embd.weight"), tens("output.weight"), vec("output_norm.weight"),
                         C.cast(layers, C.c_void_p))
        self._state = lib().ifo_state_new(C.byref(self._ccfg))

    def __del__(self):
        try:
            if self._state:
                lib().ifo_state_free(self._state)
                self._state = None
        except Exception:
            pass

    def forward(self, token: int, pos: int, nthreads: int = 0) -> np.ndarray:
        logits = np.empty(self.cfg["vocab"], np.float32)
        if lib().ifo_forward(C.byref(self._m), self._state, token, pos, _p(logits), nthreads) != 0:
            raise ValueError("oracle forward: bad token/pos")
        return logits

    def kv_cache(self, layer: int, which: str) -> np.ndarray:
        c = self.cfg
        kv_dim = c["hidden"] * c["n_kv_heads"] // c["n_heads"]
        ptr = lib().ifo_state_buffer(self._state, 1 if which == "k" else 2, layer)
        dt = np.uint16 if c.get("kv_f16", 1) else np.float32
        n = c["max_pos"] * kv_dim
        buf = (C.c_char * (n * np.dtype(dt).itemsize)).from_address(ptr)
        return np.frombuffer(buf, dt).reshape(c["max_pos"], kv_dim).copy()

    def set_kv_rows(self, layer: int, which: str, rows: np.ndarray) -> None:
        """Writes cache rows 0 .. len(rows)-1 of one layer (uint16 f16 bits or
        float32, as the cache holds), for tests that start decoding late."""
        c = self.cfg
        kv_dim = c["hidden"] * c["n_kv_heads"] // c["n_heads"]
        dt = np.dtype(np.uint16 if c.get("kv_f16", 1) else np.float32)
        rows = np.ascontiguousarray(rows, dt)
        if rows.ndim != 2 or rows.shape[1] != kv_dim or rows.shape[0] > c["max_pos"]:
            raise ValueError("kv rows shape")
        ptr = lib().ifo_state_buffer(self._state, 1 if which == "k" else 2, layer)
        C.memmove(ptr, rows.ctypes.data, rows.nbytes)

    def generate(self, prompt: list[int], n_new: int, nthreads: int = 0, margins: list | None = None) -> list[int]:
        """Greedy token loop of chat_llama2.rs:137-160 with forced prompt tokens.

        Returns the ``n_new`` tokens generated after the prompt.
        """
        out = []
        token = prompt[0]
        for pos in range(len(prompt) + n_new - 1):
            logits = self.forward(token, pos, nthreads)
            nxt = argmax(logits)
            if pos + 1 < len(prompt):
                token = prompt[pos + 1]
            else:
                if margins is not None:
                    top2 = np.partition(logits, -2)[-2:]
                    margins.append(float(top2[1] - top2[0]))
                token = nxt
                out.append(nxt)
        return out
