"""Python mirror of inferi's op/model API over the inferi_hip C ABI.

The product is ``libinferi_hip.so`` (C ABI, include/inferi_hip.h) and the
gfx950 code object it loads.  This module binds it with ctypes and keeps the
reference's names and argument order, so a test reads like the reference's:

  LlmContext.rms_norm_assign / matmul_quant_assign / add_assign / rope / silu
      crates/inferi/src/context.rs:336-719
  BatchedMultiqueryAttention.launch
      crates/inferi/src/ops/batched_multiquery_attention.rs:87-110
  Llama2.launch, Llama2State, Llama2Weights
      crates/inferi/src/models/llama2/transformer.rs:46-481

There is no CPU fallback: if the library is missing the import of a Context
raises.  Device memory is owned by ``DeviceBuffer`` objects (ifr_alloc).
"""

from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libinferi_hip.so")
HSACO_PATH = os.path.join(HERE, "inferi_kernels.hsaco")

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 8, 12, 13, 14
Q4_0, Q4_1, Q5_0, Q5_1, Q8_K = 2, 3, 6, 7, 15
BLOCK_ELEMS = {F32: 1, F16: 1, Q4_0: 32, Q4_1: 32, Q5_0: 32, Q5_1: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256,
               Q8_K: 256}
BLOCK_BYTES = {F32: 4, F16: 2, Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210,
               Q8_K: 292}
ROPE_ORIGINAL, ROPE_NEOX = 0, 1

STATUS = {0: "OK", 1: "EINVAL", 2: "EUNSUPPORTED", 3: "EHIP", 4: "ENOMEM"}


class HipError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"inferi_hip {STATUS.get(status, status)}: {msg}")
        self.status = status


class RmsNormConfig(C.Structure):
    _fields_ = [("nudge_factor", C.c_float)]


class RoPEConfig(C.Structure):
    _fields_ = [("head_size", C.c_uint32), ("kv_dim", C.c_uint32), ("pos", C.c_uint32), ("base_freq", C.c_float)]


class AttentionParams(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("seq_len", "kv_dim", "kv_mul", "n_heads", "head_size", "pos")]


class Llama2ConfigC(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("n_layers", "hidden", "ffn", "n_heads", "n_kv_heads", "vocab", "max_pos")] + [
        ("rope_theta", C.c_float), ("rms_eps", C.c_float), ("kv_dtype", C.c_int32), ("rope_variant", C.c_int32)]


class View(C.Structure):
    """ifr_view: element i of an operand at base[offset + i * stride]."""
    _fields_ = [("offset", C.c_int64), ("stride", C.c_int64)]


# Every symbol include/inferi_hip.h declares, with its ctypes signature.
_vp, _i32, _u32, _u64, _sz, _f, _cp = C.c_void_p, C.c_int32, C.c_uint32, C.c_uint64, C.c_size_t, C.c_float, C.c_char_p
SIGNATURES = {
    "ifr_create": (_i32, [_i32, _cp, C.POINTER(_vp)]),
    "ifr_destroy": (None, [_vp]),
    "ifr_last_error": (_cp, [_vp]),
    "ifr_device_info": (_i32, [_vp, _cp, _sz, C.POINTER(_i32)]),
    "ifr_set_option": (_i32, [_vp, _cp, C.c_int64]),
    "ifr_get_option": (_i32, [_vp, _cp, C.POINTER(C.c_int64)]),
    "ifr_alloc": (_i32, [_vp, _sz, C.POINTER(_vp)]),
    "ifr_free": (_i32, [_vp, _vp]),
    "ifr_upload": (_i32, [_vp, _vp, _vp, _sz]),
    "ifr_download": (_i32, [_vp, _vp, _vp, _sz]),
    "ifr_memset": (_i32, [_vp, _vp, _i32, _sz]),
    "ifr_sync": (_i32, [_vp]),
    "ifr_event_record": (_i32, [_vp, _i32]),
    "ifr_event_elapsed": (_i32, [_vp, _i32, _i32, C.POINTER(_f)]),
    "ifr_dequant": (_i32, [_vp, _vp, _vp, _i32, _u64]),
    "ifr_matmul_quant": (_i32, [_vp, _vp, _vp, _i32, _u32, _u32, _vp]),
    "ifr_matmul_quant_noalloc": (_i32, [_vp, _vp, _vp, _i32, _u32, _u32, _vp]),
    "ifr_activation_bytes": (_u64, [_u32]),
    "ifr_quantize_activation": (_i32, [_vp, _vp, _vp, _vp, _u32, _vp]),
    "ifr_matmul_quant_xq": (_i32, [_vp, _vp, _vp, _i32, _u32, _u32, _vp]),
    "ifr_gemm_quant": (_i32, [_vp, _vp, _vp, _i32, _u32, _u32, _vp, _u32, _i32]),
    "ifr_rms_norm": (_i32, [_vp, _vp, _vp, _vp, _vp, _u32]),
    "ifr_add": (_i32, [_vp, _vp, _vp, _u32]),
    "ifr_rope": (_i32, [_vp, _i32, _vp, _vp, _u32, _vp, _u32]),
    "ifr_silu": (_i32, [_vp, _vp, _vp, _u32]),
    "ifr_rms_norm_view": (_i32, [_vp, _vp, _vp, View, _vp, View, _vp, View, _u32]),
    "ifr_add_view": (_i32, [_vp, _vp, View, _vp, View, _u32]),
    "ifr_rope_view": (_i32, [_vp, _i32, _vp, _vp, View, _u32, _vp, View, _u32]),
    "ifr_silu_view": (_i32, [_vp, _vp, View, _vp, View, _u32]),
    "ifr_attention": (_i32, [_vp, C.POINTER(AttentionParams), _vp, _vp, _vp, _vp, _i32, _vp]),
    "ifr_argmax": (_i32, [_vp, _vp, _u32, _vp]),
    "ifr_sample": (_i32, [_vp, _vp, _vp, _u32, _f, _f, _vp, _vp]),
    "ifr_quantize": (_i32, [_vp, _vp, _vp, _i32, _u64]),
    "ifr_fill_normal": (_i32, [_vp, _vp, _u64, _u64, _u64, _f, _f]),
    "ifr_llama2_weights_create": (_i32, [_vp, C.POINTER(Llama2ConfigC), C.POINTER(_vp)]),
    "ifr_llama2_weights_set": (_i32, [_vp, _cp, _i32, _vp, _u32, _u32]),
    "ifr_llama2_weights_destroy": (None, [_vp]),
    "ifr_llama2_state_create": (_i32, [_vp, C.POINTER(Llama2ConfigC), C.POINTER(_vp)]),
    "ifr_llama2_state_destroy": (None, [_vp]),
    "ifr_llama2_state_reset": (_i32, [_vp, _vp, _u32, _u32]),
    "ifr_llama2_launch": (_i32, [_vp, _vp, _vp, _i32]),
    "ifr_llama2_generate": (_i32, [_vp, _vp, _vp, _u32, _i32]),
    "ifr_llama2_prefill": (_i32, [_vp, _vp, _vp, _u32]),
    "ifr_llama2_time_stage": (_i32, [_vp, _vp, _vp, C.c_char_p, _u32, C.POINTER(C.c_float)]),
    "ifr_llama2_set_sampler": (_i32, [_vp, _f, _f, _u64]),
    "ifr_llama2_read_tokens": (_i32, [_vp, _vp, _u32, _u32]),
    "ifr_llama2_state_buffer": (_i32, [_vp, _cp, _i32, C.POINTER(_vp), C.POINTER(_sz)]),
    "ifr_gguf_open": (_i32, [_cp, C.POINTER(_vp)]),
    "ifr_gguf_from_bytes": (_i32, [_vp, _sz, C.POINTER(_vp)]),
    "ifr_gguf_close": (None, [_vp]),
    "ifr_gguf_version": (_u32, [_vp]),
    "ifr_gguf_alignment": (_u32, [_vp]),
    "ifr_gguf_metadata_count": (_u64, [_vp]),
    "ifr_gguf_metadata_key": (_cp, [_vp, _u64]),
    "ifr_gguf_metadata_type": (_i32, [_vp, _cp, C.POINTER(_i32), C.POINTER(_u64)]),
    "ifr_gguf_get_scalar": (_i32, [_vp, _cp, _i32, _vp]),
    "ifr_gguf_get_string": (_i32, [_vp, _cp, C.POINTER(_vp), C.POINTER(_u64)]),
    "ifr_gguf_get_array": (_i32, [_vp, _cp, C.POINTER(_i32), C.POINTER(_u64), C.POINTER(_vp)]),
    "ifr_gguf_get_array_string": (_i32, [_vp, _cp, _u64, C.POINTER(_vp), C.POINTER(_u64)]),
    "ifr_gguf_tensor_count": (_u64, [_vp]),
    "ifr_gguf_tensor_name": (_cp, [_vp, _u64]),
    "ifr_gguf_tensor_info": (_i32, [_vp, _cp, C.POINTER(_i32), C.POINTER(_u64), C.POINTER(_u32), C.POINTER(_vp),
                                    C.POINTER(_u64)]),
    "ifr_gguf_writer_create": (_i32, [C.POINTER(_vp)]),
    "ifr_gguf_writer_destroy": (None, [_vp]),
    "ifr_gguf_writer_set": (_i32, [_vp, _cp, _i32, _vp]),
    "ifr_gguf_writer_set_array": (_i32, [_vp, _cp, _i32, _vp, _u64]),
    "ifr_gguf_writer_add_tensor": (_i32, [_vp, _cp, _i32, _u32, C.POINTER(_u64), _vp, _u64]),
    "ifr_gguf_writer_save": (_i32, [_vp, _cp]),
    "ifr_llama2_config_from_gguf": (_i32, [_vp, C.POINTER(Llama2ConfigC)]),
    "ifr_llama2_weights_from_gguf": (_i32, [_vp, _vp, C.POINTER(Llama2ConfigC), C.POINTER(_vp)]),
}

_lib = None


def lib() -> C.CDLL:
    """Loads libinferi_hip.so (raises if it was not built).  IFR_LIB names
    another build of it (the AddressSanitizer build of inferi_amd/build.py
    build_host_asan)."""
    global _lib
    if _lib is None:
        path = os.environ.get("IFR_LIB") or LIB_PATH
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run `python -c 'import __graft_entry__ as g; g.build()'`")
        L = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def row_bytes(dtype: int, cols: int) -> int:
    return cols // BLOCK_ELEMS[dtype] * BLOCK_BYTES[dtype]


class DeviceBuffer:
    """A device allocation owned by Python (ifr_alloc / ifr_free)."""

    def __init__(self, ctx: "LlmContext", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        ctx._check(lib().ifr_alloc(ctx.h, max(self.nbytes, 1), C.byref(p)))
        self.ptr = p.value

    def free(self) -> None:
        if self.ptr:
            self.ctx._check(lib().ifr_free(self.ctx.h, self.ptr))
            self.ptr = None

    def at(self, byte_offset: int) -> int:
        return self.ptr + int(byte_offset)

    def upload(self, arr: np.ndarray, byte_offset: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        assert byte_offset + a.nbytes <= self.nbytes, "upload past the end of the buffer"
        self.ctx._check(lib().ifr_upload(self.ctx.h, self.at(byte_offset), a.ctypes.data, a.nbytes))
        return self

    def download(self, dtype=np.float32, count: int | None = None, byte_offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        n = (self.nbytes - byte_offset) // dt.itemsize if count is None else int(count)
        out = np.empty(n, dt)
        self.ctx._check(lib().ifr_download(self.ctx.h, out.ctypes.data, self.at(byte_offset), out.nbytes))
        return out


def _ptr(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)


class LlmContext:
    """One device, one stream, one loaded code object (LlmOps + LlmContext,
    crates/inferi/src/context.rs:58-130)."""

    def __init__(self, device: int = 0, code_object: str | None = None):
        h = C.c_void_p()
        st = lib().ifr_create(device, (code_object or HSACO_PATH).encode(), C.byref(h))
        if st != 0:
            raise HipError(st, lib().ifr_last_error(None).decode())
        self.h = h.value

    def close(self) -> None:
        if self.h:
            lib().ifr_destroy(self.h)
            self.h = None

    def _check(self, st: int) -> None:
        if st != 0:
            raise HipError(st, lib().ifr_last_error(self.h).decode())

    # ------------------------------------------------------------ plumbing
    def device_info(self) -> tuple[str, int]:
        buf = C.create_string_buffer(256)
        n = C.c_int32()
        self._check(lib().ifr_device_info(self.h, buf, 256, C.byref(n)))
        return buf.value.decode(), n.value

    def set_option(self, key: str, value: int) -> None:
        self._check(lib().ifr_set_option(self.h, key.encode(), int(value)))

    def get_option(self, key: str) -> int:
        v = C.c_int64()
        self._check(lib().ifr_get_option(self.h, key.encode(), C.byref(v)))
        return v.value

    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def upload(self, arr: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(arr)
        return DeviceBuffer(self, a.nbytes).upload(a)

    def zeros(self, nbytes: int) -> DeviceBuffer:
        b = DeviceBuffer(self, nbytes)
        self._check(lib().ifr_memset(self.h, b.ptr, 0, b.nbytes))
        return b

    def sync(self) -> None:
        self._check(lib().ifr_sync(self.h))

    def event_record(self, slot: int) -> None:
        self._check(lib().ifr_event_record(self.h, slot))

    def event_elapsed(self, a: int, b: int) -> float:
        ms = C.c_float()
        self._check(lib().ifr_event_elapsed(self.h, a, b, C.byref(ms)))
        return ms.value

    # ----------------------------------------------------------------- ops
    def dequant(self, out, blocks, dtype: int, n_elems: int) -> None:
        self._check(lib().ifr_dequant(self.h, _ptr(out), _ptr(blocks), dtype, n_elems))

    def matmul_quant_assign(self, out, a, dtype: int, rows: int, cols: int, b) -> None:
        """out = deq(a)[rows x cols] . b (context.rs:441-456)."""
        self._check(lib().ifr_matmul_quant(self.h, _ptr(out), _ptr(a), dtype, rows, cols, _ptr(b)))

    def matmul_quant_noalloc(self, out, a, dtype: int, rows: int, cols: int, b) -> None:
        """matmul_quant_assign without allocation: the quantized input in the
        device's fixed scratch array (ifr_matmul_quant_noalloc)."""
        self._check(lib().ifr_matmul_quant_noalloc(self.h, _ptr(out), _ptr(a), dtype, rows, cols, _ptr(b)))

    def quantize_activation(self, xq, x, n: int, gamma=None, ss_out=None) -> None:
        """x (times gamma) -> the GEMV's quantized activation layout."""
        self._check(lib().ifr_quantize_activation(self.h, _ptr(xq), _ptr(x), _ptr(gamma), n, _ptr(ss_out)))

    def matmul_quant_xq(self, out, a, dtype: int, rows: int, cols: int, xq) -> None:
        self._check(lib().ifr_matmul_quant_xq(self.h, _ptr(out), _ptr(a), dtype, rows, cols, _ptr(xq)))

    def gemm_quant(self, y, w, dtype: int, rows: int, cols: int, x_f16, m: int, accumulate: bool = False) -> None:
        """y[m][rows] (+)= x_f16[m][cols] . dequant(W)^T on the matrix cores."""
        self._check(lib().ifr_gemm_quant(self.h, _ptr(y), _ptr(w), dtype, rows, cols, _ptr(x_f16), m, int(accumulate)))

    @staticmethod
    def activation_bytes(n: int) -> int:
        return int(lib().ifr_activation_bytes(n))

    def rms_norm_assign(self, config, out, value, weight, n: int) -> None:
        """config: device RmsNormConfig (context.rs:336-353)."""
        self._check(lib().ifr_rms_norm(self.h, _ptr(config), _ptr(out), _ptr(value), _ptr(weight), n))

    def add_assign(self, in_out_a, b, n: int) -> None:
        self._check(lib().ifr_add(self.h, _ptr(in_out_a), _ptr(b), n))

    def rope(self, variant: int, config, in_out_q, q_len: int, in_out_k, k_len: int) -> None:
        """config: device RoPEConfig (context.rs:687-704)."""
        self._check(lib().ifr_rope(self.h, variant, _ptr(config), _ptr(in_out_q), q_len, _ptr(in_out_k), k_len))

    def silu(self, in_out_h1, in_h2, n: int) -> None:
        self._check(lib().ifr_silu(self.h, _ptr(in_out_h1), _ptr(in_h2), n))

    # strided views (offset, stride) in elements, as the reference ops take tensor layouts
    def rms_norm_view(self, config, out, ov, value, vv, weight, wv, n: int) -> None:
        self._check(lib().ifr_rms_norm_view(self.h, _ptr(config), _ptr(out), View(*ov), _ptr(value), View(*vv),
                                            _ptr(weight), View(*wv), n))

    def add_view(self, in_out_a, av, b, bv, n: int) -> None:
        self._check(lib().ifr_add_view(self.h, _ptr(in_out_a), View(*av), _ptr(b), View(*bv), n))

    def rope_view(self, variant: int, config, q, qv, q_len: int, k, kv, k_len: int) -> None:
        self._check(lib().ifr_rope_view(self.h, variant, _ptr(config), _ptr(q), View(*qv), q_len, _ptr(k), View(*kv),
                                        k_len))

    def silu_view(self, h1, av, h2, bv, n: int) -> None:
        self._check(lib().ifr_silu_view(self.h, _ptr(h1), View(*av), _ptr(h2), View(*bv), n))

    def argmax(self, v, n: int, out_index) -> None:
        self._check(lib().ifr_argmax(self.h, _ptr(v), n, _ptr(out_index)))

    def sample(self, logits, probs, n: int, temperature: float, topp: float, coin, out_index) -> None:
        """Sampler::sample (models/sampler.rs:32-52) with a device coin;
        probs may be logits itself."""
        self._check(lib().ifr_sample(self.h, _ptr(logits), _ptr(probs), n, temperature, topp, _ptr(coin),
                                     _ptr(out_index)))

    def quantize(self, out, x, dtype: int, n_elems: int) -> None:
        self._check(lib().ifr_quantize(self.h, _ptr(out), _ptr(x), dtype, n_elems))

    def fill_normal(self, out, n: int, seed: int, stream: int, mean: float, std: float) -> None:
        self._check(lib().ifr_fill_normal(self.h, _ptr(out), n, seed, stream, mean, std))


class BatchedMultiqueryAttention:
    """crates/inferi/src/ops/batched_multiquery_attention.rs:87-110."""

    @staticmethod
    def launch(ctxt: LlmContext, params: AttentionParams, params_gpu, q, key_cache, value_cache, kv_dtype: int, xb) -> None:
        ctxt._check(lib().ifr_attention(ctxt.h, C.byref(params), _ptr(params_gpu), _ptr(q), _ptr(key_cache),
                                        _ptr(value_cache), kv_dtype, _ptr(xb)))


# ---------------------------------------------------------------- model --

@dataclass
class Llama2Config:
    """Llama2Config (crates/inferi/src/models/llama2/cpu.rs:78-141)."""

    n_layers: int
    hidden: int
    ffn: int
    n_heads: int
    n_kv_heads: int
    vocab: int
    max_pos: int
    rope_theta: float = 10000.0
    rms_eps: float = 1e-6
    kv_dtype: int = F16
    rope_variant: int = ROPE_ORIGINAL

    @property
    def head_size(self) -> int:
        return self.hidden // self.n_heads

    @property
    def kv_dim(self) -> int:
        return self.head_size * self.n_kv_heads

    def c(self) -> Llama2ConfigC:
        return Llama2ConfigC(self.n_layers, self.hidden, self.ffn, self.n_heads, self.n_kv_heads, self.vocab,
                             self.max_pos, self.rope_theta, self.rms_eps, self.kv_dtype, self.rope_variant)

    @classmethod
    def from_gguf(cls, gguf: "Gguf") -> "Llama2Config":
        """Llama2Config::from_gguf (cpu.rs:74-107); kv_dtype F32 as the reference."""
        c = Llama2ConfigC()
        _free_check(lib().ifr_llama2_config_from_gguf(gguf.h, C.byref(c)))
        return cls(n_layers=c.n_layers, hidden=c.hidden, ffn=c.ffn, n_heads=c.n_heads, n_kv_heads=c.n_kv_heads,
                   vocab=c.vocab, max_pos=c.max_pos, rope_theta=c.rope_theta, rms_eps=c.rms_eps, kv_dtype=c.kv_dtype,
                   rope_variant=c.rope_variant)

    def gguf_metadata(self, arch: str = "llama") -> list:
        """(key, type, value) of the <arch>.* keys from_gguf reads."""
        m = arch
        return [(f"{m}.embedding_length", GGUF_U32, self.hidden), (f"{m}.feed_forward_length", GGUF_U32, self.ffn),
                (f"{m}.block_count", GGUF_U32, self.n_layers), (f"{m}.attention.head_count", GGUF_U32, self.n_heads),
                (f"{m}.attention.head_count_kv", GGUF_U32, self.n_kv_heads),
                (f"{m}.context_length", GGUF_U32, self.max_pos), (f"{m}.rope.freq_base", GGUF_F32, self.rope_theta),
                (f"{m}.attention.layer_norm_rms_epsilon", GGUF_F32, self.rms_eps)]

    def shapes(self, bias: bool = False) -> dict:
        """GGUF tensor name -> (rows, cols) (transformer.rs:294-393); bias adds
        Qwen2's blk.N.attn_{q,k,v}.bias vectors."""
        h, kv, f = self.hidden, self.kv_dim, self.ffn
        s = {"token_embd.weight": (self.vocab, h), "output.weight": (self.vocab, h), "output_norm.weight": (1, h)}
        for l in range(self.n_layers):
            s.update({f"blk.{l}.attn_norm.weight": (1, h), f"blk.{l}.ffn_norm.weight": (1, h),
                      f"blk.{l}.attn_q.weight": (h, h), f"blk.{l}.attn_k.weight": (kv, h),
                      f"blk.{l}.attn_v.weight": (kv, h), f"blk.{l}.attn_output.weight": (h, h),
                      f"blk.{l}.ffn_gate.weight": (f, h), f"blk.{l}.ffn_up.weight": (f, h),
                      f"blk.{l}.ffn_down.weight": (h, f)})
            if bias:
                s.update({f"blk.{l}.attn_q.bias": (1, h), f"blk.{l}.attn_k.bias": (1, kv),
                          f"blk.{l}.attn_v.bias": (1, kv)})
        return s


class Llama2Weights:
    """Table of device tensors keyed by GGUF name; the buffers stay owned by
    this object (transformer.rs:176-196)."""

    def __init__(self, ctxt: LlmContext, config: Llama2Config):
        self.ctx = ctxt
        self.config = config
        self._cfg = config.c()
        h = C.c_void_p()
        ctxt._check(lib().ifr_llama2_weights_create(ctxt.h, C.byref(self._cfg), C.byref(h)))
        self.h = h.value
        self.buffers: dict[str, tuple[int, DeviceBuffer, int, int]] = {}

    def set(self, name: str, dtype: int, buf: DeviceBuffer, rows: int, cols: int) -> None:
        self.ctx._check(lib().ifr_llama2_weights_set(self.h, name.encode(), dtype, buf.ptr, rows, cols))
        self.buffers[name] = (dtype, buf, rows, cols)

    def set_host(self, name: str, dtype: int, data: np.ndarray, rows: int, cols: int) -> None:
        self.set(name, dtype, self.ctx.upload(np.ascontiguousarray(data)), rows, cols)

    def download(self, name: str) -> tuple[int, np.ndarray, int, int]:
        dtype, buf, rows, cols = self.buffers[name]
        if dtype == F32:
            return dtype, buf.download(np.float32, rows * cols), rows, cols
        return dtype, buf.download(np.uint8, rows * row_bytes(dtype, cols)), rows, cols

    def close(self) -> None:
        if self.h:
            lib().ifr_llama2_weights_destroy(self.h)
            self.h = None
        for _, b, _, _ in self.buffers.values():
            b.free()
        self.buffers.clear()

    @classmethod
    def from_gguf(cls, ctxt: LlmContext, gguf: "Gguf", config: Llama2Config) -> "Llama2Weights":
        """Llama2Weights::from_gguf (transformer.rs:294-393): the tensors are
        copied to device memory owned by the weights."""
        w = cls.__new__(cls)
        w.ctx, w.config, w._cfg, w.buffers = ctxt, config, config.c(), {}
        h = C.c_void_p()
        ctxt._check(lib().ifr_llama2_weights_from_gguf(ctxt.h, gguf.h, C.byref(w._cfg), C.byref(h)))
        w.h = h.value
        return w

    def to_gguf(self, path: str, tokens: list | None = None, architecture: str | None = None) -> None:
        """Writes the model as a GGUF file that from_gguf (here and in the
        reference) reads: general.architecture, the llama.* keys, a
        tokenizer.ggml.tokens list of vocab length, and every tensor's blocks."""
        if architecture is None:
            architecture = "qwen2" if self.config.rope_variant == ROPE_NEOX else "llama"
        wr = GgufWriter()
        try:
            wr.set("general.architecture", GGUF_STRING, architecture)
            wr.set("tokenizer.ggml.model", GGUF_STRING, "llama")
            for key, ty, val in self.config.gguf_metadata(architecture):
                wr.set(key, ty, val)
            toks = tokens if tokens is not None else [f"<t{i}>" for i in range(self.config.vocab)]
            wr.set_array("tokenizer.ggml.tokens", GGUF_STRING, toks)
            for name in self.buffers:
                dtype, arr, rows, cols = self.download(name)
                dims = [cols] if rows == 1 and name.endswith(("norm.weight", ".bias")) else [rows, cols]
                wr.add_tensor(name, dtype, dims, arr)
            wr.save(path)
        finally:
            wr.close()

    @classmethod
    def synthetic(cls, ctxt: LlmContext, config: Llama2Config, seed: int, mat_dtype: int = Q4_K,
                  head_dtype: int = Q6_K, embd_dtype: int = Q4_K, std: float = 0.02, norm_mean: float = 1.0,
                  norm_std: float = 0.1, qkv_bias: bool = False, bias_std: float = 0.5,
                  overrides: dict | None = None) -> "Llama2Weights":
        """Random-init model made on the device: every matrix ~ N(0, std)
        quantized with the GGUF quantizer, norms ~ N(norm_mean, norm_std) in
        F32, and with qkv_bias Qwen2's QKV biases ~ N(0, bias_std) in F32.
        ``overrides`` maps a tensor name ("blk.3.attn_v.weight") or a matrix
        kind ("attn_v", "ffn_down") to another GGUF type, as mixed files
        (Q4_K_M) store some matrices.  Tensor i (in
        ``config.shapes(qkv_bias)`` order) uses generator stream i."""
        w = cls(ctxt, config)
        shapes = config.shapes(qkv_bias)
        biggest = max(r * c for r, c in shapes.values())
        tmp = ctxt.alloc(biggest * 4)
        try:
            for i, (name, (rows, cols)) in enumerate(shapes.items()):
                n = rows * cols
                if name.endswith(("norm.weight", ".bias")):
                    buf = ctxt.alloc(n * 4)
                    bias = name.endswith(".bias")
                    ctxt.fill_normal(buf, n, seed, i, 0.0 if bias else norm_mean, bias_std if bias else norm_std)
                    w.set(name, F32, buf, rows, cols)
                    continue
                dt = head_dtype if name == "output.weight" else embd_dtype if name == "token_embd.weight" else mat_dtype
                if overrides:
                    parts = name.split(".")
                    kind = parts[2] if len(parts) == 4 and parts[0] == "blk" else None
                    dt = overrides.get(name, overrides.get(kind, dt))
                ctxt.fill_normal(tmp, n, seed, i, 0.0, std)
                buf = ctxt.alloc(rows * row_bytes(dt, cols))
                ctxt.quantize(buf, tmp, dt, n)
                w.set(name, dt, buf, rows, cols)
            ctxt.sync()
        finally:
            tmp.free()
        return w


class Llama2State:
    """Activations, logits, KV cache, device position and token sequence
    (transformer.rs:46-137)."""

    def __init__(self, ctxt: LlmContext, config: Llama2Config):
        self.ctx = ctxt
        self.config = config
        self._cfg = config.c()
        h = C.c_void_p()
        ctxt._check(lib().ifr_llama2_state_create(ctxt.h, C.byref(self._cfg), C.byref(h)))
        self.h = h.value

    def close(self) -> None:
        if self.h:
            lib().ifr_llama2_state_destroy(self.h)
            self.h = None

    def reset(self, prompt, pos: int = 0) -> None:
        p = np.ascontiguousarray(np.asarray(prompt, np.uint32))
        self.ctx._check(lib().ifr_llama2_state_reset(self.h, p.ctypes.data if p.size else None, p.size, pos))

    def buffer(self, name: str, layer: int = 0) -> tuple[int, int]:
        p = C.c_void_p()
        n = C.c_size_t()
        self.ctx._check(lib().ifr_llama2_state_buffer(self.h, name.encode(), layer, C.byref(p), C.byref(n)))
        return p.value, n.value

    def read(self, name: str, dtype=np.float32, layer: int = 0) -> np.ndarray:
        p, n = self.buffer(name, layer)
        dt = np.dtype(dtype)
        out = np.empty(n // dt.itemsize, dt)
        self.ctx._check(lib().ifr_download(self.ctx.h, out.ctypes.data, p, out.nbytes))
        return out

    def set_sampler(self, temperature: float, topp: float = 0.0, seed: int = 0) -> None:
        """Decode steps sample instead of taking the argmax (temperature 0
        restores it); sample_next_token uses temperature 0.7, topp 0.95."""
        self.ctx._check(lib().ifr_llama2_set_sampler(self.h, temperature, topp, seed))

    def tokens(self, start: int, n: int) -> np.ndarray:
        out = np.empty(n, np.uint32)
        self.ctx._check(lib().ifr_llama2_read_tokens(self.h, out.ctypes.data, start, n))
        return out


class Llama2:
    """Llama2::launch (transformer.rs:409-481) with the device-side token loop
    of ChatLlama2::forward_logits (chat_llama2.rs:191-255)."""

    @staticmethod
    def launch(ctxt: LlmContext, state: Llama2State, weights: Llama2Weights, fused: bool = True) -> None:
        ctxt._check(lib().ifr_llama2_launch(ctxt.h, state.h, weights.h, int(fused)))

    @staticmethod
    def prefill(ctxt: LlmContext, state: Llama2State, weights: Llama2Weights, n_tokens: int) -> None:
        """The next n_tokens forced prompt tokens through the batched (matrix-core) path."""
        ctxt._check(lib().ifr_llama2_prefill(ctxt.h, state.h, weights.h, n_tokens))

    @staticmethod
    def generate(ctxt: LlmContext, state: Llama2State, weights: Llama2Weights, n_steps: int,
                 use_graph: bool = True) -> None:
        ctxt._check(lib().ifr_llama2_generate(ctxt.h, state.h, weights.h, n_steps, int(use_graph)))

    @staticmethod
    def time_stage(ctxt: LlmContext, state: Llama2State, weights: Llama2Weights, stage: str, iters: int) -> float:
        """Microseconds per layer of one fused decode stage ("qkv", "attention",
        "attn_output", "ffn_gate_up", "ffn_down"), every layer in turn, `iters`
        times (ifr_llama2_time_stage; overwrites the state's activations)."""
        us = C.c_float()
        ctxt._check(lib().ifr_llama2_time_stage(ctxt.h, state.h, weights.h, stage.encode(), iters, C.byref(us)))
        return float(us.value)


# ------------------------------------------------------------------- GGUF
# Metadata value types (gguf.rs MetadataValueType).
GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32, GGUF_BOOL, GGUF_STRING, GGUF_ARRAY, \
    GGUF_U64, GGUF_I64, GGUF_F64 = range(13)
_GGUF_NP = {GGUF_U8: np.uint8, GGUF_I8: np.int8, GGUF_U16: np.uint16, GGUF_I16: np.int16, GGUF_U32: np.uint32,
            GGUF_I32: np.int32, GGUF_F32: np.float32, GGUF_BOOL: np.uint8, GGUF_U64: np.uint64, GGUF_I64: np.int64,
            GGUF_F64: np.float64}


def _free_check(st: int) -> None:
    if st != 0:
        raise HipError(st, (lib().ifr_last_error(None) or b"").decode())


class GgufTensor:
    """GgufTensor (gguf.rs:336-349): dims in [rows, cols, ...] order."""

    def __init__(self, dtype: int, dims: tuple, rank: int, data: np.ndarray | None):
        self.dtype, self.dims, self.rank, self.data = dtype, dims, rank, data


class Gguf:
    """Gguf::from_bytes (gguf.rs:516-692) through ifr_gguf_open /
    ifr_gguf_from_bytes: version, metadata and tensors."""

    def __init__(self, path: str | None = None, data: bytes | None = None):
        self.h = None
        h = C.c_void_p()
        if path is not None:
            _free_check(lib().ifr_gguf_open(os.fsencode(path), C.byref(h)))
        else:
            buf = C.create_string_buffer(bytes(data), len(data))
            _free_check(lib().ifr_gguf_from_bytes(buf, len(data), C.byref(h)))
        self.h = h.value

    def close(self) -> None:
        if self.h:
            lib().ifr_gguf_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    @property
    def version(self) -> int:
        return lib().ifr_gguf_version(self.h)

    @property
    def alignment(self) -> int:
        return lib().ifr_gguf_alignment(self.h)

    def keys(self) -> list:
        return [lib().ifr_gguf_metadata_key(self.h, i).decode() for i in range(lib().ifr_gguf_metadata_count(self.h))]

    def type_of(self, key: str) -> tuple[int, int, int]:
        et, n = C.c_int32(), C.c_uint64()
        t = lib().ifr_gguf_metadata_type(self.h, key.encode(), C.byref(et), C.byref(n))
        return t, et.value, n.value

    def get(self, key: str):
        """The value as Python data: int / float / bool / str, a numpy array
        or list of str for arrays (None for an array of arrays)."""
        t, et, n = self.type_of(key)
        k = key.encode()
        if t < 0:
            raise KeyError(key)
        if t == GGUF_STRING:
            p, ln = C.c_void_p(), C.c_uint64()
            _free_check(lib().ifr_gguf_get_string(self.h, k, C.byref(p), C.byref(ln)))
            return C.string_at(p.value, ln.value).decode("utf-8", "replace")
        if t == GGUF_ARRAY:
            if et == GGUF_STRING:
                out = []
                for i in range(n):
                    p, ln = C.c_void_p(), C.c_uint64()
                    _free_check(lib().ifr_gguf_get_array_string(self.h, k, i, C.byref(p), C.byref(ln)))
                    out.append(C.string_at(p.value, ln.value).decode("utf-8", "replace"))
                return out
            if et not in _GGUF_NP:
                return None
            p = C.c_void_p()
            _free_check(lib().ifr_gguf_get_array(self.h, k, None, None, C.byref(p)))
            dt = np.dtype(_GGUF_NP[et]).newbyteorder("<")
            a = np.frombuffer(C.string_at(p.value, n * dt.itemsize), dt).copy() if n else np.zeros(0, dt)
            return a.astype(bool) if et == GGUF_BOOL else a
        raw = (C.c_uint8 * 8)()
        _free_check(lib().ifr_gguf_get_scalar(self.h, k, t, raw))
        v = np.frombuffer(bytes(raw), np.dtype(_GGUF_NP[t]).newbyteorder("<"), 1)[0]
        if t == GGUF_BOOL:
            return bool(v)
        return float(v) if t in (GGUF_F32, GGUF_F64) else int(v)

    @property
    def metadata(self) -> dict:
        return {k: self.get(k) for k in self.keys()}

    def tensor_names(self) -> list:
        return [lib().ifr_gguf_tensor_name(self.h, i).decode() for i in range(lib().ifr_gguf_tensor_count(self.h))]

    def tensor(self, name: str) -> GgufTensor:
        dt, rank, p, nb = C.c_int32(), C.c_uint32(), C.c_void_p(), C.c_uint64()
        dims = (C.c_uint64 * 4)()
        _free_check(lib().ifr_gguf_tensor_info(self.h, name.encode(), C.byref(dt), dims, C.byref(rank), C.byref(p),
                                               C.byref(nb)))
        data = np.frombuffer(C.string_at(p.value, nb.value), np.uint8).copy() if p.value else None
        return GgufTensor(dt.value, tuple(int(d) for d in dims), rank.value, data)

    @property
    def tensors(self) -> dict:
        return {n: self.tensor(n) for n in self.tensor_names()}


class GgufWriter:
    """ifr_gguf_writer: metadata and tensors written in insertion order."""

    def __init__(self):
        self.h = None
        h = C.c_void_p()
        _free_check(lib().ifr_gguf_writer_create(C.byref(h)))
        self.h = h.value

    def close(self) -> None:
        if self.h:
            lib().ifr_gguf_writer_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def set(self, key: str, type_: int, value) -> None:
        if type_ == GGUF_STRING:
            v = C.create_string_buffer(value.encode())
        else:
            v = C.create_string_buffer(np.array([value], _GGUF_NP[type_]).astype(np.dtype(_GGUF_NP[type_]).newbyteorder("<")).tobytes(), 8)
        _free_check(lib().ifr_gguf_writer_set(self.h, key.encode(), type_, v))

    def set_array(self, key: str, elem_type: int, values) -> None:
        if elem_type == GGUF_STRING:
            enc = [str(x).encode() for x in values]
            arr = (C.c_char_p * max(len(enc), 1))(*enc)
            _free_check(lib().ifr_gguf_writer_set_array(self.h, key.encode(), elem_type, arr, len(enc)))
        else:
            a = np.ascontiguousarray(np.asarray(values, _GGUF_NP[elem_type]).astype(
                np.dtype(_GGUF_NP[elem_type]).newbyteorder("<")))
            _free_check(lib().ifr_gguf_writer_set_array(self.h, key.encode(), elem_type,
                                                        a.ctypes.data if a.size else None, a.size))

    def add_tensor(self, name: str, dtype: int, dims, data) -> None:
        b = np.ascontiguousarray(np.asarray(data)).view(np.uint8).reshape(-1)
        d = (C.c_uint64 * max(4, len(dims)))(*[int(x) for x in dims], *([1] * (4 - len(dims))))
        _free_check(lib().ifr_gguf_writer_add_tensor(self.h, name.encode(), dtype, len(dims), d,
                                                     b.ctypes.data if b.size else None, b.size))

    def save(self, path: str) -> None:
        _free_check(lib().ifr_gguf_writer_save(self.h, os.fsencode(path)))
