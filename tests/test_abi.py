"""CPU checks of the drop-in boundary: the C-ABI library loads and exports
every entry point include/inferi_hip.h declares, the Python mirror binds each
of them, and the product package never touches the oracle."""

import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "inferi_hip.h")).read()
    return sorted(set(re.findall(r"IFR_API\s+[\w\s\*]+?\b(ifr_\w+)\s*\(", text)))


def test_header_declares_the_op_api():
    syms = header_symbols()
    for s in ("ifr_create", "ifr_matmul_quant", "ifr_dequant", "ifr_rms_norm", "ifr_rope", "ifr_silu", "ifr_add",
              "ifr_attention", "ifr_argmax", "ifr_llama2_launch", "ifr_llama2_generate"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    import inferi_amd as I

    if not os.path.exists(I.LIB_PATH):
        pytest.skip("libinferi_hip.so not built")
    lib = I.lib()  # binds every signature; raises AttributeError on a missing export
    for s in header_symbols():
        assert hasattr(lib, s), s
    assert sorted(I.SIGNATURES) == header_symbols()


def test_code_object_is_gfx950():
    import inferi_amd as I

    if not os.path.exists(I.HSACO_PATH):
        pytest.skip("code object not built")
    data = open(I.HSACO_PATH, "rb").read()
    assert data[:4] == b"\x7fELF" or data.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
    assert b"gfx950" in data
    for k in (b"gemv_q4_k_qkv", b"gemv_q6_k_head", b"attn_f16_h128_g4", b"embed_k", b"argmax_final_k"):
        assert k in data


def test_create_without_gpu_fails_cleanly():
    import inferi_amd as I

    if not os.path.exists(I.LIB_PATH):
        pytest.skip("libinferi_hip.so not built")
    try:
        import torch  # noqa: F401
    except Exception:
        pass
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    with pytest.raises(I.HipError) as e:
        I.LlmContext(0)
    assert e.value.status == 3


def test_product_never_uses_the_oracle():
    pkg = os.path.join(ROOT, "inferi_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".h", ".hip")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "liboracle" not in text and "oracle.h" not in text, f
