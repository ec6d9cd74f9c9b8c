"""CPU checks of the C ABI: the library loads, exports every declared symbol, reports errors
through the documented codes, and its host-side helpers match the oracle.  No GPU is used:
entry points that need a device are only called where they must fail cleanly."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from llmplayer_amd import _lib
from llmplayer_amd import hip_forward_pass as hfp
from oracle import oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "llmp_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\bint\s+(llmp_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("llmp_init", "llmp_shutdown", "llmp_kv_create", "llmp_kv_read", "llmp_kv_write",
                 "llmp_rope_upload", "llmp_layer_config", "llmp_attn_decode"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert set(declared_functions()) == set(_lib.SIGNATURES)


def test_error_codes_match_header():
    text = open(HEADER).read()
    codes = dict((name, int(val)) for name, val in
                 re.findall(r"#define\s+(LLMP_ERR_\w+)\s+(\d+)", text))
    assert {v: k for k, v in codes.items()} == _lib.ERR_NAMES


def test_constants_match_header():
    text = open(HEADER).read()
    defs = dict((name, int(val)) for name, val in re.findall(r"#define\s+(LLMP_\w+)\s+(-?\d+)", text))
    for name in ("LLMP_KV_F32", "LLMP_KV_Q8_0", "LLMP_KV_Q8_0_TRUNC", "LLMP_ROPE_NORMAL", "LLMP_ROPE_NEOX",
                 "LLMP_ROPE_SEL_NONE", "LLMP_ROPE_SEL_GLOBAL", "LLMP_ROPE_SEL_LOCAL",
                 "LLMP_NORM_SEQUENTIAL", "LLMP_NORM_V", "LLMP_GGML_F32", "LLMP_GGML_F16",
                 "LLMP_GGML_Q4_0", "LLMP_GGML_Q8_0", "LLMP_GGML_Q4_K", "LLMP_GGML_Q6_K",
                 "LLMP_GGML_BF16", "LLMP_W_ATTN_NORM", "LLMP_W_Q", "LLMP_W_K", "LLMP_W_V",
                 "LLMP_W_QKV", "LLMP_W_O", "LLMP_W_Q_BIAS", "LLMP_W_K_BIAS", "LLMP_W_V_BIAS",
                 "LLMP_W_O_BIAS", "LLMP_W_POST_ATTN_NORM", "LLMP_INPUT_F32", "LLMP_INPUT_Q8_1"):
        assert getattr(_lib, name) == defs[name], name


def test_calls_before_init_fail_with_not_init():
    h = C.c_uint64()
    rc = _lib.status("llmp_kv_create", 1, 16, 1, 64, 0, C.byref(h))
    assert rc == 3  # LLMP_ERR_NOT_INIT
    assert "llmp_init" in _lib.last_error()
    with pytest.raises(_lib.LlmpError) as ei:
        _lib.call("llmp_attn_decode", 1, 0, 0, 1, 1, 1, 1, 0, 0)
    assert ei.value.code == 3 and str(ei.value).startswith("HIP error in llmp_attn_decode: 3")


def test_init_without_device_fails_cleanly():
    rc = _lib.status("llmp_init", 0)
    if rc == 0:  # a gfx950 device is present: nothing to check here
        _lib.call("llmp_shutdown")
        pytest.skip("a GPU is present")
    assert rc == 4  # LLMP_ERR_NO_DEVICE
    assert "device" in _lib.last_error()


@pytest.mark.parametrize("R,S,theta,lin", [(64, 600, 5e5, 1.0), (128, 2048, 1e6, 1.0),
                                           (256, 1024, 1e4, 1.0), (128, 512, 1e4, 8.0)])
def test_rope_table_helper_is_bit_identical_to_oracle(R, S, theta, lin):
    c1, s1 = hfp.rope_table(R, S, theta, lin)
    c2, s2 = orc.rope_tables(R, S, theta, lin)
    assert np.array_equal(c1, c2) and np.array_equal(s1, s2)


def test_rope_table_helper_freq_factors():
    ff = np.linspace(1, 4, 32).astype(np.float32)
    c1, s1 = hfp.rope_table(64, 100, 5e5, 1.0, ff)
    c2, s2 = orc.rope_tables(64, 100, 5e5, 1.0, ff)
    assert np.array_equal(c1, c2) and np.array_equal(s1, s2)


@pytest.mark.parametrize("R,S,theta,sf,L,lm", [(64, 300, 1.5e5, 32.0, 4096, 0.0),
                                              (128, 700, 1e6, 4.0, 32768, 0.0707),
                                              (128, 64, 1e4, 1.0, 4096, 0.1)])
def test_rope_table_yarn_helper_is_bit_identical_to_oracle(R, S, theta, sf, L, lm):
    c1, s1, m1 = hfp.rope_table_yarn(R, S, theta, sf, L, lm)
    c2, s2, m2 = orc.rope_tables_yarn(R, S, theta, sf, L, lm)
    assert np.array_equal(c1, c2) and np.array_equal(s1, s2) and m1 == m2
    ff = np.linspace(1, 4, R // 2).astype(np.float32)
    c1, s1, m1 = hfp.rope_table_yarn(R, S, theta, sf, L, lm, freq_factors=ff)
    c2, s2, m2 = orc.rope_tables_yarn(R, S, theta, sf, L, lm, freq_factors=ff)
    assert np.array_equal(c1, c2) and np.array_equal(s1, s2) and m1 == m2


def test_rope_table_rejects_bad_args():
    out = np.zeros(4, np.float32)
    p = out.ctypes.data_as(C.POINTER(C.c_float))
    assert _lib.status("llmp_rope_table", 3, 1, 1e4, 1.0, None, 0, p, p) == 1


def test_is_supported_for_attention():
    ok = hfp.ModelConfig(24, 8, 128, 28)
    assert hfp.HipForwardPass.isSupportedForAttention(ok)
    assert not hfp.HipForwardPass.isSupportedForAttention(hfp.ModelConfig(24, 8, 128, 28, use_layer_norm=True))
    # groups above the instantiated ones run as several groups per KV head: 9 (36/4) as 3 x 3,
    # 6 at head_dim 96 as 2 x 3, 3 at head_dim 80 as 3 x 1, GLM-4's 16 and 24 as 2 and 3 x 8
    for h, kv, d in ((24, 8, 96), (40, 8, 128), (28, 4, 128), (32, 32, 80), (16, 8, 80),
                     (36, 4, 128), (24, 4, 96), (24, 8, 80), (32, 2, 128), (48, 2, 128)):
        assert hfp.HipForwardPass.isSupportedForAttention(hfp.ModelConfig(h, kv, d, 28)), (h, kv, d)
    for h, kv, d in ((24, 7, 128), (16, 4, 112), (8, 8, 100)):
        assert not hfp.HipForwardPass.isSupportedForAttention(hfp.ModelConfig(h, kv, d, 28)), (h, kv, d)


def test_global_layer_and_rope_type_host_logic_match_oracle():
    for arch, oarch in ((hfp.ARCH_GEMMA2, orc.ARCH_GEMMA2), (hfp.ARCH_GEMMA3, orc.ARCH_GEMMA3),
                        (hfp.ARCH_GPT_OSS, orc.ARCH_GPT_OSS), (hfp.ARCH_COHERE2, orc.ARCH_COHERE2),
                        (hfp.ARCH_LLAMA, orc.ARCH_OTHER)):
        for layer in range(30):
            assert hfp.is_global_layer(arch, layer) == orc.is_global_layer(oarch, layer)
    assert hfp.rope_type_for("llama") == 0 and hfp.rope_type_for("qwen3") == 2
    assert hfp.rope_type_for("gemma3") == 0


def test_prompt_input_takes_fp32_or_bf16_bits_and_rejects_the_rest():
    """Multi-token inputs are either fp32 projections or bf16 bit patterns; anything else
    (float64, int arrays) raises instead of being reinterpreted."""
    a, f32 = hfp.prompt_input(np.zeros((3, 8), np.float32), 8, "q")
    assert f32 and a.shape == (3, 8) and a.dtype == np.float32
    b, f32 = hfp.prompt_input(hfp.to_bf16(np.ones(16, np.float32)), 8, "q")
    assert not f32 and b.shape == (2, 8) and b.dtype == np.uint16
    for bad in (np.zeros(8, np.float64), np.zeros(8, np.int32), np.zeros(8, np.float16)):
        with pytest.raises(TypeError):
            hfp.prompt_input(bad, 8, "q")
    with pytest.raises(ValueError):
        hfp.prompt_input(np.zeros(9, np.float32), 8, "q")
