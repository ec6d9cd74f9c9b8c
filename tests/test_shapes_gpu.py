"""GPU parity of the head shapes beyond the BASELINE configs, as the reference GPU's
attention_full runs any headSize and kvMul (attention.cu:10-34): GQA groups 5 and 7
(Qwen2.5-7B 28/4, 40/8), groups 16 and 24 (GLM-4's 32 and 48 query heads over 2 KV heads,
README.md:566, which run as 2 and 3 groups of 8 per cached KV head), head_dim 96 (Phi-3-mini,
32/32, NEOX) and head_dim 80 (Phi-2, 32/32, NEOX over 32 of the 80 dims).  Decode against the
oracle at fp32 (and Q8_0 for the groups), multi-token attention on fp32 projections, and the
K-token attention half (at head_dim 80 its tokens run one by one: that head size has no prefill
kernel).

Bar: output max-abs <= 1e-4 (and <= 1e-4 + 1e-3*|ref|); every cache row bit-identical to the
oracle's."""
import numpy as np
import pytest

from llmplayer_amd import _lib
from llmplayer_amd import hip_forward_pass as hfp
from tests import decode_cases as dc
from tests.test_prefill_f32_gpu import run_f32_case

pytestmark = pytest.mark.gpu

SHAPES = {
    "qwen2.5-7b_28-4-128": dict(h=28, kv=4, d=128, arch="qwen2", theta=1e6),
    "40-8-128": dict(h=40, kv=8, d=128, arch=hfp.ARCH_LLAMA, theta=5e5),
    "20-4-64": dict(h=20, kv=4, d=64, arch=hfp.ARCH_LLAMA, theta=5e5),
    "14-2-64": dict(h=14, kv=2, d=64, arch=hfp.ARCH_LLAMA, theta=5e5),
    "10-2-256": dict(h=10, kv=2, d=256, arch=hfp.ARCH_LLAMA, theta=1e4),
    "phi3-mini_32-32-96": dict(h=32, kv=32, d=96, arch="phi3", theta=1e4),
    "24-8-96": dict(h=24, kv=8, d=96, arch=hfp.ARCH_LLAMA, theta=1e4),
    "phi2_32-32-80": dict(h=32, kv=32, d=80, arch="phi3", theta=1e4, rope_dim=32),
    "16-8-80": dict(h=16, kv=8, d=80, arch=hfp.ARCH_LLAMA, theta=1e4),
    "glm4_32-2-128": dict(h=32, kv=2, d=128, arch=hfp.ARCH_LLAMA, theta=1e4),
    "48-2-128": dict(h=48, kv=2, d=128, arch=hfp.ARCH_LLAMA, theta=1e4),
    "36-4-64": dict(h=36, kv=4, d=64, arch=hfp.ARCH_LLAMA, theta=5e5),
}


def _config(name, layers=1):
    s = SHAPES[name]
    return hfp.ModelConfig(s["h"], s["kv"], s["d"], layers, architecture=s["arch"],
                           rope_freq_base=s["theta"], rope_dim_count=s.get("rope_dim", 0))


@pytest.mark.parametrize("splits", [0, 1, 7, 400])
@pytest.mark.parametrize("name", list(SHAPES))
def test_decode_new_shapes(name, splits):
    # 400 splits (334 effective at 1000 rows) run the combine over 2-8 column workgroups per
    # head, including 5 and 6 float4 columns per workgroup (head_dim 80 and 96)
    c = _config(name)
    assert hfp.HipForwardPass.isSupportedForAttention(c)
    pos = 999
    d = dc.make_layer(c, 1024, pos, seed=sum(map(ord, name)) + splits)
    with hfp.HipForwardPass(c, 1024) as fp:
        dc.log(f"[gpu] decode {name} pos {pos} splits {splits}")
        fp.kv.write(0, 0, d.kc, d.vc)
        st = hfp.InferenceState.create(c)
        st.q[:], st.k[:], st.v[:] = d.q, d.k, d.v
        fp.forwardAttentionOnly(st, 0, pos, splits)
        want, kc, vc = dc.oracle_call(c, 1024, d, 0, pos, n_threads=16)
        dc.compare_out(st.xb2, want, f"decode {name} splits {splits}")
        dc.compare_cache(fp, 0, kc, vc, f"decode {name} cache", rows=(0, pos + 1))


@pytest.mark.parametrize("name", ["qwen2.5-7b_28-4-128", "40-8-128", "14-2-64", "10-2-256",
                                  "glm4_32-2-128", "48-2-128", "36-4-64"])
@pytest.mark.parametrize("mode", [_lib.LLMP_KV_Q8_0, _lib.LLMP_KV_Q8_0_TRUNC], ids=["round", "trunc"])
def test_decode_groups_5_7_q8_0(name, mode):
    from oracle import oracle as orc
    c = _config(name)
    omode = orc.Q8_SCALAR if mode == _lib.LLMP_KV_Q8_0 else orc.Q8_SIMD8
    pos = 700
    d = dc.make_layer_q8(c, 1024, pos, seed=77, mode=omode)
    with hfp.HipForwardPass(c, 1024, kv_dtype=mode) as fp:
        dc.log(f"[gpu] Q8_0 decode {name} mode {mode} pos {pos}")
        fp.kv.write_q8(0, 0, d.kq, d.ks, d.vq, d.vs)
        st = hfp.InferenceState.create(c)
        st.q[:], st.k[:], st.v[:] = d.q, d.k, d.v
        fp.forwardAttentionOnly(st, 0, pos)
        want, cache = dc.oracle_call_q8(c, 1024, d, 0, pos, n_threads=16, mode=omode)
        dc.compare_out(st.xb2, want, f"Q8_0 decode {name}")
        dc.compare_cache_q8(fp, 0, cache, f"Q8_0 decode {name} cache", rows=(0, pos + 1))


@pytest.mark.parametrize("name,pos0,P", [("qwen2.5-7b_28-4-128", 100, 70), ("40-8-128", 0, 130),
                                         ("14-2-64", 3000, 4), ("10-2-256", 40, 33),
                                         ("phi3-mini_32-32-96", 50, 90), ("24-8-96", 2000, 16),
                                         ("glm4_32-2-128", 200, 40), ("48-2-128", 3000, 16),
                                         ("36-4-64", 0, 300)])
def test_prefill_f32_new_shapes(name, pos0, P):
    """Multi-token attention on fp32 projections (the split-K path for the short chunks after a
    long prefix), followed by decode steps."""
    c = _config(name)
    run_f32_case(c, pos0 + P + 8, 0, pos0, P, seed=len(name) + P, decode_steps=8,
                 what=f"prefill {name} pos0 {pos0} P {P}")


def test_head_dim_80_has_no_prefill_kernel():
    c = _config("phi2_32-32-80")
    rng = np.random.default_rng(3)
    with hfp.HipForwardPass(c, 64) as fp:
        q = rng.standard_normal((4, c.q_dim), dtype=np.float32)
        k = rng.standard_normal((4, c.kv_dim), dtype=np.float32)
        with pytest.raises(hfp.LlmpError):
            fp.prefill(0, 0, q, k, k)


def test_unsupported_shapes_are_rejected():
    for h, kv, d in ((16, 16, 112), (8, 8, 100), (12, 5, 128)):
        c = hfp.ModelConfig(h, kv, d, 1)
        assert not hfp.HipForwardPass.isSupportedForAttention(c), (h, kv, d)
    # groups beyond the instantiated ones run as several groups per KV head (group 9 at head_dim
    # 64 as 3 of 3, 6 at head_dim 96 as 2 of 3, 6 at head_dim 80 as 3 of 2)
    for h, kv, d in ((18, 2, 64), (30, 5, 96), (24, 4, 80), (32, 2, 128)):
        assert hfp.HipForwardPass.isSupportedForAttention(hfp.ModelConfig(h, kv, d, 1)), (h, kv, d)
    with hfp.HipForwardPass(hfp.ModelConfig(16, 16, 128, 1), 64) as fp:
        h = fp.kv.handle
        assert _lib.status("llmp_layer_config", h, 0, 16, 16, 112, 0, 0, 0, 1, 0.0, 0.0, 1e-6,
                           None, None) != 0


@pytest.mark.parametrize("name,dim", [("qwen2.5-7b_28-4-128", 3584), ("phi3-mini_32-32-96", 3072),
                                      ("phi2_32-32-80", 2560), ("glm4_32-2-128", 4096)])
def test_block_batch_new_shapes(name, dim):
    """The K-token attention half: 12 tokens after a 60-row prefix (head_dim 80 runs its tokens
    one by one through the decode kernel)."""
    from tests.test_block_batch_gpu import _run_batch
    from tests import ggml_pack as gp
    c = _config(name)
    _run_batch(c, dim, 128, 60, 12, (gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K),
               seed=len(name) + dim, what=f"{name} dim {dim}")
