"""The committed fixtures (tests/golden/*.npz, written by the CPU restatement from seeded inputs
by tests/golden/make_golden.py) replayed through the oracle (CPU) and the HIP path (GPU).

CPU: the oracle reproduces its own fixtures (a regression check of the restatement).
GPU: the HIP path matches them -- output max-abs <= 1e-4, appended K/V rows bit-exact."""
import glob
import os

import numpy as np
import pytest

from llmplayer_amd import hip_forward_pass as hfp
from oracle import oracle as orc
from tests import decode_cases as dc

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(glob.glob(os.path.join(HERE, "*.npz")))
_ARCH = {orc.ARCH_OTHER: hfp.ARCH_LLAMA, orc.ARCH_GEMMA3: hfp.ARCH_GEMMA3}


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _layers(f):
    Hq, Hkv, D, S, pos, rtype, window, arch = (int(x) for x in f["shape"])
    for layer in (int(x) for x in f["layers"]):
        p = f"l{layer}_"
        yield layer, {k[len(p):]: v for k, v in f.items() if k.startswith(p)}


def test_fixtures_present():
    names = {os.path.basename(p) for p in FIXTURES}
    assert {"c1_llama1b_shape.npz", "c2_qwen3_shape.npz", "c3_llama3b_shape.npz",
            "c4_gemma3_shape.npz"} <= names


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_oracle_reproduces_fixture(path):
    f = _load(path)
    Hq, Hkv, D, S, pos, rtype, window, arch = (int(x) for x in f["shape"])
    cfg = orc.OracleConfig(Hq, Hkv, D, S, rope_type=rtype, norm_eps=1e-6, sliding_window=window,
                           arch=arch)
    for layer, d in _layers(f):
        kc = np.zeros((S, Hkv * D), np.float32)
        vc = np.zeros((S, Hkv * D), np.float32)
        kc[:pos], vc[:pos] = d["kc"], d["vc"]
        glob_l = orc.is_global_layer(arch, layer)
        th = 10000.0 if (arch == orc.ARCH_GEMMA3 and window > 0 and not glob_l) else float(f["theta"])
        cs, sn = orc.rope_tables(D, S, th)
        out, q2, k2 = orc.forward_from_projections(cfg, kc, vc, d["q"], d["k"], d["v"], layer, pos,
                                                   qnorm_w=d.get("qnorm_w"), knorm_w=d.get("knorm_w"),
                                                   rope_cos=cs, rope_sin=sn)
        np.testing.assert_allclose(out, d["out"], rtol=0, atol=1e-6)
        assert np.array_equal(k2, d["k_row"]) and np.array_equal(kc[pos], d["k_row"])
        assert np.array_equal(vc[pos], d["v"])


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_hip_path_matches_fixture(path):
    f = _load(path)
    Hq, Hkv, D, S, pos, rtype, window, arch = (int(x) for x in f["shape"])
    layers = [l for l, _ in _layers(f)]
    c = hfp.ModelConfig(Hq, Hkv, D, max(layers) + 1, architecture=_ARCH[arch],
                        rope_freq_base=float(f["theta"]), rope_type=rtype, norm_eps=1e-6,
                        sliding_window=window)
    datas = dict(_layers(f))
    qk = None
    if "qnorm_w" in next(iter(datas.values())):
        ones = (np.ones(D, np.float32), np.ones(D, np.float32))
        qk = [(datas[l]["qnorm_w"], datas[l]["knorm_w"]) if l in datas else ones
              for l in range(max(layers) + 1)]
    with hfp.HipForwardPass(c, S, qk_norm=qk) as fp:
        for layer, d in datas.items():
            dc.log(f"[gpu] golden {os.path.basename(path)} layer {layer}")
            fp.kv.write(layer, 0, d["kc"], d["vc"])
            st = hfp.InferenceState.create(c)
            st.q[:], st.k[:], st.v[:] = d["q"], d["k"], d["v"]
            fp.forwardAttentionOnly(st, layer, pos)
            dc.compare_out(st.xb2, d["out"], f"golden {path} layer {layer}")
            gk, gv = fp.kv.read(layer, 0, pos + 1)
            assert np.array_equal(gk[pos], d["k_row"]) and np.array_equal(gv[pos], d["v"])
            assert np.array_equal(gk[:pos], d["kc"]) and np.array_equal(gv[:pos], d["vc"])
