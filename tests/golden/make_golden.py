"""Writes the small decode-attention fixtures in this directory.

The reference ships no golden vectors for this path and its Java cannot run here, so these
fixtures are produced by the CPU restatement (oracle/attn_oracle.c) on seeded inputs.  They
are regression vectors for the restatement and the HIP path, not outputs of the reference.
Run:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as orc  # noqa: E402

CASES = {
    # name: (Hq, Hkv, D, max_seq, pos, rope_type, theta, qk_norm, window, arch, layers)
    "c1_llama1b_shape": (32, 8, 64, 40, 39, 0, 500000.0, False, 0, orc.ARCH_OTHER, (0,)),
    "c2_qwen3_shape": (16, 8, 128, 24, 23, 2, 1e6, True, 0, orc.ARCH_OTHER, (0,)),
    "c3_llama3b_shape": (24, 8, 128, 24, 23, 0, 500000.0, False, 0, orc.ARCH_OTHER, (0,)),
    "c4_gemma3_shape": (4, 1, 256, 48, 40, 0, 1e6, True, 16, orc.ARCH_GEMMA3, (0, 5)),
}


def make(name, spec, seed):
    Hq, Hkv, D, S, pos, rtype, theta, qkn, window, arch, layers = spec
    rng = np.random.default_rng(seed)
    kv = Hkv * D
    cfg = orc.OracleConfig(Hq, Hkv, D, S, rope_type=rtype, norm_eps=1e-6, sliding_window=window,
                           arch=arch)
    out = {"shape": np.array([Hq, Hkv, D, S, pos, rtype, window, arch], np.int64),
           "theta": np.float64(theta), "layers": np.array(layers, np.int64)}
    for layer in layers:
        kc = np.zeros((S, kv), np.float32)
        vc = np.zeros((S, kv), np.float32)
        kc[:pos] = rng.standard_normal((pos, kv), dtype=np.float32)
        vc[:pos] = rng.standard_normal((pos, kv), dtype=np.float32)
        q = rng.standard_normal(Hq * D, dtype=np.float32)
        k = rng.standard_normal(kv, dtype=np.float32)
        v = rng.standard_normal(kv, dtype=np.float32)
        qw = rng.uniform(0.5, 1.5, D).astype(np.float32) if qkn else None
        kw = rng.uniform(0.5, 1.5, D).astype(np.float32) if qkn else None
        glob = orc.is_global_layer(arch, layer)
        th = 10000.0 if (arch == orc.ARCH_GEMMA3 and window > 0 and not glob) else theta
        cs, sn = orc.rope_tables(D, S, th)
        kc_in, vc_in = kc.copy(), vc.copy()
        o, q2, k2 = orc.forward_from_projections(cfg, kc, vc, q, k, v, layer, pos, qnorm_w=qw,
                                                 knorm_w=kw, rope_cos=cs, rope_sin=sn)
        p = f"l{layer}_"
        out.update({p + "kc": kc_in[:pos], p + "vc": vc_in[:pos], p + "q": q, p + "k": k,
                    p + "v": v, p + "out": o, p + "k_row": k2, p + "q_rot": q2})
        if qkn:
            out[p + "qnorm_w"] = qw
            out[p + "knorm_w"] = kw
    np.savez(os.path.join(HERE, f"{name}.npz"), **out)


if __name__ == "__main__":
    for i, (name, spec) in enumerate(CASES.items()):
        make(name, spec, 9000 + i)
        print("wrote", name)
