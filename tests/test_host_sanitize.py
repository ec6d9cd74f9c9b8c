"""The CPU code of the library and of the oracle under AddressSanitizer and
UndefinedBehaviorSanitizer:

- llmplayer_amd/csrc/host_layout.h (GGUF weight repacking, the KV re-layout between the
  reference's [pos][n_kv_heads * row] arrays and the head-major device planes, the decode step
  plan and the default split count), built with g++ into tests/host_layout_check.cpp and
  checked against the GGUF block layouts, numpy transposes and the step plan's invariants;
- the oracle (oracle/attn_oracle.c, oracle/block_oracle.c) built with the same sanitizers
  (`make -C oracle asan`), under which tests/test_oracle.py and tests/test_block_oracle.py run
  in a child process with the ASan runtime preloaded.

Any out-of-bounds access, use after free or undefined arithmetic aborts the sanitized process,
which fails the test."""
import os
import shutil
import subprocess
import sys

import numpy as np
import pytest

from tests import ggml_pack as gp

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g"]
SAN_ENV = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1", "UBSAN_OPTIONS": "print_stacktrace=1"}

pytestmark = pytest.mark.skipif(shutil.which("g++") is None or shutil.which("gcc") is None,
                                reason="needs gcc/g++ with the sanitizer runtimes")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    d = tmp_path_factory.mktemp("hostsan")
    exe = str(d / "host_layout_check")
    subprocess.run(["g++", "-std=c++17", "-O1", *SAN, "-I", os.path.join(ROOT, "llmplayer_amd", "csrc"),
                    "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "host_layout_check.cpp"),
                    "-o", exe], check=True)
    return exe, d


def _run(exe, lines):
    env = dict(os.environ, **SAN_ENV)
    r = subprocess.run([exe], input="\n".join(lines) + "\n", capture_output=True, text=True, env=env,
                       timeout=120)
    assert r.returncode == 0, f"sanitized driver failed ({r.returncode}):\n{r.stderr[-4000:]}"
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    return r.stdout.splitlines()


# GGUF block layouts (ggml's block_q8_0, block_q4_0, block_q4_K, block_q6_K), as
# (weights per block, [(field, bytes)] in memory order), and the plane each field goes to.
BLOCKS = {
    gp.GGML_Q8_0: (32, [("d", 2), ("qs", 32)], {"qs": 0, "d": 1}),
    gp.GGML_Q4_0: (32, [("d", 2), ("qs", 16)], {"qs": 0, "d": 1}),
    gp.GGML_Q4_K: (256, [("d", 2), ("dmin", 2), ("scales", 12), ("qs", 128)],
                   {"qs": 0, "d": 1, "dmin": 1, "scales": 1}),
    gp.GGML_Q6_K: (256, [("ql", 128), ("qh", 64), ("scales", 16), ("d", 2)],
                   {"ql": 0, "qh": 1, "scales": 2, "d": 3}),
    gp.GGML_Q5_0: (32, [("d", 2), ("qh", 4), ("qs", 16)], {"qs": 0, "qh": 1, "d": 2}),
    gp.GGML_Q3_K: (256, [("hmask", 32), ("qs", 64), ("scales", 12), ("d", 2)],
                   {"qs": 0, "hmask": 1, "d": 3}),
    gp.GGML_Q5_K: (256, [("d", 2), ("dmin", 2), ("scales", 12), ("qh", 32), ("qs", 128)],
                   {"qs": 0, "d": 1, "dmin": 1, "scales": 1, "qh": 2}),
    gp.GGML_IQ4_NL: (32, [("d", 2), ("qs", 16)], {"qs": 0, "d": 1}),
    gp.GGML_IQ4_XS: (256, [("d", 2), ("scales_h", 2), ("scales_l", 4), ("qs", 128)], {"qs": 0, "d": 2}),
    gp.GGML_MXFP4: (32, [("e", 1), ("qs", 16)], {"qs": 0, "e": 1}),
    gp.GGML_Q5_1: (32, [("d", 2), ("m", 2), ("qh", 4), ("qs", 16)], {"qs": 0, "qh": 1, "d": 2, "m": 3}),
    gp.GGML_Q2_K: (256, [("scales", 16), ("qs", 64), ("d", 2), ("dmin", 2)],
                   {"qs": 0, "scales": 1, "d": 2, "dmin": 3}),
    gp.GGML_IQ3_XXS: (256, [("d", 2), ("qs", 64), ("sas", 32)], {"qs": 0}),
    gp.GGML_IQ3_S: (256, [("d", 2), ("qs", 64), ("qh", 8), ("signs", 32), ("scales", 4)],
                    {"qs": 0, "signs": 1}),
    gp.GGML_IQ2_S: (256, [("d", 2), ("qs", 32), ("signs", 32), ("qh", 8), ("scales", 8)],
                    {"qs": 0, "signs": 1}),
}


def _q3k_scales(parts):
    # the 16 six-bit scales (low nibbles of bytes 0-7, then their high nibbles; top bit pairs
    # of bytes 8-11, two bits per scale in groups of four) as the int8 sc - 32
    raw = parts["scales"].astype(np.int64)
    low = np.concatenate([raw[..., 0:8] & 15, raw[..., 0:8] >> 4], axis=-1)
    top = np.concatenate([(raw[..., 8:12] >> (2 * j)) & 3 for j in range(4)], axis=-1)
    return ((low | (top << 4)) - 32).astype(np.int8).view(np.uint8)


def _iq4xs_scales(parts):
    sh = parts["scales_h"].astype(np.int64)
    sh = sh[..., 0] | (sh[..., 1] << 8)
    sl = parts["scales_l"].astype(np.int64)
    low = np.stack([sl[..., ib // 2] >> (4 * (ib % 2)) & 15 for ib in range(8)], axis=-1)
    top = np.stack([(sh >> (2 * ib)) & 3 for ib in range(8)], axis=-1)
    return ((low | (top << 4)) - 32).astype(np.int8).view(np.uint8)


def _iq3xxs_aux(parts):
    b = parts["sas"].astype(np.int64).reshape(parts["sas"].shape[:-1] + (8, 4))
    return b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16) | (b[..., 3] << 24)   # [rows, nb, 8]


def _iq3xxs_signs(parts):
    # each 8-weight group's 7-bit pattern index (bits 7l of its 32-group's word) with the parity
    # bit that makes the count of set bits even
    aux = _iq3xxs_aux(parts)
    idx = np.stack([(aux >> (7 * l)) & 0x7F for l in range(4)], axis=-1)        # [rows, nb, 8, 4]
    par = sum((idx >> k) & 1 for k in range(7)) & 1
    return (idx | (par << 7)).astype(np.uint8).reshape(aux.shape[:-1] + (32,))


def _iq3xxs_side(parts):
    # d, two zero bytes, the scales (bits 28-31 of each word) two per byte, low nibble first
    sc = _iq3xxs_aux(parts) >> 28
    packed = (sc[..., 0::2] | (sc[..., 1::2] << 4)).astype(np.uint8)
    zero = np.zeros(sc.shape[:-1] + (2,), np.uint8)
    return np.concatenate([parts["d"], zero, packed], axis=-1)


def _iq3s_side(parts):
    zero = np.zeros(parts["d"].shape, np.uint8)
    return np.concatenate([parts["qh"], parts["scales"], parts["d"], zero], axis=-1)


def _iq2s_side(parts):
    zero = np.zeros(parts["d"].shape[:-1] + (6,), np.uint8)
    return np.concatenate([parts["scales"], parts["qh"], parts["d"], zero], axis=-1)


# planes computed from a block's fields rather than copied from it
DERIVED = {gp.GGML_Q3_K: {2: _q3k_scales}, gp.GGML_IQ4_XS: {1: _iq4xs_scales},
           gp.GGML_IQ3_XXS: {1: _iq3xxs_signs, 2: _iq3xxs_side}, gp.GGML_IQ3_S: {2: _iq3s_side},
           gp.GGML_IQ2_S: {2: _iq2s_side}}
DENSE = {gp.GGML_F32: 4, gp.GGML_F16: 2, gp.GGML_BF16: 2}


def _expected_planes(t, rows, cols, raw):
    """Per plane, the [rows][pitch] bytes: each row's bytes of every field of that plane, block
    by block, the fields of one block in memory order."""
    if t in DENSE:
        return [raw.reshape(rows, cols * DENSE[t])]
    bw, fields, plane_of = BLOCKS[t]
    nb = cols // bw
    blk = raw.reshape(rows, nb, sum(n for _, n in fields))
    parts, o = {}, 0
    for name, n in fields:
        parts[name] = blk[:, :, o:o + n]
        o += n
    planes = []
    derived = DERIVED.get(t, {})
    for p in range(max(list(plane_of.values()) + list(derived)) + 1):
        if p in derived:
            planes.append(derived[p](parts).reshape(rows, -1))
            continue
        sel = [parts[name] for name, _ in fields if plane_of.get(name) == p]
        planes.append(np.concatenate(sel, axis=2).reshape(rows, -1))
    return planes


CASES = [(t, rows, cols) for t in (gp.GGML_F32, gp.GGML_F16, gp.GGML_BF16, gp.GGML_Q8_0, gp.GGML_Q4_0,
                                  gp.GGML_Q5_0, gp.GGML_IQ4_NL, gp.GGML_MXFP4, gp.GGML_Q5_1)
         for rows, cols in ((1, 32), (3, 96), (17, 2880))] + \
        [(t, rows, cols) for t in (gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q3_K, gp.GGML_Q5_K, gp.GGML_IQ4_XS,
                                  gp.GGML_Q2_K, gp.GGML_IQ3_XXS, gp.GGML_IQ3_S, gp.GGML_IQ2_S)
         for rows, cols in ((1, 256), (5, 768), (33, 3072))]


def test_repack_matches_the_gguf_block_layouts(driver):
    exe, d = driver
    rng = np.random.default_rng(11)
    lines, want = [], []
    for i, (t, rows, cols) in enumerate(CASES):
        bw = BLOCKS[t][0] if t in BLOCKS else 1
        row_bytes = cols * DENSE[t] if t in DENSE else cols // bw * sum(n for _, n in BLOCKS[t][1])
        raw = rng.integers(0, 256, rows * row_bytes, dtype=np.uint8)
        src, dst = d / f"w{i}.bin", d / f"p{i}.bin"
        raw.tofile(src)
        lines.append(f"repack {t} {rows} {cols} {src} {dst}")
        want.append((raw, dst))
    out = _run(exe, lines)
    for (t, rows, cols), line, (raw, dst) in zip(CASES, out, want):
        f = list(map(int, line.split()))
        n, off, pitch = f[0], f[1:5], f[5:9]
        planes = _expected_planes(t, rows, cols, raw)
        assert n == len(planes), (t, rows, cols)
        packed = np.fromfile(dst, np.uint8)
        assert len(packed) % 256 == 0
        end = 0
        for p, exp in enumerate(planes):
            assert off[p] % 256 == 0 and off[p] >= end, (t, p, off)
            assert pitch[p] == exp.shape[1], (t, p, pitch)
            got = packed[off[p]:off[p] + rows * pitch[p]].reshape(rows, pitch[p])
            np.testing.assert_array_equal(got, exp, err_msg=f"type {t} plane {p}")
            assert not packed[off[p] + rows * pitch[p]:(off[p + 1] if p + 1 < n else len(packed))].any()
            end = off[p] + rows * pitch[p]


def test_repack_rejects_partial_blocks_and_unknown_types(driver):
    exe, d = driver
    src = d / "tiny.bin"
    np.zeros(4096, np.uint8).tofile(src)
    out = _run(exe, [f"repack {gp.GGML_Q4_K} 1 128 {src} {d / 'x.bin'}",
                     f"repack {gp.GGML_Q8_0} 2 48 {src} {d / 'x.bin'}",
                     f"repack 99 1 32 {src} {d / 'x.bin'}",
                     f"repack {gp.GGML_F32} 1 0 {src} {d / 'x.bin'}"])
    assert [int(l.split()[0]) for l in out] == [0, 0, 0, 0]


@pytest.mark.parametrize("H,n,row", [(1, 1, 4), (8, 37, 512), (4, 5, 16), (32, 3, 80 * 4), (2, 64, 8)])
def test_kv_relayout_is_a_head_major_transpose(driver, H, n, row):
    exe, d = driver
    host = np.random.default_rng(H * n + row).integers(0, 256, (n, H * row), dtype=np.uint8)
    src, heads, back = d / "h.bin", d / "s.bin", d / "b.bin"
    host.tofile(src)
    assert _run(exe, [f"relayout {H} {n} {row} {src} {heads} {back}"]) == ["ok"]
    np.testing.assert_array_equal(np.fromfile(heads, np.uint8).reshape(H, n, row),
                                  host.reshape(n, H, row).transpose(1, 0, 2))
    np.testing.assert_array_equal(np.fromfile(back, np.uint8).reshape(n, H * row), host)


def test_step_plan_invariants(driver):
    """plan_step against its contract: the window's first row, rows that the splits cover
    exactly once (every split non-empty), at most the requested splits, rows per split a
    multiple of 16 once each split has 16 rows; positions up to 2^30."""
    exe, _ = driver
    rng = np.random.default_rng(5)
    cases = [(0, 0, 1), (0, 0, 1024), (15, 0, 1), (16, 4, 1), (4095, 0, 32), (32767, 0, 24),
             (8191, 1024, 64), (1023, 1024, 64), (1024, 1024, 64), (2**30, 0, 1024), (2**30, 4096, 7)]
    cases += [(int(rng.integers(0, 1 << 20)), int(rng.choice([0, 1, 128, 4096, rng.integers(1, 9000)])),
               int(rng.integers(1, 1025))) for _ in range(300)]
    out = _run(exe, [f"plan {p} {w} {s}" for p, w, s in cases])
    for (pos, window, splits), line in zip(cases, out):
        start, n, rps, s = map(int, line.split())
        assert start == (max(0, pos - window + 1) if window > 0 else 0)
        assert n == pos + 1 - start
        assert 1 <= s <= min(splits, n) and rps >= 1
        assert (s - 1) * rps < n <= s * rps, (pos, window, splits, line)
        if n >= 16 * min(splits, n):
            assert rps % 16 == 0


def test_default_splits(driver):
    """The measured plan at the Llama-3.2-3B shape (8 KV heads, 256 CUs): fp32 at 32k rows runs
    24 splits of 8-wave workgroups, at 4k 32 splits of 4; Q8_0 with 3 resident workgroups per CU
    runs 96 splits at 32k; Gemma-3's one KV head over a 512-row window runs 32 splits of 16 rows.
    In general 1 <= splits <= 128, fp32 splits hold >= 32 rows unless there is only one or
    32-row splits of all KV heads would fill less than half of the CUs (then >= 16), Q8_0 splits
    >= 160, and only fp32 calls widen."""
    exe, _ = driver
    out = _run(exe, ["splits 32768 8 256 1 0", "splits 4096 8 256 1 0", "splits 32768 8 256 3 1",
                     "splits 512 1 256 1 0", "splits 512 8 256 1 0"])
    assert out == ["24 1", "32 0", "96 0", "32 0", "16 0"]
    rng = np.random.default_rng(9)
    cases = [(int(rng.integers(1, 1 << 22)), int(rng.choice([1, 2, 4, 8, 32])), int(rng.choice([0, 80, 256, 304])),
              int(rng.integers(0, 6)), int(rng.integers(0, 2))) for _ in range(300)]
    out = _run(exe, [f"splits {n} {h} {c} {p} {q}" for n, h, c, p, q in cases])
    for (n, h, c, p, q), line in zip(cases, out):
        s, wide = map(int, line.split())
        assert 1 <= s <= 128
        assert not (q and wide)
        if s > 1 and not wide:
            few = 2 * h * (n // 32) < (c if c > 0 else 256)
            assert n // s >= (160 if q else (16 if few else 32)), (n, h, c, p, q, line)


def test_combine_column_groups(driver):
    """The combine's column workgroups per head (256 threads, 12 splits per thread in one batch):
    the known launches (C3 at 24/96 splits and Gemma-3's 128 splits at head_dim 256 run 1 and 4
    groups), and in general the fewest of 1/2/4/8 with which the batch covers the splits, whole
    float4 columns and at least 4 of them per group."""
    exe, _ = driver
    known = [(128, 24, 1), (128, 96, 1), (128, 97, 2), (256, 128, 4), (256, 48, 1), (128, 1000, 8),
             (80, 400, 4), (96, 400, 4), (96, 1000, 4), (64, 192, 1), (64, 193, 2), (512, 128, 8)]
    out = _run(exe, [f"cgroups {d} {s} 256 12" for d, s, _ in known])
    assert [int(x) for x in out] == [cb for _, _, cb in known]
    cases = [(d, s) for d in (64, 80, 96, 128, 256, 512) for s in (1, 2, 12, 47, 48, 49, 95, 96, 97, 191, 192,
                                                               193, 383, 384, 385, 767, 768, 769, 1024)]
    out = _run(exe, [f"cgroups {d} {s} 256 12" for d, s in cases])
    for (d, s), line in zip(cases, out):
        cb = int(line)
        nc = d // 4
        assert cb in (1, 2, 4, 8) and nc % cb == 0, (d, s, cb)
        assert cb == 1 or nc // cb >= 4, (d, s, cb)
        fits = lambda g: s <= 12 * (256 // (nc // g))
        if cb > 1:
            assert not fits(cb // 2), (d, s, cb)          # the fewest groups
        if not fits(cb):                                  # more groups only when it cannot split further
            assert cb == 8 or nc % (2 * cb) or nc // (2 * cb) < 4, (d, s, cb)


def test_kernel_group_matches_the_python_mirror(driver):
    """The group the kernels run a layer with (virtual KV heads for groups above the
    instantiated ones): the library's rule and the host mirror's (HipForwardPass's
    isSupportedForAttention) agree over head sizes and groups 0-64; GLM-4's groups 16 and 24
    run as groups of 8, a prime group as groups of 1, and head_dim 112 has no kernel."""
    from llmplayer_amd import hip_forward_pass as hfp
    exe, _ = driver
    cases = [(d, g) for d in (64, 80, 96, 112, 128, 256, 512) for g in range(0, 65)]
    out = _run(exe, [f"kgroup {d} {g}" for d, g in cases])
    got = [int(x) for x in out]
    assert got == [hfp.kernel_group(d, g) for d, g in cases]
    kg = dict(zip(cases, got))
    assert kg[(128, 16)] == 8 and kg[(128, 24)] == 8 and kg[(128, 12)] == 6 and kg[(128, 11)] == 1
    assert kg[(96, 6)] == 3 and kg[(80, 6)] == 2 and kg[(112, 1)] == 0 and kg[(64, 0)] == 0
    for (d, g), k in kg.items():
        if k:
            assert g % k == 0 and k <= {80: 2, 96: 4}.get(d, 8)


def _range_exp_ref(x):
    """max(0, floor(log2|x|) - 14), 0 for x = 0: the smallest e with |x| * 2^-e < 2^15."""
    x = np.abs(np.asarray(x, np.float64))
    out = np.zeros(x.shape, np.int64)
    nz = x > 0
    out[nz] = np.maximum(0, np.floor(np.log2(x[nz])).astype(np.int64) - 14)
    return out


def test_range_exponents(driver):
    """The host-side range exponents of rows written by llmp_kv_write / llmp_kv_write_q8 against
    the closed form, per KV head: boundary values 2^15 - ulp / 2^15 / 65504, 1e5, the fp32
    maximum, subnormals and zeros; and |x| * 2^-e < 2^15 for every value."""
    exe, d = driver
    rng = np.random.default_rng(11)
    H, n, row = 3, 5, 64
    k = rng.standard_normal((n, H * row)).astype(np.float32)
    v = rng.standard_normal((n, H * row)).astype(np.float32)
    special = np.array([np.nextafter(np.float32(32768), np.float32(0)), 32768, 65504, -1e5, 3.4e38,
                        1e-45, -0.0, 1e-7, -65535.9], np.float32)
    k[1, row:row + special.size] = special          # KV head 1
    v[4, 2 * row + 5] = np.float32(-3e7)            # KV head 2
    q = rng.integers(-128, 128, (n, H * row)).astype(np.int8)
    sc = (rng.random((n, H * row // 32)) * 1e-2).astype(np.float32)
    sc[2, 0] = np.float32(300.0)                    # KV head 0: 127 * 300 = 38100 -> e = 1
    q[2, 0] = 127
    (d / "k.bin").write_bytes(k.tobytes())
    (d / "v.bin").write_bytes(v.tobytes())
    (d / "q.bin").write_bytes(q.tobytes() + sc.tobytes())
    out = _run(exe, [f"range {H} {n} {row} {d / 'k.bin'} {d / 'v.bin'} {d / 'q.bin'}"])
    got = [int(t) for t in out[0].split()]
    deq = (q.astype(np.float32) * np.repeat(sc, 32, axis=1)).astype(np.float32)
    want = []
    for arr in (k, v, deq):
        want += [int(_range_exp_ref(arr.reshape(n, H, row)[:, h, :]).max()) for h in range(H)]
    assert got == want, (got, want)
    assert got[1] == 113 and got[H + 2] == 10 and got[2 * H] == 1
    e = _range_exp_ref(special)
    assert list(e) == [0, 1, 1, 2, 113, 0, 0, 0, 1]
    assert (np.abs(special.astype(np.float64)) * 2.0 ** -e < 2 ** 15).all()


def test_oracle_under_sanitizers(tmp_path):
    """tests/test_oracle.py and tests/test_block_oracle.py against the sanitized oracle build."""
    asan_dir = tmp_path / "asan"
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "asan", f"ASAN_DIR={asan_dir}"],
                   check=True, stdout=subprocess.DEVNULL)
    libasan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True,
                             check=True).stdout.strip()
    env = dict(os.environ, **SAN_ENV, LD_PRELOAD=libasan, LLMP_ORACLE_LIB=str(asan_dir / "libattn_oracle.so"))
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        os.path.join(ROOT, "tests", "test_oracle.py"),
                        os.path.join(ROOT, "tests", "test_block_oracle.py")],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    tail = (r.stdout[-3000:] + r.stderr[-3000:])
    assert r.returncode == 0, tail
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, tail
    assert " passed" in r.stdout and "failed" not in r.stdout, tail
