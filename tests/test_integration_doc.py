"""CPU checks of the Java (Panama FFM) binding a maintainer adds on the reference side, as the
repository's integration guide (DOC below) prints it: every `h("llmp_...", ...)` downcall descriptor against the prototype in
include/llmp_hip.h, every `NAME.invokeExact(...)` call against its descriptor's arity, and the
Java `kernelGroup` table against the Python mirror's.  No JDK is in this image, so the Java text
itself is what is checked."""
import os
import re

import pytest

from llmplayer_amd import hip_forward_pass as hfp

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "llmp_hip.h")
DOC = os.path.join(ROOT, "INTEGRATION.md")


def _ffm_layout(c_param):
    """The ValueLayout a C parameter binds as (CudaBindings.java:133-158 binds CUdeviceptr as
    JAVA_LONG): pointers ADDRESS, uint64_t/int64_t JAVA_LONG, int JAVA_INT, float JAVA_FLOAT."""
    p = c_param.strip()
    if "*" in p:
        return "ADDRESS"
    base = p.rsplit(None, 1)[0] if len(p.split()) > 1 else p
    base = base.replace("const", "").strip()
    return {"int": "JAVA_INT", "uint64_t": "JAVA_LONG", "int64_t": "JAVA_LONG",
            "float": "JAVA_FLOAT", "double": "JAVA_DOUBLE"}[base]


def header_prototypes():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    protos = {}
    for m in re.finditer(r"\bint\s+(llmp_\w+)\s*\(([^)]*)\)\s*;", text):
        args = [a for a in m.group(2).replace("\n", " ").split(",") if a.strip()]
        if len(args) == 1 and args[0].strip() == "void":
            args = []
        protos[m.group(1)] = [_ffm_layout(a) for a in args]
    return protos


def _balanced(text, start):
    """The text between the parenthesis at `start` and its match."""
    assert text[start] == "("
    depth = 0
    for i in range(start, len(text)):
        if text[i] == "(":
            depth += 1
        elif text[i] == ")":
            depth -= 1
            if depth == 0:
                return text[start + 1:i]
    raise AssertionError("unbalanced parentheses at %d" % start)


def _top_level_args(arglist):
    args, depth, cur = [], 0, ""
    for ch in arglist:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            args.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        args.append(cur.strip())
    return args


def doc_java():
    text = open(DOC).read()
    return "\n".join(re.findall(r"```java\n(.*?)```", text, flags=re.S))


def doc_descriptors():
    """{handle name: (function name, [layouts])} of every `static final MethodHandle X = h(...)`."""
    java = doc_java()
    out = {}
    for m in re.finditer(r"static final MethodHandle\s+(\w+)\s*=\s*h\(", java):
        args = _top_level_args(_balanced(java, m.end() - 1))
        fn = args[0].strip('"')
        assert m.group(1) not in out, "handle %s declared twice" % m.group(1)
        out[m.group(1)] = (fn, args[1:])
    return out


def test_every_declared_function_has_one_java_downcall():
    bound = [fn for fn, _ in doc_descriptors().values()]
    assert len(bound) == len(set(bound)), sorted(b for b in bound if bound.count(b) > 1)
    assert set(bound) == set(header_prototypes()), \
        (set(header_prototypes()) - set(bound), set(bound) - set(header_prototypes()))


@pytest.mark.parametrize("fn", sorted(header_prototypes()))
def test_java_descriptor_matches_the_prototype(fn):
    by_fn = {f: layouts for f, layouts in doc_descriptors().values()}
    assert by_fn[fn] == header_prototypes()[fn], (fn, by_fn[fn], header_prototypes()[fn])


def test_the_f32_prompt_path_is_bound_and_used():
    java = doc_java()
    d = doc_descriptors()
    for handle, fn in (("PREFILL_F32", "llmp_attn_prefill_f32"),
                       ("PREFILL_F32_STATIC", "llmp_attn_prefill_f32_static"),
                       ("PREFILL_SHARED_F32", "llmp_attn_prefill_shared_f32")):
        assert d[handle][0] == fn
        assert handle + ".invokeExact(" in java, handle


def test_every_java_call_passes_its_descriptor_arity():
    java = doc_java()
    d = doc_descriptors()
    calls = 0
    for m in re.finditer(r"\b([A-Z][A-Z0-9_]*)\.invokeExact\(", java):
        handle = m.group(1)
        assert handle in d, "call through undeclared handle %s" % handle
        args = _top_level_args(_balanced(java, m.end() - 1))
        assert len(args) == len(d[handle][1]), (handle, args, d[handle][1])
        calls += 1
    assert calls >= 20


def test_java_kernel_group_matches_the_python_mirror():
    java = doc_java()
    m = re.search(r"static int kernelGroup\(int headSize, int group\) \{(.*?)\n    \}", java, re.S)
    assert m, "kernelGroup not found"
    limits = {}
    for cases, lim in re.findall(r"case ([\d, ]+) -> (\d+);", m.group(1)):
        for c in cases.split(","):
            limits[int(c)] = int(lim)
    assert "default -> 0" in m.group(1)

    def java_kernel_group(head_size, group):
        limit = limits.get(head_size, 0)
        for g in range(min(group, limit), 0, -1):
            if group % g == 0:
                return g
        return 0

    for head_size in range(1, 600):
        for group in range(1, 49):
            assert java_kernel_group(head_size, group) == hfp.kernel_group(head_size, group), \
                (head_size, group)
