"""libflexatt.so loads and exports every entry point include/flexatt.h declares;
argument checks reject bad input before any launch — CPU only (no kernel is
ever launched here: every call below fails validation first)."""
import ctypes
import os
import re

import pytest

import flexatt_lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flexatt.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(flexatt_\w+)\s*\(", text, re.M)))


def test_header_declares_the_binding_exports():
    assert declared_functions() == sorted(L.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = L.load()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_abi_version_and_status_strings():
    lib = L.load()
    assert lib.flexatt_abi_version() == L.ABI_VERSION
    assert b"#define FLEXATT_ABI_VERSION 4" in open(HEADER, "rb").read()
    for code in (0, -1, -2, -3, -4, -5, -6):
        assert lib.flexatt_status_string(code)
    assert b"head_dim" in lib.flexatt_status_string(-3)


def test_struct_layout_matches_header():
    # flexatt_tensor: pointer + 4 x int64; flexatt_problem: 7 int32, float, 2 int32, float, 2 pointers
    assert ctypes.sizeof(L.Tensor) == 40
    assert L.Problem.alibi_slopes.offset == 48 and L.Problem.doc_bounds.offset == 56
    assert ctypes.sizeof(L.Problem) == 64


def problem(**kw):
    p = L.Problem()
    vals = dict(dtype=L.BF16, batch=1, heads_q=4, heads_kv=2, seqlen_q=64, seqlen_kv=64, head_dim=64,
                scale=0.125, causal=1, sliding_window=0, soft_cap=0.0, alibi_slopes=None, doc_bounds=None)
    vals.update(kw)
    for k, v in vals.items():
        setattr(p, k, v)
    return p


FAKE = 1 << 20  # an aligned non-null address that is never dereferenced


def tens(**kw):
    vals = dict(data=FAKE, stride_b=4 * 64 * 64, stride_h=64 * 64, stride_s=64, stride_d=1)
    vals.update(kw)
    return L.Tensor(vals["data"], vals["stride_b"], vals["stride_h"], vals["stride_s"], vals["stride_d"])


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=7), -2),
    (dict(head_dim=48), -3),
    (dict(head_dim=512), -3),
    (dict(heads_q=3, heads_kv=2), -4),
    (dict(seqlen_kv=0), -1),
    (dict(batch=-1), -1),
    (dict(causal=2), -1),
    (dict(sliding_window=-3), -1),
    (dict(soft_cap=-1.0), -1),
    (dict(scale=float("inf")), -1),
])
def test_problem_rejections(kw, code):
    lib = L.load()
    t = tens()
    assert lib.flexatt_fwd(problem(**kw), t, t, t, t, FAKE, None) == code
    assert lib.flexatt_bwd(problem(**kw), t, t, t, t, t, FAKE, FAKE, t, t, t, None) == code


@pytest.mark.parametrize("kw", [dict(stride_d=2), dict(data=FAKE + 2), dict(stride_s=65), dict(stride_h=-64)])
def test_layout_rejections(kw):
    lib = L.load()
    good, bad = tens(), tens(**kw)
    p = problem()
    assert lib.flexatt_fwd(p, bad, good, good, good, FAKE, None) == -5
    assert lib.flexatt_fwd(p, good, good, good, bad, FAKE, None) == -5
    assert lib.flexatt_bwd_dq(p, good, good, good, bad, FAKE, FAKE, good, None) == -5
    assert lib.flexatt_bwd_dkdv(p, good, good, good, good, FAKE, FAKE, good, bad, None) == -5


def test_null_pointers_rejected():
    lib = L.load()
    t = tens()
    p = problem()
    assert lib.flexatt_fwd(None, t, t, t, t, FAKE, None) == -1
    assert lib.flexatt_fwd(p, t, t, t, t, None, None) == -1
    assert lib.flexatt_bwd_delta(p, t, t, None, None) == -1
    assert lib.flexatt_fwd(p, tens(data=0), t, t, t, FAKE, None) == -1


def test_decode_workspace_range():
    """flexatt_fwd_decode_workspace: 0 outside the decode range (fp32, D = 256,
    (Hq / Hkv) * Sq > 32, invalid problem); in range, the bytes of the partials."""
    lib = L.load()
    ws = lib.flexatt_fwd_decode_workspace
    assert ws(problem(dtype=L.F32, seqlen_q=1)) == 0
    assert ws(problem(head_dim=256, seqlen_q=1)) == 0
    assert ws(problem(heads_q=8, heads_kv=1, seqlen_q=5)) == 0  # 40 query rows per KV head
    assert ws(problem(seqlen_q=1, heads_q=3)) == 0              # Hq % Hkv != 0
    # B=1, Hq=4, Hkv=2, Sq=1, Skv=8192, D=64, not causal: 256 tiles of 32 rows,
    # splits = min(512 / 2, 256 / 8) = 32, one partial (D + 1 floats) per split and row
    n = ws(problem(seqlen_q=1, seqlen_kv=8192, causal=0))
    assert n == 4 * 32 * 65 * 4
    # causal (top-left): a single query row only ever sees key 0
    assert ws(problem(seqlen_q=1, seqlen_kv=8192, causal=1)) == 4 * 1 * 65 * 4


def test_decode_rejections():
    lib = L.load()
    t = tens()
    p = problem(seqlen_q=1, seqlen_kv=8192, causal=0)
    need = lib.flexatt_fwd_decode_workspace(p)
    assert lib.flexatt_fwd_decode(problem(head_dim=256, seqlen_q=1), t, t, t, t, FAKE, FAKE, need, None) == -6
    assert lib.flexatt_fwd_decode(problem(seqlen_q=64), t, t, t, t, FAKE, FAKE, need, None) == -6
    assert lib.flexatt_fwd_decode(p, t, t, t, t, FAKE, FAKE, need - 1, None) == -1
    assert lib.flexatt_fwd_decode(p, t, t, t, t, FAKE, None, need, None) == -1
    assert lib.flexatt_fwd_decode(p, t, t, t, t, None, FAKE, need, None) == -1
    assert lib.flexatt_fwd_decode(p, t, t, t, t, FAKE, FAKE + 8, need, None) == -5
    assert lib.flexatt_fwd_decode(p, t, t, t, tens(stride_d=2), FAKE, FAKE, need, None) == -5


@pytest.mark.parametrize("entry", ["fwd", "dq", "dkdv"])
def test_overlapping_outputs_rejected(entry):
    """An output whose elements share addresses (a zero or too-small stride)
    is refused: several workgroups would store to one address."""
    lib = L.load()
    good = tens()
    p = problem(batch=2)
    for bad in (tens(stride_h=0), tens(stride_s=0), tens(stride_b=0), tens(stride_s=32), tens(stride_h=64 * 63)):
        if entry == "fwd":
            rc = lib.flexatt_fwd(p, good, good, good, bad, FAKE, None)
        elif entry == "dq":
            rc = lib.flexatt_bwd_dq(p, good, good, good, good, FAKE, FAKE, bad, None)
        else:
            rc = lib.flexatt_bwd_dkdv(p, good, good, good, good, FAKE, FAKE, good, bad, None)
        assert rc == -5, (entry, bad.stride_b, bad.stride_h, bad.stride_s)


def test_outputs_with_unit_extent_or_permuted_strides_pass_the_layout_check():
    """A zero stride over an extent-1 dimension, and a [B, S, H, D] storage
    order, are not overlaps: these calls get past the layout checks (and then
    stop at the null lse pointer, before any launch)."""
    lib = L.load()
    good = tens()
    p = problem(batch=1)
    assert lib.flexatt_fwd(p, good, good, good, tens(stride_b=0), None, None) == -1
    bsnd = tens(stride_b=64 * 4 * 64, stride_h=64, stride_s=4 * 64)
    assert lib.flexatt_fwd(p, good, good, good, bsnd, None, None) == -1


def _integration_stub():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```python\n(.*?)```", text, re.S)
    stubs = [b for b in blocks if "class FlexProblem" in b]
    assert len(stubs) == 1, "INTEGRATION.md should hold one ctypes stub"
    return stubs[0]


def test_integration_stub_matches_the_abi(monkeypatch):
    """The reference-side binding documented in INTEGRATION.md runs against
    the built library (it checks the ABI version itself) and its structs have
    the header's size and field offsets."""
    monkeypatch.setenv("FLEXATT_LIB", L.LIB_PATH)
    L.load()
    ns = {}
    exec(compile(_integration_stub(), "INTEGRATION.md", "exec"), ns)
    assert ns["_ABI"] == L.ABI_VERSION
    for stub, ours in ((ns["FlexProblem"], L.Problem), (ns["FlexTensor"], L.Tensor)):
        assert ctypes.sizeof(stub) == ctypes.sizeof(ours)
        assert [f[0] for f in stub._fields_] == [f[0] for f in ours._fields_]
        for name, _ in ours._fields_:
            assert getattr(stub, name).offset == getattr(ours, name).offset, name
    assert ctypes.sizeof(ns["FlexProblem"]) == 64 and ns["FlexProblem"].doc_bounds.offset == 56


def test_header_struct_layout_compiled(tmp_path):
    """sizeof / offsetof of the header's structs, compiled with the host C
    compiler, equal the ctypes layout of the Python binding."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "flexatt.h"\n'
        "#define F(s, m) printf(#m \" %zu\\n\", offsetof(s, m));\n"
        "int main(void) {\n"
        '  printf("problem %zu\\n", sizeof(flexatt_problem));\n'
        '  printf("tensor %zu\\n", sizeof(flexatt_tensor));\n'
        + "".join(f"  F(flexatt_problem, {f[0]})\n" for f in L.Problem._fields_)
        + "".join(f"  F(flexatt_tensor, {f[0]})\n" for f in L.Tensor._fields_)
        + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run([cc, "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    vals = [int(line.split()[1]) for line in out if line]
    assert vals[0] == ctypes.sizeof(L.Problem) and vals[1] == ctypes.sizeof(L.Tensor)
    want = [getattr(L.Problem, f[0]).offset for f in L.Problem._fields_] + \
           [getattr(L.Tensor, f[0]).offset for f in L.Tensor._fields_]
    assert vals[2:] == want
