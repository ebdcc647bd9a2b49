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
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(flexatt_\w+)\s*\(", text, re.M)))


def test_header_declares_the_binding_exports():
    assert declared_functions() == sorted(L.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = L.load()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_abi_version_and_status_strings():
    lib = L.load()
    assert lib.flexatt_abi_version() == L.ABI_VERSION
    assert b"#define FLEXATT_ABI_VERSION 1" in open(HEADER, "rb").read()
    for code in (0, -1, -2, -3, -4, -5):
        assert lib.flexatt_status_string(code)
    assert b"head_dim" in lib.flexatt_status_string(-3)


def test_struct_layout_matches_header():
    # flexatt_tensor: pointer + 4 x int64; flexatt_problem: 7 int32, float, 2 int32, float, pointer
    assert ctypes.sizeof(L.Tensor) == 40
    assert L.Problem.alibi_slopes.offset == 48 and ctypes.sizeof(L.Problem) == 56


def problem(**kw):
    p = L.Problem()
    vals = dict(dtype=L.BF16, batch=1, heads_q=4, heads_kv=2, seqlen_q=64, seqlen_kv=64, head_dim=64,
                scale=0.125, causal=1, sliding_window=0, soft_cap=0.0, alibi_slopes=None)
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
