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
    assert f"#define FLEXATT_ABI_VERSION {L.ABI_VERSION}".encode() in open(HEADER, "rb").read()
    assert f"#define FLEXATT_BWD_QUEUE_BYTES {L.BWD_QUEUE_BYTES}".encode() in open(HEADER, "rb").read()
    for code in (0, -1, -2, -3, -4, -5, -6):
        assert lib.flexatt_status_string(code)
    assert b"head_dim" in lib.flexatt_status_string(-3)


def test_struct_layout_matches_header():
    # flexatt_tensor: pointer + 4 x int64; flexatt_problem: 7 int32, float, 2 int32, float, 4 pointers,
    # 2 int32
    assert ctypes.sizeof(L.Tensor) == 40
    assert L.Problem.alibi_slopes.offset == 48 and L.Problem.doc_bounds.offset == 56
    assert L.Problem.col_bounds.offset == 64 and L.Problem.block_map.offset == 72
    assert L.Problem.block_heads.offset == 80 and ctypes.sizeof(L.Problem) == 88


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
    (dict(col_bounds=FAKE), -1),                              # column bounds without row bounds
    (dict(doc_bounds=FAKE, seqlen_q=32), -4),                 # symmetric bounds need Sq == Skv
    (dict(block_map=FAKE, block_heads=2), -1),                # block_heads not in {1, Hq}
    (dict(block_map=FAKE, block_heads=1, seqlen_kv=2048 * 128 + 1), -6),  # block row longer than 2048
    (dict(reserved=1), -1),
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
    """The reference-side ctypes binding given in the integration guide runs
    against the built library (it checks the ABI version itself) and its structs have
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
    assert ctypes.sizeof(ns["FlexProblem"]) == 88 and ns["FlexProblem"].block_map.offset == 72


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


def _staged_units(sq, skv, causal, window):
    """Units (32-row query tile t, 128-row KV block kb) the dK/dV kernel
    visits, per its rule: block kb covers query rows [q_lo, q_hi) with
    q_lo = 128 kb if causal else 0 and q_hi = min(Sq, 128 kb + 128 + W) with
    a window; also check that every unit holding an attended pair is among
    them."""
    nkb = -(-skv // 128)
    units = set()
    for kb in range(nkb):
        q_lo = 128 * kb if causal else 0
        q_hi = min(sq, 128 * kb + 128 + window) if window > 0 else sq
        if q_hi > q_lo:
            for t in range(q_lo // 32, -(-q_hi // 32)):
                units.add((t, kb))
    for t in range(-(-sq // 32)):
        for kb in range(nkb):
            j0, j1 = 128 * kb, min(skv, 128 * kb + 128) - 1
            # some row i of the tile keeps a key j of the block: j <= i (causal), i - j <= W (window)
            hit = any(max(j0, i - window if window else j0) <= (min(j1, i) if causal else j1)
                      for i in range(32 * t, min(sq, 32 * t + 32)))
            if hit:
                assert (t, kb) in units, (sq, skv, causal, window, t, kb)
    # the band each query tile is given in the workspace (ds_kb_lo / ds_kb_hi
    # of flexatt_device.h) is exactly the visited set, so every store lands
    # in its own slot
    band = set()
    for t in range(-(-sq // 32)):
        lo = min(nkb, max(0, (32 * t - window) // 128)) if window > 0 else 0
        hi = min(nkb, t // 4 + 1) if causal else nkb
        band.update((t, kb) for kb in range(lo, hi))
    assert band == units
    return len(units)


def _band(sq, skv, causal, window):
    """(t, kb) units of the staged-dS band (ds_kb_lo / ds_kb_hi of flexatt_device.h)."""
    nkb = -(-skv // 128)
    band = set()
    for t in range(-(-sq // 32)):
        lo = min(nkb, max(0, (32 * t - window) // 128)) if window > 0 else 0
        hi = min(nkb, t // 4 + 1) if causal else nkb
        band.update((t, kb) for kb in range(lo, hi))
    return band


@pytest.mark.parametrize("bn,rows", [(64, 16), (128, 16), (128, 32), (256, 32)])
@pytest.mark.parametrize("sq,skv", [(1, 1), (100, 70), (300, 129), (1000, 257), (129, 1000), (777, 900)])
@pytest.mark.parametrize("causal,window", [(0, 0), (1, 0), (1, 1), (1, 100), (0, 33), (1, 300)])
def test_f32_staged_slices_cover_the_band(bn, rows, sq, skv, causal, window):
    """The fp32 dK/dV kernels (bn KV rows per workgroup, `rows` per wave)
    store each `rows`-column slice of every band unit that the dQ kernel
    reads, and none twice: a
    workgroup at KV row n0 walks the query tiles of the whole band of the
    128-row blocks its rows fall in (q_lo = 128 floor(n0 / 128) if causal,
    q_hi = min(Sq, 128 (floor((n0 + bn - 1) / 128) + 1) + W) with a window)
    and a wave stores where its block kb_w < nkb is in the tile's band."""
    nkb = -(-skv // 128)
    band = _band(sq, skv, causal, window)
    stored = {}
    for n0 in range(0, -(-skv // bn) * bn, bn):
        q_lo = 128 * (n0 // 128) if causal else 0
        q_hi = min(sq, 128 * ((n0 + bn - 1) // 128 + 1) + window) if window > 0 else sq
        m_first = (q_lo // 32) * 32
        for m0 in range(m_first, q_hi, 32):
            t = m0 // 32
            for nw in range(n0, n0 + bn, rows):
                kb_w = nw // 128
                if kb_w < nkb and (t, kb_w) in band:
                    key = (t, kb_w, nw % 128)
                    assert key not in stored, key
                    stored[key] = True
    # the dQ kernel reads the 32-row K tiles that start below Skv
    read_end = -(-skv // 32) * 32
    want = {(t, kb, c) for (t, kb) in band for c in range(0, 128, rows) if 128 * kb + c < read_end}
    assert want <= set(stored)


@pytest.mark.parametrize("sq,skv", [(1, 1), (31, 33), (128, 128), (300, 129), (4096, 4096), (1000, 257),
                                    (129, 1000), (16384, 16383), (777, 5000)])
@pytest.mark.parametrize("causal,window", [(0, 0), (1, 0), (1, 1), (1, 100), (0, 33), (1, 128), (1, 2048), (0, 4096)])
def test_bwd_workspace_counts_the_band(sq, skv, causal, window):
    """flexatt_bwd_workspace (closed form of the staged-dS band) equals the
    units the dK/dV kernel visits, times B * Hq * 8 KB, plus the work-queue
    counters; 0 off its range."""
    lib = L.load()
    p = problem(batch=2, heads_q=6, heads_kv=2, seqlen_q=sq, seqlen_kv=skv, head_dim=128, causal=causal,
                sliding_window=window)
    assert lib.flexatt_bwd_workspace(p) == 2 * 6 * _staged_units(sq, skv, causal, window) * 8192 + L.BWD_QUEUE_BYTES


def test_bwd_workspace_range():
    lib = L.load()
    ws = lib.flexatt_bwd_workspace
    assert ws(problem(head_dim=128)) > 0
    assert ws(problem(head_dim=128, dtype=L.F16)) > 0
    assert ws(problem(head_dim=64)) == ws(problem(head_dim=128))  # 2 bytes per pair whatever D
    assert ws(problem(head_dim=256)) == ws(problem(head_dim=128))
    assert ws(problem(head_dim=32)) == 0
    # fp32 stages dS in fp32 over the same units: 4 bytes per pair, every D
    band = ws(problem(head_dim=128)) - L.BWD_QUEUE_BYTES
    for d in (32, 64, 128, 256):
        assert ws(problem(head_dim=d, dtype=L.F32)) == 2 * band + L.BWD_QUEUE_BYTES
    # masks keep the causal / window band of stored units (masked entries hold zeros)
    assert ws(problem(head_dim=128, doc_bounds=FAKE)) == ws(problem(head_dim=128))
    assert ws(problem(head_dim=128, block_map=FAKE, block_heads=1)) == ws(problem(head_dim=128))
    assert ws(problem(head_dim=128, heads_q=3)) == 0  # invalid problem


def test_staged_bwd_rejections():
    lib = L.load()
    t = tens(stride_b=4 * 64 * 128, stride_h=64 * 128, stride_s=128)
    p = problem(head_dim=128)
    need = lib.flexatt_bwd_workspace(p)
    band = need - L.BWD_QUEUE_BYTES  # the two kernels on their own need the dS band only
    st = lib.flexatt_bwd_dkdv_ds(p, t, t, t, t, FAKE, FAKE, t, t, FAKE, band - 1, None)
    assert st == -1
    assert lib.flexatt_bwd_dkdv_ds(p, t, t, t, t, FAKE, FAKE, t, t, None, need, None) == -1
    assert lib.flexatt_bwd_dkdv_ds(p, t, t, t, t, FAKE, FAKE, t, t, FAKE + 8, need, None) == -5
    assert lib.flexatt_bwd_dq_ds(p, t, FAKE, band - 1, t, None) == -1
    assert lib.flexatt_bwd_dq_ds(problem(head_dim=32), tens(), FAKE, need, tens(), None) == -6
    assert lib.flexatt_bwd_dkdv_ds(problem(head_dim=32), tens(), tens(), tens(), tens(), FAKE, FAKE, tens(),
                                   tens(), FAKE, need, None) == -6
    # a workspace below one (batch, KV-head) group's band (here half of the
    # band: B = 1, Hkv = 2) is rejected; between that and the whole band the
    # call would run in passes
    assert lib.flexatt_bwd_ws(p, t, t, t, t, t, FAKE, FAKE, t, t, t, FAKE, band // 2 - 1, None) == -1
    assert lib.flexatt_bwd_ws(p, t, t, t, t, t, FAKE, FAKE, t, t, t, None, band, None) == -1
    assert lib.flexatt_bwd_ws(p, t, t, t, t, t, FAKE, FAKE, t, t, t, FAKE + 8, band, None) == -5
    assert lib.flexatt_bwd_ws(p, t, t, t, t, t, FAKE, FAKE, tens(stride_h=0, stride_s=128), t, t, FAKE, need,
                              None) == -5


@pytest.mark.parametrize("B,hq,hkv", [(2, 6, 2), (1, 8, 8), (3, 4, 1), (2, 32, 8)])
@pytest.mark.parametrize("sq,skv,causal,window", [(4096, 4096, 1, 0), (300, 129, 0, 0), (1000, 1000, 1, 100)])
def test_bwd_workspace_limited_plan(B, hq, hkv, sq, skv, causal, window):
    """flexatt_bwd_workspace_limited under a byte budget: the whole band when it
    fits; else the band of the most whole (batch, KV-head) groups that fit,
    rounded down to whole batches when at least one batch fits; else 0 (the
    recomputing backward).  A group's band is G query heads' units x 8 KB."""
    lib = L.load()
    p = problem(batch=B, heads_q=hq, heads_kv=hkv, seqlen_q=sq, seqlen_kv=skv, head_dim=128, causal=causal,
                sliding_window=window)
    q = L.BWD_QUEUE_BYTES
    full = lib.flexatt_bwd_workspace(p)
    gb = (hq // hkv) * _staged_units(sq, skv, causal, window) * 8192
    assert full == B * hkv * gb + q
    lim = lib.flexatt_bwd_workspace_limited
    assert lim(p, full) == full and lim(p, 1 << 62) == full
    assert lim(p, gb + q - 1) == 0 and lim(p, 0) == 0
    assert lim(p, gb + q) == (gb + q if B * hkv > 1 else full)
    for groups in range(1, B * hkv):
        want = groups if groups < hkv else groups // hkv * hkv
        assert lim(p, groups * gb + q) == want * gb + q, groups
        assert lim(p, groups * gb + q + gb - 1) == want * gb + q, groups
    # fp32 stages 4 bytes per pair: twice the bytes per group
    p32 = problem(batch=B, heads_q=hq, heads_kv=hkv, seqlen_q=sq, seqlen_kv=skv, head_dim=128, causal=causal,
                  sliding_window=window, dtype=L.F32)
    if B * hkv > 1:
        assert lim(p32, 2 * gb + q) == 2 * gb + q
        assert lim(p32, 2 * gb + q - 1) == 0
    # outside the staged range (head_dim 32 fp16/bf16), or an invalid problem: 0
    assert lim(problem(head_dim=32), 1 << 40) == 0 and lim(problem(heads_q=3), 1 << 40) == 0


@pytest.mark.parametrize("kw,want", [
    (dict(head_dim=128), 1),
    (dict(head_dim=256, soft_cap=50.0), 1),
    (dict(head_dim=64), 0),                       # the recomputing backward is faster
    (dict(head_dim=64, dtype=L.F16, causal=0, sliding_window=30), 0),
    (dict(head_dim=64, soft_cap=30.0), 1),        # its tanh recompute in dQ makes it slower
    (dict(head_dim=64, doc_bounds=FAKE), 1),      # masks: the recomputing dQ is the general kernel
    (dict(head_dim=64, dtype=L.F32), 1),
    (dict(head_dim=32), 0),                       # outside the staged range (fp16/bf16)
    (dict(head_dim=48), 0),                       # invalid problem
])
def test_bwd_prefers_staging(kw, want):
    """flexatt_bwd_prefers_staging: 1 inside the staged range except fp16/bf16
    at head_dim 64 without soft-cap or interval/block masks."""
    assert L.load().flexatt_bwd_prefers_staging(problem(**kw)) == want


def test_backward_staging_follows_the_preference(monkeypatch):
    """The Python layer stages at head_dim 64 without soft-cap only when
    ds_staging_auto is off; with soft-cap, or at head_dim 128, it stages
    either way."""
    import npu_flash_attention as nfa

    lib = L.load()
    plain = problem(batch=2, heads_q=8, heads_kv=2, seqlen_q=1000, seqlen_kv=1000, head_dim=64)
    capped = problem(batch=2, heads_q=8, heads_kv=2, seqlen_q=1000, seqlen_kv=1000, head_dim=64, soft_cap=30.0)
    d128 = problem(batch=2, heads_q=8, heads_kv=2, seqlen_q=1000, seqlen_kv=1000, head_dim=128)
    assert nfa.ds_staging_auto is True
    assert nfa._staged_workspace_bytes(lib, plain) == 0
    assert nfa._staged_workspace_bytes(lib, capped) == lib.flexatt_bwd_workspace(capped) > 0
    assert nfa._staged_workspace_bytes(lib, d128) == lib.flexatt_bwd_workspace(d128) > 0
    monkeypatch.setattr(nfa, "ds_staging_auto", False)
    assert nfa._staged_workspace_bytes(lib, plain) == lib.flexatt_bwd_workspace(plain) > 0


def test_workspace_budget_takes_a_share_of_free_memory(monkeypatch):
    """The staged-dS budget is the larger of ds_workspace_limit and
    ds_workspace_free_fraction of the free device memory; without a free-memory
    figure (or with the fraction at 0) it is the fixed limit, never negative."""
    import npu_flash_attention as nfa

    assert nfa.ds_workspace_free_fraction == 0.25
    assert nfa._workspace_budget(0) == 4 << 30
    assert nfa._workspace_budget(8 << 30) == 4 << 30                # a quarter of 8 GiB is below the limit
    assert nfa._workspace_budget(100 << 30) == 25 << 30
    assert nfa._workspace_budget(-(1 << 40)) == 4 << 30
    monkeypatch.setattr(nfa, "ds_workspace_free_fraction", 0.0)
    assert nfa._workspace_budget(100 << 30) == 4 << 30
    monkeypatch.setattr(nfa, "ds_workspace_limit", -5)
    assert nfa._workspace_budget(100 << 30) == 0
    # a long bf16 causal problem whose groups exceed 4 GiB: staged in passes
    # once the budget covers one group, the recomputing backward below that
    monkeypatch.setattr(nfa, "ds_workspace_limit", 4 << 30)
    monkeypatch.setattr(nfa, "ds_workspace_free_fraction", 0.25)
    lib = L.load()
    big = problem(batch=1, heads_q=32, heads_kv=8, seqlen_q=65536, seqlen_kv=65536, head_dim=128, causal=1)
    gb = 4 * _staged_units(65536, 65536, 1, 0) * 8192
    assert gb > 4 << 30
    assert lib.flexatt_bwd_workspace_limited(big, nfa._workspace_budget(0)) == 0
    n = lib.flexatt_bwd_workspace_limited(big, nfa._workspace_budget(250 << 30))
    assert n == ((250 << 30) // 4 - L.BWD_QUEUE_BYTES) // gb * gb + L.BWD_QUEUE_BYTES and n > gb


def test_backward_selects_staging_within_the_limit(monkeypatch):
    """The Python layer's choice for one backward call: the staged backward
    with the workspace flexatt_bwd_workspace_limited gives under
    ds_workspace_limit (whole band or one chunk of groups), the recomputing
    backward (0) when not even one group's band fits, or when staging is off."""
    import npu_flash_attention as nfa

    lib = L.load()
    p = problem(batch=2, heads_q=32, heads_kv=8, seqlen_q=4096, seqlen_kv=4096, head_dim=128, causal=1)
    full = lib.flexatt_bwd_workspace(p)
    gb = 4 * _staged_units(4096, 4096, 1, 0) * 8192
    assert nfa.ds_workspace_limit == 4 << 30 and full < nfa.ds_workspace_limit
    assert nfa._staged_workspace_bytes(lib, p) == full  # the bench workload runs in one pass
    monkeypatch.setattr(nfa, "ds_workspace_limit", full - 1)
    assert nfa._staged_workspace_bytes(lib, p) == 8 * gb + L.BWD_QUEUE_BYTES  # one batch per pass
    monkeypatch.setattr(nfa, "ds_workspace_limit", 3 * gb + L.BWD_QUEUE_BYTES)
    assert nfa._staged_workspace_bytes(lib, p) == 3 * gb + L.BWD_QUEUE_BYTES  # three KV heads per pass
    monkeypatch.setattr(nfa, "ds_workspace_limit", gb)
    assert nfa._staged_workspace_bytes(lib, p) == 0  # recomputing backward
    monkeypatch.setattr(nfa, "ds_workspace_limit", -5)
    assert nfa._staged_workspace_bytes(lib, p) == 0
    monkeypatch.setattr(nfa, "ds_workspace_limit", 1 << 40)
    monkeypatch.setattr(nfa, "ds_staging_enabled", False)
    assert nfa._staged_workspace_bytes(lib, p) == 0
    # B=1 Hq=32 S=64k causal bf16: 137 GB of band, 17 GB per group: recompute at the default limit
    big = problem(batch=1, heads_q=32, heads_kv=8, seqlen_q=65536, seqlen_kv=65536, head_dim=128, causal=1)
    monkeypatch.setattr(nfa, "ds_staging_enabled", True)
    monkeypatch.setattr(nfa, "ds_workspace_limit", 4 << 30)
    assert lib.flexatt_bwd_workspace(big) > 130e9
    assert nfa._staged_workspace_bytes(lib, big) == 0


def test_build_rejects_scratch_in_async_load_kernels():
    """The build guard reads the compiler's resource remarks: any kernel of a
    source with asm register loads that uses scratch fails the build."""
    import build_lib
    remarks = "\n".join([
        "x.hip:1:1: remark: Function Name: _ZN7flexatt1aE [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark: Function Name: _ZN7flexatt1bE [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     VGPRs: 128 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     ScratchSize [bytes/lane]: 92 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert build_lib.scratch_kernels(remarks) == [("_ZN7flexatt1bE", 92)]
    assert build_lib.scratch_kernels("") == []
    assert "bwd_dq_ds.hip" in build_lib.NO_SCRATCH_SOURCES
