"""Numerical stability and steady-state GPU tests, after the reference's
stability suite (test/test_comprehensive.py:381-453, C01-C06) and its
memory check (test/test_supplementary.py, S04), at its shapes (B=1 H=1 S=128
D=64) and at D=128, in every dtype the case applies to.

The reference checks only that outputs are finite (and O = 0 for V = 0);
here the outputs are also compared with the float64 oracle or with a closed
form that does not go through it:
  * Q = 0: every allowed key has the same score, so causal O is the running
    mean of V (cumsum / count) and LSE = log(count);
  * LSE = logsumexp of the masked scaled scores (torch.logsumexp in float64);
  * V = 0: O, dQ and dK are exactly zero (Delta = 0 and dP = 0).
"""
import math

import pytest
import torch

import npu_flash_attention as nfa
from gpu_helpers import TOL, check, draw, fwd_bwd, oracle_fwd_bwd

pytestmark = pytest.mark.gpu

DTYPES = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


def _finite(*xs):
    return all(bool(torch.isfinite(x.float()).all()) for x in xs)


def _inputs(seed, d, dtype, mult, dev):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, 2, 128, d, generator=g) * mult
    k = torch.randn(1, 2, 128, d, generator=g) * mult
    v = torch.randn(1, 2, 128, d, generator=g)
    do = torch.randn(1, 2, 128, d, generator=g)
    cpu = [t.to(dtype) for t in (q, k, v, do)]
    return cpu, [t.to(dev) for t in cpu]


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dt", list(DTYPES))
def test_small_scale(gpu_device, dt, d):
    """C02: scale 0.01 (nearly uniform rows); forward and backward against the
    oracle at the usual bounds."""
    dtype = DTYPES[dt]
    cpu, dev = _inputs(102, d, dtype, 1.0, gpu_device)
    got = fwd_bwd(nfa, *dev, causal=True, scale=0.01)
    ref = oracle_fwd_bwd(*cpu, causal=True, scale=0.01)
    for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
        check(name, x, r, dtype)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dt", list(DTYPES))
def test_large_scale(gpu_device, dt, d):
    """C01: scale 10 on Q and K x10 (scores ~1e4: one-hot rows, the running
    max jumping from tile to tile).  Every output is finite and LSE matches the
    oracle at the usual bound.  At such magnitudes an fp32 score carries a
    rounding error of ~1e-3, which moves the weights of near-tied keys, so O is
    held to 1e-2 of its scale (a wrong max or rescale is off by O(1)) and the
    gradients, whose dS = P (dP - Delta) is most sensitive exactly there, only
    to being finite (as the reference's C01 holds the forward)."""
    dtype = DTYPES[dt]
    cpu, dev = _inputs(101, d, dtype, 10.0, gpu_device)
    got = fwd_bwd(nfa, *dev, causal=True, scale=10.0)
    assert _finite(*got), "non-finite output"
    ref = oracle_fwd_bwd(*cpu, causal=True, scale=10.0)
    check("lse", got[1], ref[1], dtype)
    check("o", got[0], ref[0], dtype, factor=1e-2 / TOL[dtype]["o"])


@pytest.mark.parametrize("d", [64, 128])
def test_extreme_inputs_fp16(gpu_device, d):
    """C03: fp16 Q and K x100 at the default scale (scores ~1e4; P is one-hot
    per row) stay finite and match the oracle."""
    g = torch.Generator().manual_seed(103)
    q = torch.randn(1, 2, 128, d, generator=g) * 100
    k = torch.randn(1, 2, 128, d, generator=g) * 100
    v = torch.randn(1, 2, 128, d, generator=g)
    do = torch.randn(1, 2, 128, d, generator=g)
    cpu = [t.to(torch.float16) for t in (q, k, v, do)]
    dev = [t.to(gpu_device) for t in cpu]
    got = fwd_bwd(nfa, *dev, causal=True)
    assert _finite(got[0], got[1]), "non-finite forward output"
    ref = oracle_fwd_bwd(*cpu, causal=True)
    check("o", got[0], ref[0], torch.float16)
    check("lse", got[1], ref[1], torch.float16)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dt", list(DTYPES))
def test_zero_value(gpu_device, dt, d):
    """C04: V = 0 gives O = 0 and dQ = dK = 0 exactly; dV = P^T dO matches the
    oracle."""
    dtype = DTYPES[dt]
    cpu, dev = draw(104, 1, 2, 1, 200, 200, d, dtype)
    cpu[2] = torch.zeros_like(cpu[2])
    dev[2] = torch.zeros_like(dev[2])
    o, lse, dq, dk, dv = fwd_bwd(nfa, *dev, causal=True)
    assert (o == 0).all() and (dq == 0).all() and (dk == 0).all()
    ref = oracle_fwd_bwd(*cpu, causal=True)
    check("lse", lse, ref[1], dtype)
    check("dv", dv, ref[4], dtype)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dt", list(DTYPES))
def test_zero_query_running_mean(gpu_device, dt, d):
    """C05: Q = 0 makes every allowed score 0: causal O is the running mean of
    V and LSE = log(i + 1), computed here in float64 without the oracle."""
    dtype = DTYPES[dt]
    cpu, dev = draw(105, 1, 2, 1, 300, 300, d, dtype)
    q = torch.zeros_like(dev[0])
    o, lse = nfa.npu_flash_attention_forward(q, dev[1], dev[2], causal=True, return_lse=True)
    v = cpu[2].double()[:, :1]  # one KV head
    n = torch.arange(1, 301, dtype=torch.float64).view(1, 1, -1, 1)
    want = (v.cumsum(2) / n).expand(-1, 2, -1, -1)
    check("o", o, want, dtype)
    check("lse", lse, torch.log(n.view(1, 1, -1)).expand(1, 2, -1), dtype)


@pytest.mark.parametrize("s", [128, 256, 512, 1024, 2048])
def test_lse_is_logsumexp(gpu_device, s):
    """C06: LSE is finite and equals torch.logsumexp of the masked scaled
    scores (float64) for S = 128 .. 2048."""
    cpu, dev = draw(106 + s, 1, 1, 1, s, s, 64, torch.float32)
    _, lse = nfa.npu_flash_attention_forward(*dev[:3], causal=True, return_lse=True)
    assert _finite(lse) and float(lse.abs().max()) < 1000
    x = cpu[0].double() @ cpu[1].double().transpose(-1, -2) / math.sqrt(64)
    x = x.masked_fill(torch.ones(s, s, dtype=torch.bool).triu(1), float("-inf"))
    check("lse", lse, torch.logsumexp(x, dim=-1), torch.float32)


@pytest.mark.parametrize("dt", ["bf16", "fp32"])
def test_no_memory_growth(gpu_device, dt):
    """S04: repeated forward + backward steps return device memory to the same
    level (the library allocates nothing; the backward's dS workspace comes
    from torch's caching allocator and is released with the call)."""
    dtype = DTYPES[dt]
    _, dev = draw(107, 1, 4, 2, 512, 512, 128, dtype)
    for _ in range(3):
        fwd_bwd(nfa, *dev, causal=True)
    torch.cuda.synchronize(gpu_device)
    base = torch.cuda.memory_allocated(gpu_device)
    for _ in range(20):
        out = fwd_bwd(nfa, *dev, causal=True)
        del out
        torch.cuda.synchronize(gpu_device)
        assert torch.cuda.memory_allocated(gpu_device) == base
