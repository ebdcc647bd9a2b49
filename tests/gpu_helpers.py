"""Helpers shared by the GPU parity tests (not collected by pytest).

Inputs are drawn on the CPU from torch.Generator().manual_seed(seed) as fp32
N(0,1) in the order q, k, v, dO, cast to the test dtype and copied to the GPU,
so the kernels and the CPU oracle see bit-identical inputs.

Tolerance criterion (stated once, used everywhere):
    err(x, ref) = max|x - ref| / max(1, max|ref|)
i.e. max-abs error for O(1) tensors and max-abs relative to the tensor's
magnitude for large gradients.  The oracle runs in float64 on the same
(rounded) inputs.  Every checked error, with the plain max-abs error beside
it, is recorded in RECORDS; the test session writes them to a JSON-lines file
(see conftest.py) so a GPU run returns the measured numbers.
"""
import math
import os

import torch

from oracle import attention_oracle as orc

# north-star tolerances (max-abs 5e-3 fp16, 2e-2 bf16 relative to the fp32 /
# float64 eager math) for all five outputs; LSE is held tighter.
TOL = {
    torch.float32: {"o": 1e-5, "lse": 1e-5, "dq": 1e-4, "dk": 1e-4, "dv": 1e-4},
    torch.float16: {"o": 5e-3, "lse": 1e-3, "dq": 5e-3, "dk": 5e-3, "dv": 5e-3},
    torch.bfloat16: {"o": 2e-2, "lse": 5e-3, "dq": 2e-2, "dk": 2e-2, "dv": 2e-2},
}

# The fp32 bounds hold while the largest attended score (after scale,
# soft-cap and ALiBi bias) stays within about 100: an fp32 score x carries a
# rounding error of up to half an ulp, |x| 2^-24, which exp(x - m) passes on
# to P, O and the gradients.  Above that the fp32 bound scales with the score
# magnitude: tolerance x fp32_score_factor(...) = max(1, max|x| / 100).
FP32_SCORE_REF = 100.0


def fp32_score_factor(q, k, scale=None, soft_cap=0.0, alibi_slope=None, causal=False, sliding_window=0):
    """max(1, max |attended score| / 100) for the fp32 tolerances."""
    qf, kf, _, sc, _ = orc._prep(q, k, k, scale, torch.float64)
    x, _ = orc.scores(qf, kf, sc, soft_cap, alibi_slope)
    ok = orc.allowed_mask(x.shape[-2], x.shape[-1], causal, sliding_window)
    return max(1.0, x.abs().masked_fill(~ok, 0.0).max().item() / FP32_SCORE_REF)


# One dict per checked output: test id, output name, dtype, err, max-abs, tol.
RECORDS = []


def draw(seed, b, hq, hkv, sq, skv, d, dtype, scale_inputs=1.0, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, sq, d, generator=g) * scale_inputs
    k = torch.randn(b, hkv, skv, d, generator=g) * scale_inputs
    v = torch.randn(b, hkv, skv, d, generator=g) * scale_inputs
    do = torch.randn(b, hq, sq, d, generator=g)
    cpu = [t.to(dtype) for t in (q, k, v, do)]
    return cpu, [t.to(device) for t in cpu]


def err_abs(x, ref):
    """(err, plain max-abs error) over the entries where ref is finite."""
    x = x.detach().to("cpu", torch.float64)
    ref = ref.detach().to("cpu", torch.float64)
    fin = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(x), fin), "non-finite pattern differs"
    if not bool(fin.any()):
        return 0.0, 0.0
    d = (x[fin] - ref[fin]).abs().max().item()
    return d / max(1.0, ref[fin].abs().max().item()), d


def err(x, ref):
    return err_abs(x, ref)[0]


def check(name, x, ref, dtype, report=None, factor=1.0):
    e, d = err_abs(x, ref)
    tol = TOL[dtype][name] * factor
    if report is not None:
        report[name] = e
    RECORDS.append({"test": os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0], "out": name,
                    "dtype": str(dtype).replace("torch.", ""), "err": e, "max_abs": d, "tol": tol})
    assert e <= tol, f"{name}: err {e:.3e} > tol {tol:.1e}"
    return e


def fwd_bwd(nfa, q, k, v, do, **kw):
    o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    dq, dk, dv = nfa.npu_flash_attention_backward(q, k, v, o, lse, do, **kw)
    torch.cuda.synchronize()
    return o, lse, dq, dk, dv


def oracle_fwd_bwd(q, k, v, do, causal=False, sliding_window=0, alibi_slope=None, scale=None, soft_cap=0.0,
                   dtype=torch.float64):
    sl = None if alibi_slope is None else alibi_slope.cpu()
    o, lse = orc.forward(q, k, v, causal, sliding_window, sl, scale, soft_cap, dtype)
    dq, dk, dv = orc.backward(q, k, v, do, causal, sliding_window, sl, scale, soft_cap, dtype)
    return o, lse, dq, dk, dv


def alibi_slopes(hq):
    """Config 5's slopes 2^(-8(h+1)/Hq)."""
    return torch.tensor([2.0 ** (-8.0 * (h + 1) / hq) for h in range(hq)], dtype=torch.float32)


def flops(b, hq, sq, skv, d, causal, window):
    pairs = orc.attention_pairs(sq, skv, causal, window)
    return 4.0 * d * pairs * b * hq, 10.0 * d * pairs * b * hq


def default_scale(d):
    return 1.0 / math.sqrt(d)
