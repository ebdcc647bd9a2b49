"""GPU tests of the torch.library operators (flexatt_ops).

* torch.library.opcheck on both operators: schema, fake implementation
  against the real outputs, autograd registration, AOT dispatch;
* the operator path is bitwise identical to npu_flex_attention (forward and
  the three gradients), and matches the oracle;
* torch.compile(fullgraph=True) of a loss around the operator (aot_eager
  backend: the traced graph runs the same kernels, no graph break) gives the
  eager gradients, bitwise.
"""
import pytest
import torch

import flexatt_ops
import npu_flash_attention as nfa
from gpu_helpers import alibi_slopes, check, draw, oracle_fwd_bwd

pytestmark = pytest.mark.gpu


def _inputs(seed, dtype=torch.bfloat16, hq=4, hkv=2, sq=67, sk=93, d=64, grad=False):
    cpu, dev = draw(seed, 2, hq, hkv, sq, sk, d, dtype)
    if grad:
        dev = [t.clone().requires_grad_(i < 3) for i, t in enumerate(dev)]
    return cpu, dev


def test_opcheck_forward(gpu_device):
    _, (q, k, v, _) = _inputs(1, grad=True)
    torch.library.opcheck(torch.ops.flexatt.fwd.default, (q, k, v, None, 0.125, True, 0, 0.0))
    slopes = alibi_slopes(4).to(gpu_device)
    torch.library.opcheck(torch.ops.flexatt.fwd.default, (q, k, v, slopes, 0.1, False, 19, 25.0))


def test_opcheck_backward(gpu_device):
    _, (q, k, v, do) = _inputs(2)
    o, lse = torch.ops.flexatt.fwd(q, k, v, None, 0.125, True, 0, 0.0)
    torch.library.opcheck(torch.ops.flexatt.bwd.default, (do, q, k, v, o, lse, None, 0.125, True, 0, 0.0))


@pytest.mark.parametrize("kw", [dict(causal=True), dict(causal=False, sliding_window=23, soft_cap=30.0, scale=0.09)])
def test_matches_autograd_function(gpu_device, kw):
    cpu, (q, k, v, do) = _inputs(3, grad=True)
    o = flexatt_ops.attention(q, k, v, **kw)
    o.backward(do)
    grads = [t.grad.clone() for t in (q, k, v)]
    for t in (q, k, v):
        t.grad = None
    o_ref = nfa.npu_flex_attention(q, k, v, **kw)
    o_ref.backward(do)
    assert torch.equal(o, o_ref)
    for name, g, t in zip(("dq", "dk", "dv"), grads, (q, k, v)):
        assert torch.equal(g, t.grad), f"{name} differs from npu_flex_attention"
    ref = oracle_fwd_bwd(*cpu, **kw)
    check("o", o, ref[0], torch.bfloat16)
    for name, g, r in zip(("dq", "dk", "dv"), grads, ref[2:]):
        check(name, g, r, torch.bfloat16)


def test_documents_through_the_operator(gpu_device):
    _, (q, k, v, do) = _inputs(5, hq=4, hkv=2, sq=90, sk=90, grad=True)
    ids = torch.tensor([[0] * 30 + [1] * 45 + [2] * 15, [4] * 90], dtype=torch.int32, device=gpu_device)
    o = flexatt_ops.attention(q, k, v, causal=True, document_ids=ids)
    o.backward(do)
    grads = [t.grad.clone() for t in (q, k, v)]
    for t in (q, k, v):
        t.grad = None
    o_ref = nfa.npu_flex_attention(q, k, v, causal=True, document_ids=ids)
    o_ref.backward(do)
    assert torch.equal(o, o_ref)
    for g, t in zip(grads, (q, k, v)):
        assert torch.equal(g, t.grad)


def test_compile_fullgraph(gpu_device):
    torch._dynamo.reset()
    _, (q, k, v, do) = _inputs(4, dtype=torch.float16, grad=True)
    w = torch.linspace(-1.0, 1.0, q.shape[-1], device=gpu_device)

    def loss_fn(q, k, v):
        o = flexatt_ops.attention(q, k, v, causal=True, soft_cap=20.0)
        return (o.float() * w).sum()

    eager = loss_fn(q, k, v)
    g_eager = torch.autograd.grad(eager, (q, k, v))
    compiled = torch.compile(loss_fn, backend="aot_eager", fullgraph=True)
    out = compiled(q, k, v)
    g_comp = torch.autograd.grad(out, (q, k, v))
    assert torch.equal(out, eager)
    for a, b in zip(g_comp, g_eager):
        assert torch.equal(a, b)
