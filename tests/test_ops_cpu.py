"""The torch.library operators (flexatt_ops) without a GPU: registration,
fake (meta) shapes, dtypes and strides, the shape assertions at trace time,
the autograd formula's wiring, and that a traced graph keeps each kernel
call as one node.  Real kernel calls are covered by tests/test_gpu_ops.py."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

import flexatt_ops


def fake_qkv(mode, B=2, Hq=8, Hkv=2, Sq=40, Sk=56, D=64, dtype=torch.bfloat16, grad=False):
    with mode:
        q = torch.empty(B, Hq, Sq, D, dtype=dtype, device="cuda", requires_grad=grad)
        k = torch.empty(B, Hkv, Sk, D, dtype=dtype, device="cuda", requires_grad=grad)
        v = torch.empty(B, Hkv, Sk, D, dtype=dtype, device="cuda", requires_grad=grad)
    return q, k, v


def test_ops_registered():
    assert hasattr(torch.ops.flexatt, "fwd")
    assert hasattr(torch.ops.flexatt, "bwd")
    schema = str(torch.ops.flexatt.fwd.default._schema)
    assert "Tensor q" in schema and "float scale" in schema and "bool causal" in schema


def test_fake_forward_shapes():
    mode = FakeTensorMode()
    q, k, v = fake_qkv(mode)
    with mode:
        o, lse = torch.ops.flexatt.fwd(q, k, v, None, 0.125, True, 0, 0.0)
    assert o.shape == q.shape and o.dtype == q.dtype and o.is_contiguous()
    assert lse.shape == (2, 8, 40) and lse.dtype == torch.float32
    assert o.device.type == "cuda"


def test_fake_backward_shapes():
    mode = FakeTensorMode()
    q, k, v = fake_qkv(mode, dtype=torch.float16)
    with mode:
        o, lse = torch.ops.flexatt.fwd(q, k, v, None, 0.125, False, 7, 30.0)
        dq, dk, dv = torch.ops.flexatt.bwd(torch.empty_like(o), q, k, v, o, lse, None, 0.125, False, 7, 30.0)
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
    assert dq.dtype == dk.dtype == dv.dtype == torch.float16


def test_fake_shape_assertions():  # npu_flash_attention.py:620-622
    mode = FakeTensorMode()
    with mode:
        q = torch.empty(1, 6, 16, 64, device="cuda", dtype=torch.bfloat16)
        k = torch.empty(1, 4, 16, 64, device="cuda", dtype=torch.bfloat16)
        k2 = torch.empty(1, 2, 16, 32, device="cuda", dtype=torch.bfloat16)
        with pytest.raises(AssertionError):
            torch.ops.flexatt.fwd(q, k, k, None, 0.1, False, 0, 0.0)  # Hq % Hkv
        with pytest.raises(AssertionError):
            torch.ops.flexatt.fwd(q, k2, k2, None, 0.1, False, 0, 0.0)  # head dims


def test_meta_autograd_wiring():
    """Backward through the registered formula produces gradients of the
    inputs' shapes (meta tensors: the fake operators run, no device needed)."""
    q = torch.empty(2, 8, 40, 64, dtype=torch.bfloat16, device="meta", requires_grad=True)
    k = torch.empty(2, 2, 56, 64, dtype=torch.bfloat16, device="meta", requires_grad=True)
    v = torch.empty(2, 2, 56, 64, dtype=torch.bfloat16, device="meta", requires_grad=True)
    o = flexatt_ops.attention(q, k, v, causal=True, alibi_slope=torch.ones(8, device="meta"))
    o.float().sum().backward()
    assert q.grad.shape == q.shape and k.grad.shape == k.shape and v.grad.shape == v.shape


def test_traced_graph_has_single_kernel_nodes():
    """make_fx with fake tensors (what torch.compile's tracer does): each
    kernel call appears as one flexatt node and nothing is decomposed."""
    def fn(q, k, v):
        return flexatt_ops.attention(q, k, v, causal=True, soft_cap=20.0) * 2.0

    mode = FakeTensorMode()
    q, k, v = fake_qkv(mode)
    gm = make_fx(fn, tracing_mode="fake")(q, k, v)
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    assert sum("flexatt.fwd" in t for t in targets) == 1, targets


def test_meta_autograd_with_documents():
    q = torch.empty(1, 4, 24, 32, dtype=torch.float16, device="meta", requires_grad=True)
    k = torch.empty(1, 2, 24, 32, dtype=torch.float16, device="meta", requires_grad=True)
    v = torch.empty(1, 2, 24, 32, dtype=torch.float16, device="meta", requires_grad=True)
    doc = torch.empty(1, 24, 2, dtype=torch.int32, device="meta")
    o, lse = torch.ops.flexatt.fwd(q, k, v, None, 0.2, True, 0, 0.0, doc)
    o.float().sum().backward()
    assert o.shape == q.shape and k.grad.shape == k.shape
