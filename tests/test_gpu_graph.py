"""HIP graph capture of a whole training step (forward + backward).

The library launches only kernels on the caller's stream and allocates
nothing itself; the backward's work-queue counters are cleared by its Delta
kernel, not by a memset.  A step captured with torch.cuda.graph must
therefore replay to the eager results.  Each replay follows new inputs copied
into the captured buffers and an eager step with synchronisation, and is
compared bitwise with that eager step (the kernels are deterministic).
"""
import pytest
import torch

import npu_flash_attention as nfa
from gpu_helpers import check, draw, oracle_fwd_bwd

pytestmark = pytest.mark.gpu

CASES = {
    # name: (dtype, head_dim, Hq, Hkv, Sq, Skv, causal, window)
    "bf16_d128_staged": (torch.bfloat16, 128, 8, 2, 640, 640, True, 0),
    "fp16_d64_window": (torch.float16, 64, 6, 2, 500, 470, True, 100),
    "bf16_d256_staged": (torch.bfloat16, 256, 4, 2, 384, 384, True, 0),
    "fp32_d128": (torch.float32, 128, 4, 2, 300, 280, False, 0),
}


def _step(q, k, v, do, causal, window):
    o, lse = nfa.npu_flash_attention_forward(q, k, v, causal=causal, sliding_window=window, return_lse=True)
    dq, dk, dv = nfa.npu_flash_attention_backward(q, k, v, o, lse, do, causal=causal, sliding_window=window)
    return o, lse, dq, dk, dv


@pytest.mark.parametrize("name", list(CASES))
def test_graph_replays_match_eager(gpu_device, name):
    dtype, d, hq, hkv, sq, skv, causal, window = CASES[name]
    _, dev = draw(31, 1, hq, hkv, sq, skv, d, dtype, device=gpu_device)
    bufs = [t.clone() for t in dev]  # the captured input buffers

    side = torch.cuda.Stream(gpu_device)
    side.wait_stream(torch.cuda.current_stream(gpu_device))
    with torch.cuda.stream(side):
        _step(*bufs, causal, window)  # warm-up outside the capture
    torch.cuda.current_stream(gpu_device).wait_stream(side)
    torch.cuda.synchronize(gpu_device)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _step(*bufs, causal, window)
    torch.cuda.synchronize(gpu_device)

    for rep, seed in enumerate((41, 42, 43)):
        cpu, fresh = draw(seed, 1, hq, hkv, sq, skv, d, dtype, device=gpu_device)
        for b, f in zip(bufs, fresh):
            b.copy_(f)
        eager = _step(*fresh, causal, window)
        torch.cuda.synchronize(gpu_device)
        graph.replay()
        torch.cuda.synchronize(gpu_device)
        for nm, x, e in zip(("o", "lse", "dq", "dk", "dv"), outs, eager):
            assert torch.equal(x, e), f"{name} replay {rep}: {nm} differs from the eager step"
        if rep == 0:  # and the eager step itself against the oracle
            ref = oracle_fwd_bwd(*cpu, causal=causal, sliding_window=window)
            for nm, x, r in zip(("o", "lse", "dq", "dk", "dv"), eager, ref):
                check(nm, x, r, dtype)
