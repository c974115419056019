"""kdec_adain_act_bwd_noalloc (the AdaIN + activation backward with its
scratch in a fixed device array) against kdec_adain_act_bwd on the same
inputs: two calls in a row, the second with a smaller input and on the other
kernel path (chunked passes for rows longer than 49152, then one block per
row), each equal to the allocating entry point bit for bit (same kernels,
same summation order); and a call beyond the array's size is refused before
anything is launched.
"""
import ctypes

import numpy as np
import pytest

from brosoundml_amd import synth

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

ACT_LEAKY, ACT_SNAKE = 1, 2


def P(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def run_pair(ctx, N, C, L, act, tag):
    x = dev(synth.normal(f"{tag}.x", (N, C, L), 1.3))
    dy = dev(synth.normal(f"{tag}.dy", (N, C, L)))
    res = dev(synth.normal(f"{tag}.r", (N, C, L)))
    gb = dev(synth.normal(f"{tag}.gb", (N, 2 * C), 0.3))
    alpha = dev(synth.uniform(f"{tag}.alpha", (C,), 0.5, 2.0))
    st = torch.empty(N * C, 2, device="cuda")
    ctx.call("kdec_instnorm_stats", P(x), C * L, N, C, L, 1e-5, P(st))
    g_p, b_p = P(gb), ctypes.c_void_p(gb.data_ptr() + 4 * C)
    outs = []
    for name in ("kdec_adain_act_bwd", "kdec_adain_act_bwd_noalloc"):
        dx = torch.empty_like(x)
        dgb = torch.empty(N, 2 * C, device="cuda")
        da = torch.zeros(C, device="cuda")
        ctx.call(name, P(x), C * L, P(st), g_p, b_p, 2 * C, act, 0.2, P(alpha), P(dy), C * L, P(res), C * L,
                 P(dx), C * L, P(dgb), ctypes.c_void_p(dgb.data_ptr() + 4 * C), 2 * C,
                 P(da) if act == ACT_SNAKE else None, N, C, L)
        torch.cuda.synchronize()
        outs.append((dx.cpu().numpy(), dgb.cpu().numpy(), da.cpu().numpy()))
    return outs


def test_noalloc_equals_allocating_backward():
    from brosoundml_amd import native
    ctx = native.Context(0)
    # first call: rows of 61441 (chunked passes), alpha grads over 2 utterances
    (a, b) = run_pair(ctx, 2, 128, 61441, ACT_SNAKE, "noalloc.1")
    for u, v in zip(a, b):
        assert np.array_equal(u, v)
    # second call, smaller: rows of 3000 (one block per row), leaky
    (a, b) = run_pair(ctx, 1, 64, 3000, ACT_LEAKY, "noalloc.2")
    for u, v in zip(a, b):
        assert np.array_equal(u, v)
    # beyond the scratch array: 2^21 rows need 8 MiB of alpha-grad shares
    # alone; refused with the sizes in the message before anything launches
    # (the buffers are real and sized for the call all the same)
    C, L = 1 << 21, 4
    x = torch.zeros(C * L, device="cuda")
    big = [torch.zeros(C * L, device="cuda") for _ in range(2)]
    st = torch.zeros(C, 2, device="cuda")
    small = [torch.zeros(C, device="cuda") for _ in range(6)]
    with pytest.raises(native.KdecError, match="scratch"):
        ctx.call("kdec_adain_act_bwd_noalloc", P(x), C * L, P(st), P(small[0]), P(small[1]), 0, ACT_SNAKE, 0.0,
                 P(small[2]), P(big[0]), C * L, None, 0, P(big[1]), C * L, P(small[3]), P(small[4]), 0,
                 P(small[5]), 1, C, L)
