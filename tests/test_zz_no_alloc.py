"""kdec_adain_act_bwd_noalloc (the AdaIN + activation backward with its
scratch in a fixed device array) against kdec_adain_act_bwd on the same
inputs: calls in a row, each smaller than the one before and on another
kernel path -- rows of 70000 (longer than every row kernel: the chunked
passes, whose chunk partials, row means and alpha shares sit in the array),
rows of 61441 (one block per row holding the whole row; alpha shares of two
utterances), rows of 3000 (one block per row, one utterance, leaky) -- each
equal to the allocating entry point bit for bit (same kernels, same
summation order); and a call whose scratch exceeds the array is refused
before anything is launched.
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
    for N, C, L, act, tag in ((2, 64, 70000, ACT_SNAKE, "noalloc.0"),     # chunked passes
                              (2, 128, 61441, ACT_SNAKE, "noalloc.1"),    # one block per long row
                              (1, 64, 3000, ACT_LEAKY, "noalloc.2")):     # one block per row
        print(f"noalloc: N={N} C={C} L={L} act={act}", flush=True)
        (a, b) = run_pair(ctx, N, C, L, act, tag)
        for u, v in zip(a, b):
            assert np.array_equal(u, v)
    # beyond the scratch array: two utterances of 2^20 rows with alpha grads
    # keep 8 MiB of alpha-grad shares alone; refused with the sizes in the
    # message before anything launches (the buffers are real and sized for
    # the call all the same)
    N, C, L = 2, 1 << 20, 4
    x, dy, dx = (torch.zeros(N * C * L, device="cuda") for _ in range(3))
    st = torch.zeros(N * C, 2, device="cuda")
    gam, bet, alpha, dalpha = (torch.zeros(C, device="cuda") for _ in range(4))
    dgam, dbet = (torch.zeros(N * C, device="cuda") for _ in range(2))
    with pytest.raises(native.KdecError, match="scratch"):
        ctx.call("kdec_adain_act_bwd_noalloc", P(x), C * L, P(st), P(gam), P(bet), 0, ACT_SNAKE, 0.0,
                 P(alpha), P(dy), C * L, None, 0, P(dx), C * L, P(dgam), P(dbet), C, P(dalpha), N, C, L)
