"""tgohip_linear_noalloc -- the linear whose split-K partials live in the library's
static device workspace -- against tgohip_linear, through the C ABI: the same kernels and
splits, so the outputs are equal to the bit. Two calls in a row, the second with fewer
rows, so the second runs on the array the first left behind; every call here splits K
(tgohip_linear_workspace says so), so both use the array; an empty batch launches nothing;
a call needing more than the array holds is refused; and calls captured into a HIP graph
replay to the same bits as eager calls."""
import numpy as np
import pytest

import oracle
import tgo_amd

pytestmark = pytest.mark.gpu


def weight(ctx, form, K, N, seed):
    return ctx.weight_synth(form, K, N, seed, 7, 0.02)


@pytest.mark.parametrize("form,K,N,Ms,xf", [
    (tgo_amd.FORM_I4_SYM, 12288, 4096, (256, 40), tgo_amd.F16),   # pipelined kernel, 8 splits both
    (tgo_amd.FORM_I4_SYM, 12288, 4096, (1024, 512), tgo_amd.F16),  # 4 then 8 splits, 64 MiB each
    (tgo_amd.FORM_I8, 4096, 6144, (64, 48), tgo_amd.F16),          # 8 splits both
    (tgo_amd.FORM_F16, 4096, 4096, (200, 33), tgo_amd.F32),       # gemm_kernel, 16 splits, f32 x
    (tgo_amd.FORM_I4_TGO, 4096, 12288, (130, 65), tgo_amd.F16),    # 3 then 4 splits
    (tgo_amd.FORM_I4_SYM, 4096, 4096, (128, 64), tgo_amd.F16X2),   # exact kernel, 8 splits both
])
def test_noalloc_linear_equals_linear(ctx, torch_gpu, form, K, N, Ms, xf):
    torch = torch_gpu
    h = weight(ctx, form, K, N, 3 + form)
    try:
        for M in Ms:
            print("no-alloc linear: form %d [%d,%d] M=%d" % (form, K, N, M), flush=True)
            assert ctx.linear_workspace(h, M, x_dtype=xf) > 0, "this call should split K"
            g = torch.Generator(device="cuda").manual_seed(M)
            x = torch.randn(M, K, device="cuda", generator=g)
            if xf == tgo_amd.F16:
                x = x.half()
            elif xf == tgo_amd.F16X2:  # the activation pair: f16 hi plane, then lo plane
                hi = x.half()
                x = torch.cat([hi.reshape(-1), (x - hi.float()).half().reshape(-1)])
            want = torch.full((M, N), float("nan"), device="cuda")
            got = torch.full((M, N), float("nan"), device="cuda")
            ctx.linear(h, x, M, want, x_dtype=xf)
            ctx.linear_noalloc(h, x, M, got, x_dtype=xf)
            torch.cuda.synchronize()
            assert torch.isfinite(want).all()
            assert torch.equal(got, want), (M, (got - want).abs().max().item())
    finally:
        ctx.weight_free(h)


def test_noalloc_linear_refuses_beyond_its_workspace(ctx, torch_gpu):
    """f32 activations over [12288, 4096] at M = 2100: two partial planes of 34 MiB."""
    torch = torch_gpu
    h = weight(ctx, tgo_amd.FORM_F16, 12288, 4096, 5)
    try:
        x = torch.zeros(2100, 12288, device="cuda")
        y = torch.zeros(2100, 4096, device="cuda")
        with pytest.raises(tgo_amd.TgoError, match="static workspace holds 67108864"):
            ctx.linear_noalloc(h, x, 2100, y)
        ctx.linear_noalloc(h, x, 2000, y)  # two planes of 32 MiB fit
        torch.cuda.synchronize()
    finally:
        ctx.weight_free(h)


def test_noalloc_linear_empty_batch_launches_nothing(ctx, torch_gpu):
    """M = 0 (an empty batch in a serving loop): both linear entry points return at once,
    with nothing written and no split-K arithmetic over zero tiles."""
    torch = torch_gpu
    h = weight(ctx, tgo_amd.FORM_I4_SYM, 4096, 6144, 9)
    try:
        assert ctx.linear_workspace(h, 0, x_dtype=tgo_amd.F16) == 0
        x = torch.zeros(1, 4096, device="cuda").half()
        y = torch.full((1, 6144), 7.0, device="cuda")
        ctx.linear(h, x, 0, y, x_dtype=tgo_amd.F16)
        ctx.linear_noalloc(h, x, 0, y, x_dtype=tgo_amd.F16)
        torch.cuda.synchronize()
        assert bool((y == 7.0).all())
    finally:
        ctx.weight_free(h)


def test_noalloc_linear_replays_under_graph_capture(ctx, torch_gpu):
    """The allocation-free linear is meant for code under HIP graph capture. Captured on a
    torch stream (the library launching there), a graph of two calls -- symmetric int4 over
    f16 activations and over an activation pair, both 8-way split-K at 128 rows, so both
    use the static workspace -- is replayed five times, with eager work and a
    synchronization between replays and new inputs written before each. Every replay's
    outputs equal an eager tgohip_linear of the same inputs to the bit."""
    torch = torch_gpu
    K = N = 4096
    M = 128
    h = ctx.weight_synth(tgo_amd.FORM_I4_SYM, K, N, 23, 7, 0.02)
    try:
        assert ctx.linear_workspace(h, M, x_dtype=tgo_amd.F16) > 0
        assert ctx.linear_workspace(h, M, x_dtype=tgo_amd.F16X2) > 0
        x16 = torch.zeros(M, K, device="cuda").half()
        xp = torch.zeros(2 * M * K, device="cuda").half()
        y16 = torch.zeros(M, N, device="cuda")
        yp = torch.zeros(M, N, device="cuda")
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        ctx.set_stream(s.cuda_stream)
        try:
            with torch.cuda.graph(g, stream=s):
                ctx.linear_noalloc(h, x16, M, y16, x_dtype=tgo_amd.F16)
                ctx.linear_noalloc(h, xp, M, yp, x_dtype=tgo_amd.F16X2)
        finally:
            ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        gen = torch.Generator(device="cuda").manual_seed(5)
        for rep in range(5):
            print("graph replay %d" % rep, flush=True)
            x = torch.randn(M, K, device="cuda", generator=gen)
            x16.copy_(x.half())
            hi = x.half()
            xp.copy_(torch.cat([hi.reshape(-1), (x - hi.float()).half().reshape(-1)]))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            w16 = torch.full((M, N), float("nan"), device="cuda")
            wp = torch.full((M, N), float("nan"), device="cuda")
            ctx.linear(h, x16, M, w16, x_dtype=tgo_amd.F16)
            ctx.linear(h, xp, M, wp, x_dtype=tgo_amd.F16X2)
            torch.cuda.synchronize()
            assert torch.isfinite(w16).all() and torch.isfinite(wp).all()
            assert torch.equal(y16, w16), (rep, (y16 - w16).abs().max().item())
            assert torch.equal(yp, wp), (rep, (yp - wp).abs().max().item())
        del g
    finally:
        ctx.weight_free(h)
