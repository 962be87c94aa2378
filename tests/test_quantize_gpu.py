"""The device quantizers behind tgohip_weight_f32 / tgohip_weight_upload_f32
(weights.Load's quantize-then-upload, weights/weights.go:694-743; quantizeInto,
weights/convert.go:206-217) against the host quantizers tgohip_quantize_int8 /
tgohip_quantize_int4, whose codes the CPU tests pin to the reference's vectors: the same
plane quantized both ways and dequantized on the device must give the same f32 bits.
The planes carry what the host rules decide case by case: an all-zero group, NaN first
in a group and inside one, infinities, values past f16's range, values that divide
below f16's normal range, and exact half-way ties (round half to even). The whole-model
path (the loader quantizing every port on the device) is tests/test_checkpoint_gpu.py,
against ports quantized on the host."""
import numpy as np
import pytest

import tgo_amd

pytestmark = pytest.mark.gpu


def plane(K, N, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(K * N) * 0.05).astype(np.float32)
    w[0:128] = 0.0                                          # an all-zero group
    w[128] = np.nan                                         # NaN first in a group
    w[256 + 17] = np.nan                                    # NaN inside one
    w[384 + 3], w[384 + 90] = np.inf, -np.inf               # infinities
    w[512 + 5] = 1e30                                       # past f16's range
    w[640:768] = (rng.standard_normal(128) * 1e-30).astype(np.float32)  # below f16 normal
    # exact ties at scale 1/16: int8 groups of 32 each peaking at 127/16 ...
    m = rng.integers(-100, 100, 128)
    g = (m + 0.5) / 16.0
    g[0::32] = 127.0 / 16.0
    w[768:896] = g.astype(np.float32)
    # ... and one int4 group of 128 spanning [0, 15/16]
    t = rng.integers(0, 14, 128) + 0.5
    t[0], t[1] = 0.0, 15.0
    w[896:1024] = (t / 16.0).astype(np.float32)
    return w


@pytest.mark.parametrize("form", [tgo_amd.FORM_I8, tgo_amd.FORM_I4_TGO])
@pytest.mark.parametrize("KN", [(256, 512), (4096, 1024)])
def test_device_quantizer_equals_the_host_quantizer(ctx, torch_gpu, form, KN):
    torch = torch_gpu
    K, N = KN
    w = plane(K, N, 7 + form)
    if form == tgo_amd.FORM_I8:
        q, s = tgo_amd.quantize_int8(w)
        host = ctx.weight_upload(form, K, N, q, s)
    else:
        c, s, z = tgo_amd.quantize_int4(w)
        host = ctx.weight_upload(form, K, N, c, s, z)
    dev = ctx.weight_upload_f32(form, K, N, w)
    try:
        a = torch.empty((K, N), dtype=torch.float32, device="cuda")
        b = torch.empty((K, N), dtype=torch.float32, device="cuda")
        ctx.dequant(host, a)
        ctx.dequant(dev, b)
        torch.cuda.synchronize()
        ha, hb = a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32)
        assert np.array_equal(ha, hb), int(np.count_nonzero(ha != hb))
        # the planted ties dequantize to whole sixteenths, the even neighbour
        lo = 768 if form == tgo_amd.FORM_I8 else 896
        got = a.cpu().numpy().ravel()[lo:lo + 128].astype(np.float64) * 16.0
        want = w[lo:lo + 128].astype(np.float64) * 16.0
        assert np.array_equal(got, np.round(want))  # numpy rounds half to even
    finally:
        ctx.weight_free(host)
        ctx.weight_free(dev)


def test_weight_f32_refuses_other_forms(ctx, torch_gpu):
    w = np.zeros(256 * 512, np.float32)
    for form in (tgo_amd.FORM_F16, tgo_amd.FORM_I4_SYM):
        with pytest.raises(tgo_amd.TgoError, match="quantizes to I8 or I4_TGO"):
            ctx.weight_upload_f32(form, 256, 512, w)
