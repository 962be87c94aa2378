"""tgohip_probe_peaks, the benchmark's measure of what the box reaches beside the
published peaks: plausible rates (a read cannot beat the published 8 TB/s by much, an MFMA
loop cannot beat 2.5 PFLOP/s) and a refusal that names its arguments."""
import pytest

import tgo_amd

pytestmark = pytest.mark.gpu


def test_probe_peaks_are_plausible(ctx):
    read_gbps, mfma_tflops = ctx.probe_peaks(256 << 20, 3)
    print("probe: read %.0f GB/s, f16 MFMA %.0f TFLOP/s" % (read_gbps, mfma_tflops), flush=True)
    assert 500 < read_gbps < 9000, read_gbps
    assert 200 < mfma_tflops <= 2500, mfma_tflops


def test_probe_peaks_refuses_a_small_buffer(ctx):
    with pytest.raises(tgo_amd.TgoError, match="read_bytes"):
        ctx.probe_peaks(1000, 3)
    with pytest.raises(tgo_amd.TgoError, match="reps"):
        ctx.probe_peaks(2 << 20, 0)
