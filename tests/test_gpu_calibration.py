"""The same-run MFMA rate calibration bench.py reports beside the published
peak (fa_mfma_peak): plausible rate and clock, and the operand pool option."""
import pytest

from test_gpu_parity import fa  # noqa: F401 (fa: fixture)

pytestmark = pytest.mark.gpu


def test_mfma_peak_is_plausible(fa):
    import torch

    print("calibration", flush=True)
    r = fa.mfma_peak(mfma_per_wave=1024, launches=3)
    print(r)
    # at most the published 2.5 PFLOP/s (2.4 GHz), at least a quarter of it
    assert 600.0 < r["tflops"] < 2500.0 * 1.03
    assert 0.5 < r["clock_ghz"] < 2.6
    # the rate follows the clock: 256 CUs x 4096 FLOP per clock
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert r["tflops"] == pytest.approx(cus * 4096 * r["clock_ghz"] * 1e9 / 1e12, rel=0.25)
    ops = torch.zeros(4096, dtype=torch.bfloat16, device="cuda")
    r0 = fa.mfma_peak(mfma_per_wave=1024, launches=3, operands=ops)
    assert 600.0 < r0["tflops"] < 2500.0 * 1.03
    with pytest.raises(ValueError):
        fa.mfma_peak(operands=ops[:100])
