"""GPU checks of the benchmark's box-calibration entries (gonn_hip_calib_*)
and of the device-timed fp64 backward bench entry: they run, and what they
report is physically plausible for an MI355X.

The calibration loop's rate cannot pass the dense bf16 peak at the clock it
reports (1024 FLOP per cycle per SIMD, 1024 SIMDs), so rate / clock is
checked against that bound in both operand modes; the clock probe, run
beside a busy stream, reads the shader clock against the fixed 100 MHz
counter."""
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

FLOP_PER_CLOCK = 1024 * 1024  # per cycle over the device: 1024 SIMDs x 1024 bf16 FLOP


@pytest.mark.parametrize("random", [False, True])
def test_calib_mfma_rate_within_the_clock_bound(random):
    from gonn_amd import hip
    tflops, ghz = hip.calib_mfma(random)
    print(f"[calib] random={random}: {tflops:.1f} TFLOP/s at {ghz:.3f} GHz", flush=True)
    assert 0.5 < ghz < 3.0
    assert 100.0 < tflops
    # at most the peak rate at the measured clock (3% for timing granularity)
    assert tflops * 1e12 <= 1.03 * FLOP_PER_CLOCK * ghz * 1e9


def test_calib_clock_probe_beside_work():
    from gonn_amd import hip
    side = torch.cuda.Stream()
    a = torch.randn(4096, 4096, device="cuda")
    torch.cuda.synchronize()
    hip.calib_clock_start(20.0, stream=side)
    for _ in range(20):
        a = a @ a.T * 1e-3
    side.synchronize()
    torch.cuda.synchronize()
    ghz = hip.calib_clock_read()
    print(f"[calib] shader clock beside a GEMM stream: {ghz:.3f} GHz", flush=True)
    assert 0.5 < ghz < 3.0


def test_calib_argument_errors():
    from gonn_amd import hip
    with pytest.raises(hip.GonnHipError):
        hip.calib_clock_start(0.0)
    with pytest.raises(hip.GonnHipError):
        hip.calib_clock_start(1e9)


def test_bench_entry_times_the_fp64_backward():
    """BenchFlashAttnF64Bwd: the exact-mode backward, timed on the device;
    refused outside the f64 mode (the MFMA modes' backward is attn_bwd)."""
    from gonn_amd import hip
    prev = hip.AttnMode()
    try:
        hip.SetAttnMode("f64")
        ms = hip.BenchFlashAttnF64Bwd(4, 256, 64, 3, True)
        assert ms > 0.0, ms
        hip.SetAttnMode("fp32")
        with pytest.raises(hip.GonnHipError):
            hip.BenchFlashAttnF64Bwd(4, 256, 64, 3, True)
    finally:
        hip.SetAttnMode(prev)
