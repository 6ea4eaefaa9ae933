"""ponni_forward_timed: the same output as ponni_forward, and the two events
stamped with a positive kernel duration, on every kernel family; null
events are rejected before any device work."""
import pytest

import ponni_amd as P
from ponni_amd import configs as C


@pytest.mark.gpu
@pytest.mark.parametrize("path,cfg", [("generic", "c2"), ("narrow", "c1"), ("mfma", "c2"), ("fused", "c2")])
def test_timed_forward_matches_and_stamps_events(path, cfg, cuda):
    import torch

    from bench import HipEvents

    c = C.CONFIGS[cfg]
    m = P.create_inference_model(*c.layers(True), path=path)
    B = 70_001
    x = torch.empty((c.n_in, B), dtype=torch.float32, device=cuda)
    P.fill_synthetic(x, 5, C.INPUT_TAG, "normal", 0.0, 1.0)
    y0 = torch.full((c.n_out, B), float("nan"), device=cuda)
    y1 = torch.full((c.n_out, B), float("nan"), device=cuda)
    stream = torch.cuda.current_stream().cuda_stream
    m.forward_raw(x.data_ptr(), B, y0.data_ptr(), B, B, stream)
    ev = HipEvents()
    a, b = ev.create(), ev.create()
    try:
        print(f"timed forward: path={path} B={B}", flush=True)
        m.forward_raw_timed(x.data_ptr(), B, y1.data_ptr(), B, B, stream, a, b)
        torch.cuda.synchronize()
        ms = ev.elapsed_ms(a, b)
    finally:
        ev.destroy(a)
        ev.destroy(b)
    assert torch.equal(y0, y1)
    assert 0.0 < ms < 1000.0, ms


def test_timed_forward_rejects_null_events():
    layers = C.c1_layers()
    m = P.create_inference_model(*layers)
    with pytest.raises(P.PonniError) as e:
        m.forward_raw_timed(0, 1, 0, 1, 1, 0, 0, 0)
    assert e.value.status == P._abi.PONNI_ERR_INVALID_ARGUMENT


@pytest.mark.gpu
def test_measured_peaks_are_plausible(cuda):
    """ponni_measure_peaks: every rate positive and under MI355X's published
    peak (8 TB/s HBM, 2.5 PFLOP/s fp16 and 157.3 TFLOP/s fp32 dense MFMA) with
    a margin for clocks above the nominal one."""
    import ctypes

    from ponni_amd import _abi as A

    pk = A.Peaks()
    print("measure peaks", flush=True)
    A.check(A.lib().ponni_measure_peaks(ctypes.byref(pk), None))
    assert 1000.0 < pk.hbm_copy_gbps < 1.2 * 8000.0, pk.hbm_copy_gbps
    assert 1000.0 < pk.hbm_read_gbps < 1.2 * 8000.0, pk.hbm_read_gbps
    assert 500.0 < pk.mfma_f16_tflops < 1.2 * 2500.0, pk.mfma_f16_tflops
    assert 30.0 < pk.mfma_f32_tflops < 1.2 * 157.3, pk.mfma_f32_tflops


def test_measured_peaks_rejects_null_output():
    from ponni_amd import _abi as A

    assert A.lib().ponni_measure_peaks(None, None) == A.PONNI_ERR_INVALID_ARGUMENT
