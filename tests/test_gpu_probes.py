"""The measurement probes run on the GPU and report plausible rates: the
matrix-core probes complete and leave the sink untouched (the folded products
never equal the sentinel), and bench.py's measured peaks are positive and
below twice the published figures."""
import ctypes

import pytest
import torch

from nv4 import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_probe_kernels_run():
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    sink = torch.full((1024,), 7, dtype=torch.int32, device=DEV)
    for kind in (0, 1, 2):
        assert lib.nv4_probe_mfma(kind, 10, 64, ctypes.c_void_p(sink.data_ptr()), stream) == 0
    buf = torch.ones(1 << 22, dtype=torch.uint8, device=DEV)
    assert lib.nv4_probe_read(ctypes.c_void_p(buf.data_ptr()), buf.numel(), ctypes.c_void_p(sink.data_ptr()),
                              stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(sink.cpu(), torch.full((1024,), 7, dtype=torch.int32))


def test_bench_measured_peaks_are_plausible():
    import bench
    peaks = bench.measured_peaks(torch, torch.device(DEV))
    print(peaks, flush=True)
    for key in ("int8_mfma_tops", "fp8_mfma_tops", "fp6_mfma_tops", "hbm_read_gbs"):
        assert 0 < peaks[key] < 2 * peaks["published"][key], key


def test_hardware_bf16_rounding_is_rne_for_every_input():
    """Every bf16 the kernels produce comes from the hardware conversion;
    over all 2^32 fp32 inputs (NaN skipped) it gives the integer
    round-to-nearest-even bits, denormals included."""
    lib = _lib.load()
    bad = torch.zeros(1, dtype=torch.int64, device=DEV)
    assert lib.nv4_probe_bf16_rne(ctypes.c_void_p(bad.data_ptr()),
                                  ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
    torch.cuda.synchronize()
    assert int(bad.item()) == 0
