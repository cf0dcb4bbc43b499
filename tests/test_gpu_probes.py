"""GPU tests of the peak probes (fa_probe_launch), the measurement aid behind
bench.py's ``extra.measured_peaks``: the copy probe copies exactly, the MFMA
probes' checksums are finite, equal across waves and launches, and the rates
they give stay within loose bounds of the MI355X data sheet (a rate above it
would mean wrong FLOP accounting)."""
from __future__ import annotations

import numpy as np
import pytest

import flash_attention_amd as fa

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    fa.init()


def _torch():
    import torch
    return torch


def _num_cus(torch) -> int:
    return torch.cuda.get_device_properties(0).multi_processor_count


def test_copy_probe_copies_every_element():
    torch = _torch()
    for nbytes in (32, 4096 + 32, (64 << 20) + 96):   # one element, ragged tails, 32 MiB halves
        half = nbytes // 32 * 4
        buf = torch.full((nbytes // 4 + 4,), -1.0, dtype=torch.float32, device="cuda")
        buf[:half] = torch.arange(half, dtype=torch.float32, device="cuda")
        stream = torch.cuda.current_stream().cuda_stream
        work = fa.probe_launch(fa.PROBE_COPY, stream, buf.data_ptr(), nbytes)
        torch.cuda.synchronize()
        assert work == 32.0 * (nbytes // 32)
        got = buf.cpu().numpy()
        assert np.array_equal(got[half:2 * half], np.arange(half, dtype=np.float32)), nbytes
        assert np.all(got[2 * half:] == -1.0), "wrote past the destination half"


def test_read_probe_reads_and_writes_nothing():
    torch = _torch()
    nbytes = (64 << 20) + 96
    buf = torch.rand(nbytes // 4 + 8, dtype=torch.float32, device="cuda")
    before = buf.cpu().numpy()
    work = fa.probe_launch(fa.PROBE_READ, torch.cuda.current_stream().cuda_stream, buf.data_ptr(), nbytes)
    torch.cuda.synchronize()
    assert work == 16.0 * (nbytes // 32)
    assert np.array_equal(buf.cpu().numpy(), before), "the read stream wrote to the buffer"


@pytest.mark.parametrize("kind", [fa.PROBE_MFMA_F32_32X32X2, fa.PROBE_MFMA_F32_16X16X4, fa.PROBE_MFMA_BF16_16X16X32,
                                  fa.PROBE_MFMA_BF16_32X32X16])
def test_mfma_probe_checksums(kind):
    torch = _torch()
    waves = 8 * _num_cus(torch) * 4
    buf = torch.zeros(waves + 64, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    sums = []
    for _ in range(2):
        buf[:waves] = 0.0
        work = fa.probe_launch(kind, stream, buf.data_ptr(), buf.numel() * 4, 16)
        torch.cuda.synchronize()
        per_iter = {fa.PROBE_MFMA_F32_32X32X2: 2 * 32 * 32 * 2 * 4, fa.PROBE_MFMA_F32_16X16X4: 2 * 16 * 16 * 4 * 8,
                    fa.PROBE_MFMA_BF16_16X16X32: 2 * 16 * 16 * 32 * 16,
                    fa.PROBE_MFMA_BF16_32X32X16: 2 * 32 * 32 * 16 * 4}[kind]   # FLOP x chains
        assert work == waves * 16 * per_iter
        got = buf.cpu().numpy()
        assert np.all(np.isfinite(got[:waves])) and got[0] != 0.0
        assert np.all(got[:waves] == got[0]), "every wave runs the same chains"
        assert np.all(got[waves:] == 0.0), "wrote past one float per wave"
        sums.append(got[0])
    assert sums[0] == sums[1]
    with pytest.raises(fa.FaError) as e:   # too small for one float per wave
        fa.probe_launch(kind, stream, buf.data_ptr(), (waves - 1) * 4, 16)
    assert e.value.status == fa.FA_ERR_INVALID_ARG


def test_probe_rates_are_plausible():
    torch = _torch()
    import bench   # the repo-root benchmark's probe routine, as the bench runs it

    peaks = bench.measure_peaks(torch, fa)
    for label, ent in peaks.items():
        frac = ent["frac_of_datasheet"]
        assert 0.25 < frac < 1.1, (label, ent)
