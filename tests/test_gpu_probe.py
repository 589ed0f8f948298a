"""The hand-off micro-benchmark (fl_probe_handoff) completes in every mode: no wait times out and the
time per hand-off is positive. (Whether every workgroup ran on XCD blockIdx % 8, which the
XCD-local modes' figures and the decode attention's unit placement assume for speed only, is
logged.) Its figures are a bench leg."""
import ctypes

import pytest
import torch

from tests.helpers import log

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", [0, 1, 2, 3 | 1 << 8, 3 | 2 << 8 | 8 << 16, 3 | 3 << 8 | 4 << 16 | 2 << 24, 4])
@pytest.mark.parametrize("words", [256, 2560])
def test_probe_handoff_modes(dev, mode, words):
    from flint_amd import _lib
    grid = ctypes.c_int32()
    out = torch.zeros(2 * 1024, dtype=torch.int64, device=dev)
    _lib.call("fl_probe_handoff", mode, words, 50, _lib.ptr(out), ctypes.byref(grid), _lib.stream_ptr())
    torch.cuda.synchronize()
    o = out[:2 * grid.value].view(-1, 2).cpu()
    assert grid.value >= 8
    assert int(((o[:, 1] >> 32) & 1).sum()) == 0, "a wait timed out"
    assert bool((o[:, 0] > 0).all())
    xcc = (o[:, 1] & 0xF).tolist()
    us = float(o[:, 0].double().median()) * 0.01 / 50
    log(f"probe mode {mode:#x} words {words}: {us:.3f} us per hand-off, "
        f"xcd = blockIdx % 8: {all(x == i % 8 for i, x in enumerate(xcc))}")


@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4])
def test_probe_dequant_modes(dev, mode):
    """The dequantisation-rate probe (fl_probe_dequant) runs every form to completion with a
    positive time in every workgroup; the rate is logged (and reported by bench.py)."""
    from flint_amd import _lib
    grid = ctypes.c_int32()
    out = torch.zeros(2 * 1024, dtype=torch.int64, device=dev)
    _lib.call("fl_probe_dequant", mode, 50, _lib.ptr(out), ctypes.byref(grid), _lib.stream_ptr())
    torch.cuda.synchronize()
    o = out[:2 * grid.value].view(-1, 2).cpu()
    assert grid.value >= 8
    assert bool((o[:, 0] > 0).all())
    rate = grid.value * 8 * 3 * 2048 * 50 / (float(o[:, 0].max()) * 1e-8) / 1e12
    log(f"probe dequant mode {mode}: {rate:.2f} Tweights/s (50 passes)")
