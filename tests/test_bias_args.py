"""The binding rejects a bias the kernels would misread (they read fp32
bias[N] from the device): wrong dtype, non-contiguous, wrong length, host
array, other device.  CPU only: the checks run before any library call."""
import pytest
import torch

import sneppx_quant as sq


def test_bias_checks():
    y = torch.empty((2, 8))
    good = torch.zeros(8)
    assert sq._bias_ptr(None, 8, y) is None
    assert sq._bias_ptr(good, 8, y).value == good.data_ptr()
    with pytest.raises(ValueError, match="float32"):
        sq._bias_ptr(good.to(torch.bfloat16), 8, y)
    with pytest.raises(ValueError, match="contiguous"):
        sq._bias_ptr(torch.zeros(16)[::2], 8, y)
    with pytest.raises(ValueError, match="elements"):
        sq._bias_ptr(torch.zeros(7), 8, y)
    with pytest.raises(ValueError, match="elements"):
        sq._bias_ptr(torch.zeros(8), 16, y)          # SwiGLU form needs 2F
    with pytest.raises(ValueError, match="torch tensor"):
        sq._bias_ptr(good.numpy(), 8, y)
    with pytest.raises(ValueError, match="the output on"):
        sq._bias_ptr(good, 8, torch.empty((2, 8), device="meta"))
