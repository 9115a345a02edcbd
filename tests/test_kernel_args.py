"""Argument checks of the Python wrappers that run before any launch (no GPU needed)."""
import pytest
import torch

from drama3 import kernels


def test_fp8_linear_rejects_a_weight_of_another_dtype():
    x = torch.zeros((1, 512), dtype=torch.bfloat16)
    s = torch.zeros((16,), dtype=torch.bfloat16)
    # a bf16 weight's bytes would be read as twice as many e4m3 columns
    with pytest.raises(TypeError, match="float8_e4m3fn"):
        kernels.fp8_linear(x, torch.zeros((16, 512), dtype=torch.bfloat16), s)
    with pytest.raises(TypeError, match="float8_e4m3fn"):
        kernels.fp8_linear(x, torch.zeros((16, 512), dtype=torch.float32), s)


def test_fp8_linear_rejects_host_tensors():
    x = torch.zeros((1, 512), dtype=torch.bfloat16)
    s = torch.zeros((16,), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="one GPU"):
        kernels.fp8_linear(x, torch.zeros((16, 512), dtype=torch.uint8), s)
