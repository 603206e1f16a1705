"""The torch-facing launchers refuse host tensors (and tensors on another device)
with a Python exception before anything reaches the library: a host pointer
handed to a kernel would be a GPU memory fault instead."""

import pytest
import torch

from icpp_tuning_amd import runtime as RT

H = torch.float16


def _host_calls():
    q = torch.zeros(2, 32, 64, dtype=H)
    return {
        "gemm": lambda: RT.gemm(0, "f16", torch.zeros(16, 64, dtype=H), torch.zeros(64, 128, dtype=H)),
        "gemm_bias_layernorm": lambda: RT.gemm_bias_layernorm(
            "gemm_ln_stats", 0, torch.zeros(16, 64, dtype=H), torch.zeros(64, 128, dtype=H), None,
            torch.ones(128, dtype=H), torch.zeros(128, dtype=H)),
        "conv2d_nhwc": lambda: RT.conv2d_nhwc(0, torch.zeros(1, 4, 4, 8, dtype=H), torch.zeros(3, 3, 8, 8, dtype=H),
                                              torch.zeros(1, 4, 4, 8, dtype=H)),
        "layernorm_fwd": lambda: RT.layernorm_fwd(torch.zeros(4, 64, dtype=H), torch.ones(64, dtype=H),
                                                  torch.zeros(64, dtype=H)),
        "softmax": lambda: RT.softmax(torch.zeros(4, 64, dtype=H)),
        "softmax_scaled_masked": lambda: RT.softmax_scaled_masked(torch.zeros(4, 64, dtype=H), 0.125,
                                                                  torch.zeros(4, 64, dtype=H)),
        "qkv_split_heads": lambda: RT.qkv_split_heads(torch.zeros(1, 32, 192, dtype=H), 1,
                                                      torch.zeros(192, dtype=H)),
        "attention_fwd": lambda: RT.attention_fwd(q, q.clone(), torch.zeros(2, 64, 32, dtype=H), 1, 0.125,
                                                  torch.zeros(32, 32, dtype=H)),
        "merge_heads": lambda: RT.merge_heads(q, 1),
    }


@pytest.mark.parametrize("name", sorted(_host_calls()))
def test_host_tensors_are_refused_before_launch(name):
    with pytest.raises(ValueError):
        _host_calls()[name]()


@pytest.mark.gpu
def test_host_side_operand_next_to_device_tensors(gpu):
    """Device q / k / vt with a host mask, a device qkv with a host bias, device x
    with a host mask: each is refused before the launch."""
    q = torch.zeros(2, 32, 64, dtype=H, device=gpu)
    with pytest.raises(ValueError, match="mask"):
        RT.attention_fwd(q, q.clone(), torch.zeros(2, 64, 32, dtype=H, device=gpu), 1, 0.125,
                         torch.zeros(32, 32, dtype=H))
    with pytest.raises(ValueError, match="bias"):
        RT.qkv_split_heads(torch.zeros(1, 32, 192, dtype=H, device=gpu), 1, torch.zeros(192, dtype=H))
    with pytest.raises(ValueError, match="mask"):
        RT.softmax_scaled_masked(torch.zeros(4, 64, dtype=H, device=gpu), 0.125, torch.zeros(4, 64, dtype=H))
    with pytest.raises(ValueError, match="bias"):
        RT.gemm(0, "f16", torch.zeros(16, 64, dtype=H, device=gpu), torch.zeros(64, 128, dtype=H, device=gpu),
                bias=torch.zeros(128, dtype=H))
