"""BERT encoder layer forward on the gfx950 fused kernels.

Restates the reference's end-to-end harness layer (evaluation/end2end.py
``bert_fwd_std`` :43-89) with its two GEMM blocks on this library:

  attention output   LN(h @ Wo + bo + input)         icpp_gemm_bias_residual_layernorm  (:76-79)
  FFN in             GELU(x @ Wi + bi)               icpp_gemm, act GELU-erf            (:82-83)
  FFN out            LN(inter @ Wo2 + bo2 + x)       icpp_gemm_bias_residual_layernorm  (:84-87)

The attention core (:52-71: scores = q k^T / sqrt(d) + causal mask, softmax,
attention @ v; dropout is p = 0 there, :230) dispatches by shape: head size 64
and a sequence that is a multiple of 32 up to 512 go through the head split
(icpp_qkv_split_heads) and one fused launch (icpp_attention_fwd: per-wave K
streaming up to 128 keys, K / V^T staged through LDS from 160 keys); any other
shape runs the scores and P V as batched library products around this library's
scaled masked softmax.  Like the
reference, the layer takes the QKV projections as given activations
(``qkv_kernel[layer] + qkv_bias[layer]``, :47) rather than computing them.

The reference imports helpers from a ``util`` package it does not ship
(``transpose_for_scores``, ``set_dtype``, ``time_stamp_cudasync``, ...); the
two this layer needs are restated below.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import torch

from . import runtime
from .kernels import gemm_bias_act, gemm_bias_layernorm


def transpose_for_scores(x: torch.Tensor, head_num: int, head_size: int) -> torch.Tensor:
    """[b, s, head_num * head_size] -> [b, s, head_num, head_size] (the reference's util helper,
    used at end2end.py:49-51 before its permute(0, 2, 1, 3))."""
    return x.view(x.shape[0], x.shape[1], head_num, head_size)


def causal_mask(seq_len: int, device, dtype=torch.float16) -> torch.Tensor:
    """Additive mask: -10000 above the diagonal, 0 elsewhere (end2end.py:62)."""
    return torch.triu(torch.full((seq_len, seq_len), -10000.0, device=device), 1).to(dtype)


@dataclass
class BertLayerWeights:
    """One layer's parameters, names as the reference's lists (end2end.py:276-286)."""
    qkv_bias: torch.Tensor                     # [3H]
    attr_output_kernel: torch.Tensor           # [H, H]
    attr_output_bias: torch.Tensor             # [H]
    attr_output_layernorm_gamma: torch.Tensor  # [H]
    attr_output_layernorm_beta: torch.Tensor   # [H]
    inter_kernel: torch.Tensor                 # [H, 4H]
    inter_bias: torch.Tensor                   # [4H]
    output_kernel: torch.Tensor                # [4H, H]
    output_bias: torch.Tensor                  # [H]
    output_layernorm_gamma: torch.Tensor       # [H]
    output_layernorm_beta: torch.Tensor        # [H]

    @staticmethod
    def random(hidden: int, seed: int, device="cpu", dtype=torch.float16) -> "BertLayerWeights":
        """U(-0.4, 0.4) for every parameter, as the reference initialises them."""
        g = torch.Generator().manual_seed(seed)

        def u(*shape):
            return (torch.rand(*shape, generator=g) * 0.8 - 0.4).to(dtype).to(device)

        H = hidden
        return BertLayerWeights(u(3 * H), u(H, H), u(H), u(H), u(H), u(H, 4 * H), u(4 * H), u(4 * H, H), u(H), u(H), u(H))

    def to(self, device) -> "BertLayerWeights":
        return BertLayerWeights(*[getattr(self, f).to(device) for f in self.__dataclass_fields__])


# Longest sequence sent to the fused attention kernel (its limit).  Measured against the
# batched-product path (split, bmm, scaled masked softmax, bmm, merge), b x s = 32x128 /
# 16x256 / 8x384 / 8x512: 28.3 / 37.0 / 43.6 / 51.7 us fused against 59.6 / 60.1 / 82.4 /
# 86.2 us.
ATTENTION_FUSED_MAX_SEQ = 512


def attention_core(qkv: torch.Tensor, head_num: int, head_size: int, mask: torch.Tensor,
                   softmax=None, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """softmax(q k^T / sqrt(d) + mask) v over heads, [b, s, 3H] -> [b, s, H] (end2end.py:47-71),
    with q, k, v taken from qkv (+ bias, [3H], when given).

    Default path: icpp_qkv_split_heads writes q, k and v per head with the bias added,
    then icpp_attention_fwd computes softmax(q k^T / sqrt(d) + mask) v in one launch and
    writes [b, s, H] (head_size 64, seq a multiple of 32 up to ATTENTION_FUSED_MAX_SEQ).  Other sequence
    lengths: k^T from the split, the scores from one batched product,
    icpp_softmax_scaled_masked (scale, additive mask and softmax in one pass), and
    icpp_merge_heads; other head sizes: one strided add into [3, b, h, s, d] and a k copy.  With ``softmax`` given (a row softmax),
    the reference's order is kept op for op -- scale, mask add, softmax -- as the torch
    composition this layer is measured against."""
    b, s, _ = qkv.shape
    H = head_num * head_size
    if softmax is not None:
        if bias is not None:
            qkv = qkv + bias
        q1, k1, v1 = qkv.chunk(3, dim=-1)
        q = transpose_for_scores(q1, head_num, head_size).permute(0, 2, 1, 3).reshape(b * head_num, s, head_size).contiguous()
        k = transpose_for_scores(k1, head_num, head_size).permute(0, 2, 3, 1).reshape(b * head_num, head_size, s).contiguous()
        v = transpose_for_scores(v1, head_num, head_size).permute(0, 2, 1, 3).reshape(b * head_num, s, head_size).contiguous()
        scores = torch.bmm(q, k) * (1.0 / math.sqrt(head_size))
        scores = (scores.view(b, head_num, s, s) + mask).reshape(b * head_num * s, s)
        attn = softmax(scores.contiguous()).view(b * head_num, s, s)
    else:
        fused = head_size == runtime.HEAD_DIM and qkv.dtype in (torch.float16, torch.bfloat16)
        if fused and s % 32 == 0 and s <= ATTENTION_FUSED_MAX_SEQ:
            # one kernel for the scores, the scaled masked softmax and P V (K, V^T per head)
            q, k, vt = runtime.qkv_split_heads(qkv.contiguous(), head_num, bias, layout=1)
            return runtime.attention_fwd(q, k, vt, b, 1.0 / math.sqrt(head_size), mask.to(qkv.dtype).contiguous())
        if fused:
            q, k, v = runtime.qkv_split_heads(qkv.contiguous(), head_num, bias)   # k: [b*h, d, s]
        else:
            heads = qkv.view(b, s, 3, head_num, head_size).permute(2, 0, 3, 1, 4)   # [3, b, h, s, d] view
            t = torch.empty((3, b, head_num, s, head_size), dtype=qkv.dtype, device=qkv.device)
            if bias is not None:
                torch.add(heads, bias.view(3, 1, head_num, 1, head_size), out=t)
            else:
                t.copy_(heads)
            q = t[0].view(b * head_num, s, head_size)
            v = t[2].view(b * head_num, s, head_size)
            k = t[1].view(b * head_num, s, head_size).transpose(1, 2).contiguous()    # [b*h, d, s]
        scores = torch.bmm(q, k).view(b * head_num * s, s)
        attn = runtime.softmax_scaled_masked(scores, 1.0 / math.sqrt(head_size),
                                             mask.to(qkv.dtype).contiguous()).view(b * head_num, s, s)
        h = torch.bmm(attn, v)                                   # [b*h, s, d]
        if fused:
            return runtime.merge_heads(h, b)
        return h.view(b, head_num, s, head_size).permute(0, 2, 1, 3).reshape(b, s, H).contiguous()
    h = torch.bmm(attn, v)                                       # [b*h, s, d]
    return h.view(b, head_num, s, head_size).permute(0, 2, 1, 3).reshape(b, s, H).contiguous()


class BertLayer:
    """One encoder layer at a fixed (batch, seq_len): the three GEMM blocks are
    resolved to compiled instances once (adaptive select), then ``forward``
    launches them."""

    def __init__(self, weights: BertLayerWeights, batch: int, seq_len: int, head_num: int = 12, head_size: int = 64,
                 eps: float = 1e-5):
        H = head_num * head_size
        M = batch * seq_len
        self.w, self.batch, self.seq, self.heads, self.hsize, self.eps = weights, batch, seq_len, head_num, head_size, eps
        self.attn_out = gemm_bias_layernorm.build_fused_kernel(M, H, H, eps=eps)
        self.ffn_in = gemm_bias_act.build_kernel(M, 4 * H, H, act="gelu_erf", dtype="f16")
        self.ffn_out = gemm_bias_layernorm.build_fused_kernel(M, H, 4 * H, eps=eps)
        self._mask: Optional[torch.Tensor] = None

    def forward(self, qkv_kernel: torch.Tensor, input_tensor: torch.Tensor) -> torch.Tensor:
        """qkv_kernel: [b, s, 3H] projections (the layer adds qkv_bias); input_tensor: [b, s, H]."""
        w = self.w
        b, s = self.batch, self.seq
        H = self.heads * self.hsize
        if self._mask is None or self._mask.device != qkv_kernel.device:
            self._mask = causal_mask(s, qkv_kernel.device, qkv_kernel.dtype)
        h = attention_core(qkv_kernel, self.heads, self.hsize, self._mask, bias=w.qkv_bias).view(b * s, H)
        x1 = self.attn_out(h, w.attr_output_kernel, w.attr_output_bias, w.attr_output_layernorm_gamma,
                           w.attr_output_layernorm_beta, residual=input_tensor.reshape(b * s, H))
        inter = self.ffn_in(x1, w.inter_kernel, w.inter_bias)
        out = self.ffn_out(inter, w.output_kernel, w.output_bias, w.output_layernorm_gamma, w.output_layernorm_beta,
                           residual=x1)
        return out.view(b, s, H)


def bert_forward(layers: List[BertLayer], input_from_tensor: torch.Tensor, qkv_kernels: List[torch.Tensor]):
    """The reference's layer loop (end2end.py:45-89): each layer's output feeds the next
    layer's residual input; the QKV activations are given per layer."""
    hidden = input_from_tensor
    for layer, qkv in zip(layers, qkv_kernels):
        hidden = layer.forward(qkv, hidden)
    return hidden


__all__ = ["ATTENTION_FUSED_MAX_SEQ", "BertLayer", "BertLayerWeights", "attention_core", "bert_forward", "causal_mask", "transpose_for_scores"]
