"""fp32 CPU restatement of the reference's torch programs for each fused op.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

FP8_MAX = 448.0  # OCP e4m3fn largest finite value


def gemm_ref(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """C = A @ B with fp32 accumulation (reference gemm.py:19-21 computes
    ``(A @ B).to(float32)``; restated in fp32 on CPU)."""
    return A.float().cpu() @ B.float().cpu()


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) -- reference evaluation/end2end.py:37-38."""
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * torch.pow(x, 3.0))))


def apply_act(x: torch.Tensor, act: str) -> torch.Tensor:
    if act == "none":
        return x
    if act == "relu":
        return torch.clamp_min(x, 0.0)                 # gemm_bias_act.py:47 torch.relu
    if act in ("gelu_tanh", "gelu"):
        return gelu_tanh(x)
    if act == "silu":
        return x * torch.sigmoid(x)                    # SiLU = x * sigmoid(x)
    if act == "gelu_erf":
        return 0.5 * x * (1.0 + torch.erf(x * (1.0 / math.sqrt(2.0))))   # F.gelu (end2end.py:83)
    raise ValueError(act)


def gemm_bias_act_ref(A, B, bias, act: str = "relu") -> torch.Tensor:
    """act(A @ B + bias) in fp32 -- reference gemm_bias_act.py:43-47 (ReLU), with the
    GELU-tanh / SiLU epilogues the build adds."""
    x = gemm_ref(A, B)
    if bias is not None:
        x = x + bias.float().cpu().unsqueeze(0)
    return apply_act(x, act)


def gemm_bias_layernorm_ref(A, B, bias, gamma, beta, eps: float = 1e-5, residual=None) -> torch.Tensor:
    """layer_norm(A @ B + bias, (N,), gamma, beta, eps) in fp32 -- reference
    gemm_bias_layernorm.py:43-49 (torch_baseline); with a residual, layer_norm(A @ B +
    bias + residual) as the BERT attention-output / FFN-output blocks (end2end.py:76-79, :84-87)."""
    x = gemm_ref(A, B)
    if bias is not None:
        x = x + bias.float().cpu().unsqueeze(0)
    if residual is not None:
        x = x + residual.float().cpu()
    mean = x.mean(dim=1, keepdim=True)
    var = ((x - mean) ** 2).mean(dim=1, keepdim=True)  # biased variance, two-pass
    return (x - mean) * torch.rsqrt(var + eps) * gamma.float().cpu() + beta.float().cpu()


def conv2d_nhwc_ref(X, Wt, stride: int = 1, padding: int = 1, dilation: int = 1) -> torch.Tensor:
    """NHWC x HWIO conv2d in fp32 -- reference conv2d.py:35-62 (permute to NCHW/OIHW,
    F.conv2d, permute back)."""
    x = X.float().cpu().permute(0, 3, 1, 2)
    w = Wt.float().cpu().permute(3, 2, 0, 1)
    y = F.conv2d(x, w, stride=stride, padding=padding, dilation=dilation)
    return y.permute(0, 2, 3, 1).contiguous()


def conv2d_bn_act_ref(X, Wt, stride: int = 1, padding: int = 1, dilation: int = 1, bn=None, eps: float = 1e-5,
                      var_clamp: bool = False, residual=None, act: str = "none") -> torch.Tensor:
    """Fused conv epilogues in fp32, following the reference's torch programs:
      conv2d_relu.py:29-60       relu(conv)
      conv2d_bn.py:29-62         BN(conv), eps 1e-3 there
      conv2d_bn_relu.py:123-160  relu(BN(conv)), eps 1e-5
      conv_bn_add_relu.py:28-68  relu(BN(conv) + residual), var clamped at 0, eps 1e-5
    Each runs F.conv2d on f16 tensors, so its conv output is f16 before the
    epilogue's fp32 arithmetic: the conv is rounded to f16 here too.  BN(x) =
    (x - mean) * rsqrt(var + eps) * gamma + beta per output channel."""
    y = conv2d_nhwc_ref(X, Wt, stride, padding, dilation).to(torch.float16).float()
    if bn is not None:
        gamma, beta, mean, var = (t.float().cpu() for t in bn)
        if var_clamp:
            var = torch.clamp(var, min=0.0)
        y = (y - mean) * torch.rsqrt(var + eps) * gamma + beta
    if residual is not None:
        y = y + residual.float().cpu()
    return apply_act(y, act)


def layernorm_fwd_ref(x, w, b, eps: float = 1e-5):
    """Row LayerNorm in fp32 over the last dimension, as kernel/triton/layernorm.py
    _layer_norm_fwd_fused (:64-91): mean, centred variance, rstd = 1/sqrt(var + eps),
    y = (x - mean) * rstd * w + b.  Returns (y, mean, rstd)."""
    x = x.float().cpu()
    n = x.shape[-1]
    mean = x.sum(-1) / n
    d = x - mean.unsqueeze(-1)
    var = (d * d).sum(-1) / n
    rstd = 1.0 / torch.sqrt(var + eps)
    y = d * rstd.unsqueeze(-1) * w.float().cpu() + b.float().cpu()
    return y, mean, rstd


def layernorm_bwd_ref(dy, x, w, mean, rstd):
    """LayerNorm backward in fp32, as _layer_norm_bwd_dx_fused (:148-170) and
    _layer_norm_bwd_dwdb (:194-207): xhat = (x - mean) * rstd, wdy = w * dy,
    c1 = sum(xhat * wdy) / N, c2 = sum(wdy) / N, dx = (wdy - (xhat * c1 + c2)) * rstd,
    dw = sum over rows of dy * xhat, db = sum over rows of dy.  Returns (dx, dw, db)."""
    x = x.float().cpu().reshape(-1, x.shape[-1])
    dy = dy.float().cpu().reshape(x.shape)
    n = x.shape[-1]
    xhat = (x - mean.float().cpu().unsqueeze(-1)) * rstd.float().cpu().unsqueeze(-1)
    wdy = w.float().cpu() * dy
    c1 = (xhat * wdy).sum(-1, keepdim=True) / n
    c2 = wdy.sum(-1, keepdim=True) / n
    dx = (wdy - (xhat * c1 + c2)) * rstd.float().cpu().unsqueeze(-1)
    return dx, (dy * xhat).sum(0), dy.sum(0)


def softmax_ref(x):
    """Row softmax in fp32, as kernel/triton/softmax.py naive_softmax (:10-28):
    z = x - max(x), exp(z) / sum(exp(z)) over the last dimension."""
    x = x.float().cpu()
    z = x - x.max(dim=-1, keepdim=True)[0]
    num = torch.exp(z)
    return num / num.sum(dim=-1, keepdim=True)


def softmax_scaled_masked_ref(x, scale: float, mask=None):
    """softmax(x * scale + mask[row % R]) in fp32 over the last dimension: the attention
    scores of evaluation/end2end.py (:52-66, matmul / sqrt(d) + mask, then softmax) for a
    [rows, N] score matrix whose rows repeat the [R, N] mask (rows = batch*heads*R)."""
    z = x.float().cpu() * scale
    if mask is not None:
        m = mask.float().cpu()
        z = z + m.repeat(z.shape[0] // m.shape[0], 1)
    return softmax_ref(z)


def qkv_split_heads_ref(qkv, heads: int, bias=None):
    """evaluation/end2end.py:48-58 on the CPU: qkv + bias (rounded to qkv's dtype), chunk(3),
    transpose_for_scores, permute(0, 2, 1, 3) and k rearranged to '(b h) d s'.
    qkv [b, s, 3H] -> (q [b*h, s, d], k^T [b*h, d, s], v [b*h, s, d]), d = H / heads."""
    x = qkv.cpu()
    if bias is not None:
        x = (x.float() + bias.cpu().float()).to(qkv.dtype)
    b, s, w = x.shape
    d = w // 3 // heads
    q1, k1, v1 = x.chunk(3, dim=-1)
    per_head = [t.reshape(b, s, heads, d).permute(0, 2, 1, 3).reshape(b * heads, s, d).contiguous()
                for t in (q1, k1, v1)]
    return per_head[0], per_head[1].transpose(1, 2).contiguous(), per_head[2]


def attention_ref(q, k, v, batch: int, scale: float, mask=None):
    """softmax(q k^T * scale + mask) v per (batch, head) in fp32 on the CPU, merged to
    [batch, seq, heads*d] (end2end.py:59-73).  q, k, v [batch*heads, seq, d]; mask [seq, seq]."""
    qf, kf, vf = q.float().cpu(), k.float().cpu(), v.float().cpu()
    z = torch.bmm(qf, kf.transpose(1, 2)) * scale
    if mask is not None:
        z = z + mask.float().cpu()
    p = torch.softmax(z, dim=-1)
    return merge_heads_ref(torch.bmm(p, vf), batch)


def merge_heads_ref(ctx, batch: int):
    """[batch*heads, s, d] -> [batch, s, heads*d] (end2end.py:72-73: the context's
    'b h t d -> b t (h d)' reshape), on the CPU."""
    x = ctx.cpu()
    bh, s, d = x.shape
    return x.reshape(batch, bh // batch, s, d).permute(0, 2, 1, 3).reshape(batch, s, bh // batch * d).contiguous()


def bert_layer_ref(qkv_kernel, input_tensor, w, head_num: int, head_size: int, eps: float = 1e-5):
    """One BERT encoder layer in fp32, as evaluation/end2end.py bert_fwd_std (:47-87):
    qkv = qkv_kernel + qkv_bias; per head scores = q k^T / sqrt(d) + causal mask
    (-10000 above the diagonal), softmax, @ v; x = LN(h @ Wo + bo + input);
    out = LN(gelu_erf(x @ Wi + bi) @ Wo2 + bo2 + x).  w: a BertLayerWeights-like object."""
    f = lambda t: t.float().cpu()  # noqa: E731
    b, s, _ = qkv_kernel.shape
    H = head_num * head_size
    qkv = f(qkv_kernel) + f(w.qkv_bias)
    q, k, v = (t.reshape(b, s, head_num, head_size).permute(0, 2, 1, 3) for t in qkv.chunk(3, dim=-1))
    scores = (q @ k.transpose(-1, -2)) / math.sqrt(head_size)
    scores = scores + torch.triu(torch.full((s, s), -10000.0), 1)
    h = (softmax_ref(scores) @ v).permute(0, 2, 1, 3).reshape(b * s, H)

    def ln(x, g, be):
        mean = x.mean(-1, keepdim=True)
        var = ((x - mean) ** 2).mean(-1, keepdim=True)
        return (x - mean) * torch.rsqrt(var + eps) * f(g) + f(be)

    x1 = ln(h @ f(w.attr_output_kernel) + f(w.attr_output_bias) + f(input_tensor).reshape(b * s, H),
            w.attr_output_layernorm_gamma, w.attr_output_layernorm_beta)
    inter = apply_act(x1 @ f(w.inter_kernel) + f(w.inter_bias), "gelu_erf")
    out = ln(inter @ f(w.output_kernel) + f(w.output_bias) + x1, w.output_layernorm_gamma, w.output_layernorm_beta)
    return out.reshape(b, s, H)


def conv_out_hw(H, W, KH, KW, S, P, D=1):
    """reference conv2d.py:65-68"""
    return (H + 2 * P - D * (KH - 1) - 1) // S + 1, (W + 2 * P - D * (KW - 1) - 1) // S + 1


def fp8_gemm_bias_act_ref(Aq, Bq, scale_a: float, scale_b: float, bias, act: str = "silu") -> torch.Tensor:
    """act(scale_a*scale_b * deq(Aq) @ deq(Bq) + bias) in fp32 (no reference kernel exists;
    this is the dequantised-fp32 oracle BASELINE.json names for config 5)."""
    a = Aq.cpu().float()
    b = Bq.cpu().float()
    x = (a @ b) * (scale_a * scale_b)
    if bias is not None:
        x = x + bias.float().cpu().unsqueeze(0)
    return apply_act(x, act)
