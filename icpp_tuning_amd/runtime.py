"""Torch-facing launchers over the C ABI.

PyTorch provides device memory and the stream; every launch goes through
libicpp_hip.so.  Inputs are validated here (device, dtype, contiguity) so a
mismatch is a Python exception rather than a fault; shape constraints are
validated again by the library itself.
"""

from __future__ import annotations

from typing import Optional

import torch

from ._lib import ACT, CONV_EPI, DTYPE, FAMILY, LN_STRATEGY, lib

TORCH_DTYPE = {"f16": torch.float16, "bf16": torch.bfloat16, "fp8": torch.float8_e4m3fn}
OUT_DTYPE = {"f16": torch.float16, "bf16": torch.bfloat16, "fp8": torch.bfloat16}
BIAS_DTYPE = {"f16": torch.float16, "bf16": torch.bfloat16, "fp8": torch.float32}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check(t: Optional[torch.Tensor], name: str, dtype: Optional[torch.dtype] = None, shape=None,
           device: Optional[torch.device] = None) -> int:
    """Device pointer of t after checking that it lives on the GPU (on `device` when
    given), is contiguous and has the dtype / shape asked for; None for None."""
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor (got {t.device})")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, the other operands on {device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype} (got {t.dtype})")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)} (got {tuple(t.shape)})")
    return t.data_ptr()


def workspace_bytes(family: str, inst: int, M: int, N: int, K: int, split_k: int = 1) -> int:
    return lib().workspace_bytes(FAMILY[family], inst, M, N, K, split_k)


def ln_workspace_bytes(family: str, inst: int, M: int, N: int, K: int) -> int:
    """Workspace of a GEMM+bias+LayerNorm call (icpp_gemm_bias_layernorm_workspace_bytes);
    family is an instance family name or "gemm_ln_cr" (co-resident, an f16 GEMM instance)."""
    return lib().ln_workspace_bytes(LN_STRATEGY[family], inst, M, N, K)


def alloc_workspace(nbytes: int, device, zeroed: bool = False) -> Optional[torch.Tensor]:
    """A workspace of at least nbytes (16-byte aligned); zeroed for the co-resident
    LayerNorm, whose counter block must start at zero (each call leaves it zero)."""
    if nbytes <= 0:
        return None
    shape = ((nbytes + 15) // 16 * 4,)
    if zeroed:
        return torch.zeros(shape, dtype=torch.float32, device=device)
    return torch.empty(shape, dtype=torch.float32, device=device)


def gemm(inst: int, dtype: str, a: torch.Tensor, b: torch.Tensor, bias: Optional[torch.Tensor] = None,
         out: Optional[torch.Tensor] = None, act: str = "none", scale_a: float = 1.0, scale_b: float = 1.0,
         split_k: int = 1, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[M,N] = act(scale_a*scale_b * a[M,K] @ b[K,N] + bias[N]) through icpp_gemm."""
    M, K = a.shape
    K2, N = b.shape
    if K2 != K:
        raise ValueError(f"inner dimensions differ: a is {tuple(a.shape)}, b is {tuple(b.shape)}")
    tdt = TORCH_DTYPE[dtype]
    pa = _check(a, "a", tdt)
    pb = _check(b, "b", tdt, device=a.device)
    pbias = _check(bias, "bias", BIAS_DTYPE[dtype], (N,), device=a.device)
    if out is None:
        out = torch.empty((M, N), dtype=OUT_DTYPE[dtype], device=a.device)
    pc = _check(out, "out", OUT_DTYPE[dtype], (M, N), device=a.device)
    need = workspace_bytes("gemm", inst, M, N, K, split_k)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = alloc_workspace(need, a.device)
    pws = workspace.data_ptr() if (need and workspace is not None) else None
    wsb = workspace.numel() * workspace.element_size() if (need and workspace is not None) else 0
    lib().call("icpp_gemm", inst, pa, pb, pbias, pc, M, N, K, K, N, N, ACT[act],
               float(scale_a), float(scale_b), split_k, pws, wsb, _stream())
    return out


def gemm_bias_layernorm(family: str, inst: int, a: torch.Tensor, b: torch.Tensor, bias: Optional[torch.Tensor],
                        gamma: torch.Tensor, beta: torch.Tensor, out: Optional[torch.Tensor] = None,
                        eps: float = 1e-5, workspace: Optional[torch.Tensor] = None,
                        residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = LayerNorm_N(a @ b + bias [+ residual]) * gamma + beta through icpp_gemm_bias_layernorm
    (or icpp_gemm_bias_residual_layernorm with a residual [M, N] f16; it may be out itself).
    family "gemm_ln_cr" (an f16 "gemm" instance) is the co-resident strategy: a workspace
    passed in must have been zero-filled once (alloc_workspace(..., zeroed=True)); the
    calls keep it zero, and calls sharing it must not overlap in time."""
    M, K = a.shape
    _, N = b.shape
    h = torch.float16
    pa, pb = _check(a, "a", h), _check(b, "b", h, (K, N), device=a.device)
    pbias = _check(bias, "bias", h, (N,), device=a.device)
    pg, pbe = _check(gamma, "gamma", h, (N,), device=a.device), _check(beta, "beta", h, (N,), device=a.device)
    if out is None:
        out = torch.empty((M, N), dtype=h, device=a.device)
    py = _check(out, "out", h, (M, N), device=a.device)
    need = ln_workspace_bytes(family, inst, M, N, K)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = alloc_workspace(need, a.device, zeroed=family == "gemm_ln_cr")
    pws = workspace.data_ptr() if (need and workspace is not None) else None
    wsb = workspace.numel() * workspace.element_size() if (need and workspace is not None) else 0
    if residual is None:
        lib().call("icpp_gemm_bias_layernorm", LN_STRATEGY[family], inst, pa, pb, pbias, pg, pbe, py,
                   M, N, K, float(eps), pws, wsb, _stream())
    else:
        pr = _check(residual, "residual", h, (M, N), device=a.device)
        lib().call("icpp_gemm_bias_residual_layernorm", LN_STRATEGY[family], inst, pa, pb, pbias, pr, pg, pbe, py,
                   M, N, K, float(eps), pws, wsb, _stream())
    return out


def fp8_pack_b(b: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """B [K, N] fp8 e4m3 (row-major) rearranged for fp8_gemm_packed through icpp_fp8_pack_b:
    every 16-column block one contiguous run over K, each 128-deep K step 2 KiB in the
    16x16x128 MFMA operand layout.  Returns (or fills) a uint8 tensor of K * N bytes.
    Needs K % 128 == 0 and N % 16 == 0; run once per weight matrix."""
    K, N = b.shape
    pb = _check(b, "b", torch.float8_e4m3fn)
    if out is None:
        out = torch.empty(K * N, dtype=torch.uint8, device=b.device)
    po = _check(out, "out", torch.uint8, (K * N,), device=b.device)
    lib().call("icpp_fp8_pack_b", pb, po, K, N, _stream())
    return out


def fp8_gemm_packed(a: torch.Tensor, bp: torch.Tensor, N: int, bias: Optional[torch.Tensor] = None,
                    out: Optional[torch.Tensor] = None, act: str = "silu", scale_a: float = 1.0,
                    scale_b: float = 1.0) -> torch.Tensor:
    """out[M, N] (bf16) = act(scale_a*scale_b * a[M, K] @ B + bias[N]) for M <= 32, B given
    packed by fp8_pack_b: one launch through icpp_fp8_gemm_packed."""
    M, K = a.shape
    pa = _check(a, "a", torch.float8_e4m3fn)
    pb = _check(bp, "bp", torch.uint8, (K * N,), device=a.device)
    pbias = _check(bias, "bias", torch.float32, (N,), device=a.device)
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    pc = _check(out, "out", torch.bfloat16, (M, N), device=a.device)
    lib().call("icpp_fp8_gemm_packed", pa, pb, pbias, pc, M, N, K, ACT[act], float(scale_a), float(scale_b),
               _stream())
    return out


def coresident_layout(inst: int, M: int, N: int) -> tuple:
    """(error word index, counter index, counter count) of a co-resident LayerNorm workspace
    viewed as int32: M * ceil(N / block_n) (mean, M2) fp32 pairs, padded to 16 bytes, then
    16 bytes whose first int is the error word, then two counters per block_m rows."""
    from .instances import INSTANCES
    t = sorted((i for i in INSTANCES if i.family == "gemm"), key=lambda i: i.name)[inst]
    err = (M * -(-N // t.bn) * 2 + 3) // 4 * 4
    return err, err + 4, 2 * -(-M // t.bm)


def coresident_wait_failed(workspace: torch.Tensor, inst: int, M: int, N: int, clear: bool = False) -> bool:
    """Whether a co-resident LayerNorm call on this workspace ran out of its bounded wait: a
    row block's workgroups were not resident together (another kernel holding CUs, or two
    calls on the workspace overlapping), and that call's output is invalid.  The word
    stays set across calls until cleared (clear=True).  Reads device memory: synchronises
    the current stream."""
    err, _, _ = coresident_layout(inst, M, N)
    words = workspace.view(torch.int32)
    failed = bool(words[err].item())
    if failed and clear:
        words[err] = 0
    return failed


def conv2d_nhwc(inst: int, x: torch.Tensor, w: torch.Tensor, y: torch.Tensor, stride: int = 1, pad: int = 1,
                dilation: int = 1, split_k: int = 1, workspace: Optional[torch.Tensor] = None, *,
                act: str = "none", bn: Optional[tuple] = None, eps: float = 1e-5, var_clamp: bool = False,
                residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y[N,OH,OW,F] = conv2d(x[N,H,W,C], w[KH,KW,C,F]) (f16) through icpp_conv2d_nhwc, or with
    a fused epilogue y = act(BN(conv) + residual) through icpp_conv2d_nhwc_fused:
    bn = (gamma, beta, mean, var), each [F] f16; residual [N,OH,OW,F] f16; act "none" / "relu"."""
    N, H, W, C = x.shape
    KH, KW, C2, F = w.shape
    if C2 != C:
        raise ValueError(f"channel mismatch: x has C={C}, w has C={C2}")
    OH = (H + 2 * pad - dilation * (KH - 1) - 1) // stride + 1
    OW = (W + 2 * pad - dilation * (KW - 1) - 1) // stride + 1
    h = torch.float16
    px, pw = _check(x, "x", h), _check(w, "w", h, device=x.device)
    py = _check(y, "y", h, (N, OH, OW, F), device=x.device)
    Mg, Kg = N * OH * OW, KH * KW * C
    need = workspace_bytes("conv2d", inst, Mg, F, Kg, split_k)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = alloc_workspace(need, x.device)
    pws = workspace.data_ptr() if (need and workspace is not None) else None
    wsb = workspace.numel() * workspace.element_size() if (need and workspace is not None) else 0
    if act == "none" and bn is None and residual is None:
        lib().call("icpp_conv2d_nhwc", inst, px, pw, py, N, H, W, C, F, KH, KW, stride, pad, dilation,
                   split_k, pws, wsb, _stream())
        return y
    flags = 0
    pbn = [None] * 4
    if bn is not None:
        if len(bn) != 4:
            raise ValueError("bn must be (gamma, beta, mean, var)")
        pbn = [_check(t, nm, h, (F,), device=x.device) for t, nm in zip(bn, ("gamma", "beta", "mean", "var"))]
        flags |= CONV_EPI["bn"] | (CONV_EPI["var_clamp"] if var_clamp else 0)
    elif var_clamp:
        raise ValueError("var_clamp needs bn")
    pres = _check(residual, "residual", h, (N, OH, OW, F), device=x.device)
    if residual is not None:
        flags |= CONV_EPI["residual"]
    lib().call("icpp_conv2d_nhwc_fused", inst, px, pw, py, pres, *pbn, float(eps), flags, ACT[act],
               N, H, W, C, F, KH, KW, stride, pad, dilation, split_k, pws, wsb, _stream())
    return y


ROW_DTYPE = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}


def _rows(x: torch.Tensor, name: str):
    """A [M, N] view of x (last dimension = row) with unit column stride."""
    if x.dtype not in ROW_DTYPE:
        raise TypeError(f"{name} must be float16, bfloat16 or float32 (got {x.dtype})")
    if not x.is_cuda:
        raise ValueError(f"{name} must be a device tensor (got {x.device})")
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1:
        raise ValueError(f"{name} must have unit stride in its last dimension")
    return x2


def layernorm_fwd(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float = 1e-5,
                  out: Optional[torch.Tensor] = None):
    """y = (x - mean) * rstd * weight + bias over the last dimension through icpp_layernorm_fwd;
    returns (y, mean, rstd) with fp32 per-row statistics."""
    x2 = _rows(x, "x")
    M, N = x2.shape
    dt = ROW_DTYPE[x.dtype]
    pw = _check(weight, "weight", x.dtype, (N,), device=x.device)
    pb = _check(bias, "bias", x.dtype, (N,), device=x.device)
    if out is None:
        out = torch.empty_like(x)
    y2 = _rows(out, "out")
    if tuple(y2.shape) != (M, N) or out.dtype != x.dtype or out.device != x.device:
        raise ValueError("out must match x")
    mean = torch.empty((M,), dtype=torch.float32, device=x.device)
    rstd = torch.empty((M,), dtype=torch.float32, device=x.device)
    lib().call("icpp_layernorm_fwd", DTYPE[dt], x2.data_ptr(), pw, pb, y2.data_ptr(), mean.data_ptr(),
               rstd.data_ptr(), M, N, x2.stride(0), y2.stride(0), float(eps), _stream())
    return out, mean, rstd


def layernorm_bwd(dy: torch.Tensor, x: torch.Tensor, weight: torch.Tensor, mean: torch.Tensor, rstd: torch.Tensor):
    """(dx, dw, db) of the LayerNorm above through icpp_layernorm_bwd (dx in x's dtype and
    layout; dw, db in weight's dtype)."""
    x2 = _rows(x.contiguous(), "x")
    dy2 = _rows(dy.contiguous(), "dy")
    M, N = x2.shape
    if tuple(dy2.shape) != (M, N) or dy.dtype != x.dtype or dy.device != x.device:
        raise ValueError("dy must match x")
    dt = ROW_DTYPE[x.dtype]
    pw = _check(weight, "weight", x.dtype, (N,), device=x.device)
    pm = _check(mean, "mean", torch.float32, (M,), device=x.device)
    pr = _check(rstd, "rstd", torch.float32, (M,), device=x.device)
    dx = torch.empty((M, N), dtype=x.dtype, device=x.device)
    dw = torch.empty((N,), dtype=weight.dtype, device=x.device)
    db = torch.empty((N,), dtype=weight.dtype, device=x.device)
    need = lib().layernorm_bwd_workspace_bytes(DTYPE[dt], M, N, N)
    ws = alloc_workspace(need, x.device)
    lib().call("icpp_layernorm_bwd", DTYPE[dt], dy2.data_ptr(), x2.data_ptr(), pw, pm, pr, dx.data_ptr(),
               dw.data_ptr(), db.data_ptr(), M, N, N, ws.data_ptr() if ws is not None else None, need, _stream())
    return dx.reshape(x.shape), dw, db


def softmax(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Row-wise softmax over the last dimension through icpp_softmax (fp32 arithmetic)."""
    x2 = _rows(x, "x")
    M, N = x2.shape
    if out is None:
        out = torch.empty_like(x)
    y2 = _rows(out, "out")
    if tuple(y2.shape) != (M, N) or out.dtype != x.dtype or out.device != x.device:
        raise ValueError("out must match x")
    lib().call("icpp_softmax", DTYPE[ROW_DTYPE[x.dtype]], x2.data_ptr(), y2.data_ptr(), M, N, x2.stride(0),
               y2.stride(0), _stream())
    return out


def softmax_scaled_masked(x: torch.Tensor, scale: float, mask: Optional[torch.Tensor] = None,
                          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """softmax(x * scale + mask) over the last dimension through icpp_softmax_scaled_masked.
    x: [..., R, N] rows; mask: [R, N] in x's dtype (broadcast over the leading dims), or None."""
    x2 = _rows(x, "x")
    M, N = x2.shape
    if out is None:
        out = torch.empty_like(x)
    y2 = _rows(out, "out")
    if tuple(y2.shape) != (M, N) or out.dtype != x.dtype:
        raise ValueError("out must match x")
    if out.device != x.device:
        raise ValueError(f"out is on {out.device}, x on {x.device}")
    pm, rows = None, 1
    if mask is not None:
        if mask.dtype != x.dtype or mask.dim() != 2 or mask.shape[1] != N or not mask.is_contiguous():
            raise ValueError(f"mask must be a contiguous [R, {N}] {x.dtype} tensor")
        if M % mask.shape[0]:
            raise ValueError("the number of rows must be a multiple of the mask's")
        pm, rows = _check(mask, "mask", device=x.device), mask.shape[0]
    lib().call("icpp_softmax_scaled_masked", DTYPE[ROW_DTYPE[x.dtype]], x2.data_ptr(), y2.data_ptr(), pm,
               float(scale), M, N, x2.stride(0), y2.stride(0), rows, _stream())
    return out


HEAD_DIM = 64  # head size the attention layout kernels serve


def qkv_split_heads(qkv: torch.Tensor, heads: int, bias: Optional[torch.Tensor] = None, layout: int = 0):
    """[batch, seq, 3*heads*64] (+ bias [3*heads*64]) -> per head, through icpp_qkv_split_heads
    (end2end.py:48-58: qkv + bias, chunk, transpose_for_scores, permute, k rearranged):
    layout 0: (q [b*h, seq, 64], k^T [b*h, 64, seq], v [b*h, seq, 64]);
    layout 1: (q, k [b*h, seq, 64], v^T [b*h, 64, seq]) for attention_fwd."""
    if qkv.dim() != 3 or qkv.dtype not in (torch.float16, torch.bfloat16) or not qkv.is_contiguous():
        raise ValueError("qkv_split_heads: qkv must be a contiguous [batch, seq, 3H] f16 / bf16 tensor")
    b, s, w = qkv.shape
    if w != 3 * heads * HEAD_DIM:
        raise ValueError(f"qkv_split_heads: last dim {w} != 3 * heads * {HEAD_DIM}")
    if bias is not None and (bias.dtype != qkv.dtype or not bias.is_contiguous() or bias.numel() != w):
        raise ValueError("qkv_split_heads: bias must be a contiguous [3H] tensor of qkv's dtype")
    pqkv = _check(qkv, "qkv")
    pbias = _check(bias, "bias", device=qkv.device)
    q = torch.empty((b * heads, s, HEAD_DIM), dtype=qkv.dtype, device=qkv.device)
    t = torch.empty((b * heads, HEAD_DIM, s), dtype=qkv.dtype, device=qkv.device)
    u = torch.empty_like(q)
    k, v = (t, u) if layout == 0 else (u, t)
    lib().call("icpp_qkv_split_heads", DTYPE[ROW_DTYPE[qkv.dtype]], pqkv, pbias, q.data_ptr(), k.data_ptr(),
               v.data_ptr(),
               b, s, heads, HEAD_DIM, int(layout), _stream())
    return q, k, v


def attention_fwd(q: torch.Tensor, k: torch.Tensor, vt: torch.Tensor, batch: int, scale: float,
                  mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """softmax(q k^T * scale + mask) v per (batch, head) -> [batch, seq, heads*64] through
    icpp_attention_fwd (end2end.py:59-73).  q, k [b*h, seq, 64], vt [b*h, 64, seq]
    (qkv_split_heads layout 1); mask [seq, seq] in q's dtype or None."""
    bh, s, d = q.shape
    if d != HEAD_DIM or k.shape != q.shape or vt.shape != (bh, d, s) or bh % batch \
            or any(not t.is_contiguous() or t.dtype != q.dtype for t in (q, k, vt)):
        raise ValueError("attention_fwd: q, k [b*h, s, 64] and vt [b*h, 64, s], contiguous, one dtype")
    if mask is not None and (mask.shape != (s, s) or mask.dtype != q.dtype or not mask.is_contiguous()):
        raise ValueError("attention_fwd: mask must be a contiguous [seq, seq] tensor of q's dtype")
    pq = _check(q, "q")
    pk, pvt = _check(k, "k", device=q.device), _check(vt, "vt", device=q.device)
    pmask = _check(mask, "mask", device=q.device)
    heads = bh // batch
    o = torch.empty((batch, s, heads * HEAD_DIM), dtype=q.dtype, device=q.device)
    lib().call("icpp_attention_fwd", DTYPE[ROW_DTYPE[q.dtype]], pq, pk, pvt, pmask, float(scale), o.data_ptr(),
               batch, s, heads, HEAD_DIM, _stream())
    return o


def merge_heads(ctx: torch.Tensor, batch: int) -> torch.Tensor:
    """[batch*heads, seq, 64] -> [batch, seq, heads*64] through icpp_merge_heads (end2end.py:72-73)."""
    if ctx.dim() != 3 or ctx.shape[2] != HEAD_DIM or ctx.dtype not in (torch.float16, torch.bfloat16) \
            or not ctx.is_contiguous() or ctx.shape[0] % batch:
        raise ValueError("merge_heads: ctx must be a contiguous [batch*heads, seq, 64] f16 / bf16 tensor")
    pctx = _check(ctx, "ctx")
    heads, s = ctx.shape[0] // batch, ctx.shape[1]
    y = torch.empty((batch, s, heads * HEAD_DIM), dtype=ctx.dtype, device=ctx.device)
    lib().call("icpp_merge_heads", DTYPE[ROW_DTYPE[ctx.dtype]], pctx, y.data_ptr(), batch, s, heads,
               HEAD_DIM, _stream())
    return y


__all__ = ["BIAS_DTYPE", "HEAD_DIM", "OUT_DTYPE", "ROW_DTYPE", "TORCH_DTYPE", "alloc_workspace", "conv2d_nhwc", "gemm",
           "attention_fwd", "gemm_bias_layernorm", "layernorm_bwd", "layernorm_fwd", "merge_heads", "qkv_split_heads", "softmax",
           "softmax_scaled_masked", "ln_workspace_bytes", "workspace_bytes"]
