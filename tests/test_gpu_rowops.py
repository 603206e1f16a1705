"""GPU parity of the standalone row kernels (LayerNorm forward / backward, softmax)
against the CPU oracle, through the C ABI (icpp_layernorm_fwd / _bwd, icpp_softmax).

Tolerances, elementwise |got - want| <= atol + rtol |want|:
  LayerNorm y, dx, dw, db   atol 1e-2 (the reference's test_layer_norm, layernorm.py:300-303)
                            + rtol one unit in the last place of the storage type
                            (2^-10 f16, 2^-7 bf16, 2^-20 f32): the reference's atol alone is
                            below an ulp for the large |dw| of long columns
  softmax f32               rtol 1e-5, atol 1e-8 (torch.allclose defaults, softmax.py:109)
  softmax f16 / bf16        rtol one ulp, atol 1e-6
Inputs follow the reference tests: x = -2.3 + 0.5 randn, w, b ~ U(0, 1), dy = 0.1 randn.
"""

import pytest
import torch

from icpp_tuning_amd import runtime
from icpp_tuning_amd.kernels.layernorm import layer_norm
from icpp_tuning_amd.kernels.softmax import softmax
from oracle import ops as O

pytestmark = pytest.mark.gpu

ULP = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7, torch.float32: 2.0 ** -20}
DT = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def _close(got, want, atol, rtol, what):
    got = got.float().cpu()
    want = want.float().cpu()
    assert got.shape == want.shape, what
    assert torch.isfinite(got).all(), f"{what}: non-finite"
    err = (got - want).abs()
    bad = err > atol + rtol * want.abs()
    if bad.any():
        idx = bad.nonzero()[0].tolist()
        raise AssertionError(f"{what}: {int(bad.sum())} / {got.numel()} outside tol, max err {err.max().item():.4g}; "
                             f"first at {idx}: got {got[tuple(idx)].item():.6g} want {want[tuple(idx)].item():.6g}")


def _ln_inputs(M, N, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = (-2.3 + 0.5 * torch.randn(M, N, generator=g)).to(dtype)
    w = torch.rand(N, generator=g).to(dtype)
    b = torch.rand(N, generator=g).to(dtype)
    dy = (0.1 * torch.randn(M, N, generator=g)).to(dtype)
    return x, w, b, dy


LN_CASES = [
    # (M, N, dtype): the reference test (1151 x 8192 f16), bench-like rows, ragged / scalar-path N, tiny rows
    (1151, 8192, "f16"),
    (4096, 1024, "f16"),
    (512, 15872, "f16"),
    (333, 4096, "bf16"),
    (257, 2048, "f32"),
    (64, 781, "f16"),       # N % 8 != 0: per-element path
    (7, 3, "f32"),
    (1, 16384, "bf16"),
    (3, 64, "f16"),
]


@pytest.mark.parametrize("M,N,dt", LN_CASES)
def test_layernorm_fwd_bwd(gpu, M, N, dt):
    dtype = DT[dt]
    x, w, b, dy = _ln_inputs(M, N, dtype, 100 + M + N)
    print(f"[parity] layernorm M={M} N={N} {dt}", flush=True)
    y, mean, rstd = runtime.layernorm_fwd(x.cuda(), w.cuda(), b.cuda(), 1e-5)
    dx, dw, db = runtime.layernorm_bwd(dy.cuda(), x.cuda(), w.cuda(), mean, rstd)
    torch.cuda.synchronize()
    y_ref, m_ref, r_ref = O.layernorm_fwd_ref(x, w, b, 1e-5)
    dx_ref, dw_ref, db_ref = O.layernorm_bwd_ref(dy, x, w, m_ref, r_ref)
    u = ULP[dtype]
    _close(mean, m_ref, 1e-5, 1e-5, "mean")
    _close(rstd, r_ref, 1e-5, 1e-4, "rstd")
    _close(y, y_ref, 1e-2, u, f"y {M}x{N} {dt}")
    _close(dx, dx_ref, 1e-2, u, f"dx {M}x{N} {dt}")
    _close(dw, dw_ref, 1e-2, u, f"dw {M}x{N} {dt}")
    _close(db, db_ref, 1e-2, u, f"db {M}x{N} {dt}")


def test_layernorm_bwd_deterministic(gpu):
    x, w, b, dy = [t.cuda() for t in _ln_inputs(3000, 4096, torch.float16, 7)]
    _, mean, rstd = runtime.layernorm_fwd(x, w, b)
    first = runtime.layernorm_bwd(dy, x, w, mean, rstd)
    for _ in range(3):
        again = runtime.layernorm_bwd(dy, x, w, mean, rstd)
        for a, c in zip(first, again):
            assert torch.equal(a, c)


def test_layer_norm_autograd(gpu):
    """The reference's usage (layernorm.py:282-303): layer_norm(x, w_shape, weight, bias, eps),
    then y.backward(dy); compared with the oracle (atol 1e-2 as the reference's test)."""
    M, N = 1151, 8192
    x, w, b, dy = _ln_inputs(M, N, torch.float16, 11)
    xc = x.cuda().requires_grad_(True)
    wc = w.cuda().requires_grad_(True)
    bc = b.cuda().requires_grad_(True)
    y = layer_norm(xc, (N,), wc, bc, 1e-5)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    y_ref, m_ref, r_ref = O.layernorm_fwd_ref(x, w, b, 1e-5)
    dx_ref, dw_ref, db_ref = O.layernorm_bwd_ref(dy, x, w, m_ref, r_ref)
    u = ULP[torch.float16]
    _close(y.detach(), y_ref, 1e-2, u, "y")
    _close(xc.grad, dx_ref, 1e-2, u, "dx")
    _close(wc.grad, dw_ref, 1e-2, u, "dw")
    _close(bc.grad, db_ref, 1e-2, u, "db")


SOFTMAX_CASES = [
    (1823, 781, "f32"),     # the reference's test (softmax.py:104-108), per-element path
    (4096, 4096, "f32"),
    (4096, 12672, "f32"),   # the top of the reference's benchmark sweep
    (1000, 1024, "f16"),
    (300, 32768, "bf16"),
    (5, 1, "f32"),
    (2, 65536, "f16"),
]


@pytest.mark.parametrize("M,N,dt", SOFTMAX_CASES)
def test_softmax(gpu, M, N, dt):
    dtype = DT[dt]
    g = torch.Generator().manual_seed(200 + N)
    x = (3.0 * torch.randn(M, N, generator=g)).to(dtype)
    print(f"[parity] softmax M={M} N={N} {dt}", flush=True)
    y = softmax(x.cuda())
    torch.cuda.synchronize()
    want = O.softmax_ref(x)
    if dtype == torch.float32:
        _close(y, want, 1e-8, 1e-5, f"softmax {M}x{N}")
    else:
        _close(y, want, 1e-6, ULP[dtype], f"softmax {M}x{N} {dt}")


def test_softmax_strided_rows(gpu):
    """Rows of a wider buffer (row stride > N), as the reference's x.stride(0) argument allows."""
    g = torch.Generator().manual_seed(5)
    base = torch.randn(64, 1040, generator=g)
    x = base[:, :1000]
    y = torch.empty(64, 1000).cuda()
    runtime.softmax(x.cuda().contiguous(), out=y)   # contiguous input
    xs = base.cuda()[:, :1000]                      # strided input view
    ys = runtime.softmax(xs)
    torch.cuda.synchronize()
    _close(ys, O.softmax_ref(x), 1e-8, 1e-5, "strided")
    assert torch.equal(ys, y)


@pytest.mark.parametrize("rows,R,N,dt", [(12 * 128, 128, 128, "f16"), (8 * 64, 64, 64, "bf16"),
                                         (6 * 20, 20, 1000, "f32"), (5 * 8, 8, 781, "f16")])
def test_softmax_scaled_masked(gpu, rows, R, N, dt):
    """softmax(x * scale + mask[row % R]) (the BERT layer's attention scores) against the oracle;
    N = 781 takes the per-element path.  Tolerances as test_softmax."""
    dtype = DT[dt]
    g = torch.Generator().manual_seed(300 + N)
    x = (4.0 * torch.randn(rows, N, generator=g)).to(dtype)
    mask = torch.triu(torch.full((R, N), -10000.0), 1).to(dtype)
    scale = 0.125
    print(f"[parity] softmax_scaled_masked rows={rows} R={R} N={N} {dt}", flush=True)
    y = runtime.softmax_scaled_masked(x.cuda(), scale, mask.cuda())
    y0 = runtime.softmax_scaled_masked(x.cuda(), scale)
    torch.cuda.synchronize()
    want = O.softmax_scaled_masked_ref(x, scale, mask)
    want0 = O.softmax_scaled_masked_ref(x, scale)
    if dtype == torch.float32:
        _close(y, want, 1e-8, 1e-5, f"masked softmax {rows}x{N}")
        _close(y0, want0, 1e-8, 1e-5, f"scaled softmax {rows}x{N}")
    else:
        _close(y, want, 1e-6, ULP[dtype], f"masked softmax {rows}x{N} {dt}")
        _close(y0, want0, 1e-6, ULP[dtype], f"scaled softmax {rows}x{N} {dt}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b,s,heads,with_bias", [(2, 128, 12, True), (3, 100, 4, True), (1, 37, 2, False),
                                                  (4, 64, 1, True), (1, 1, 3, True)])
def test_qkv_split_and_merge_heads(gpu, dtype, b, s, heads, with_bias):
    """icpp_qkv_split_heads / icpp_merge_heads against the CPU restatement, bit for bit:
    sequence tiles of 64 with a partial last one (100), lengths off the 8-token chunk
    (37, 1: the element-wise K^T path), no bias, one head."""
    g = torch.Generator().manual_seed(b * 1000 + s * 10 + heads)
    H = heads * 64
    qkv = (torch.rand(b, s, 3 * H, generator=g) * 4 - 2).to(dtype)
    bias = (torch.rand(3 * H, generator=g) - 0.5).to(dtype) if with_bias else None
    want = O.qkv_split_heads_ref(qkv, heads, bias)
    print(f"[parity] qkv_split_heads b={b} s={s} heads={heads} {dtype} bias={with_bias}", flush=True)
    got = runtime.qkv_split_heads(qkv.cuda(), heads, bias.cuda() if bias is not None else None)
    torch.cuda.synchronize()
    for name, w, o in zip(("q", "k^T", "v"), want, got):
        assert torch.equal(o.cpu().view(torch.int16), w.view(torch.int16)), name
    # layout 1: k untransposed, v transposed
    got1 = runtime.qkv_split_heads(qkv.cuda(), heads, bias.cuda() if bias is not None else None, layout=1)
    torch.cuda.synchronize()
    want1 = (want[0], want[1].transpose(1, 2).contiguous(), want[2].transpose(1, 2).contiguous())
    for name, w, o in zip(("q", "k", "v^T"), want1, got1):
        assert torch.equal(o.cpu().view(torch.int16), w.view(torch.int16)), name
    ctx = (torch.rand(b * heads, s, 64, generator=g) - 0.5).to(dtype)
    y = runtime.merge_heads(ctx.cuda(), b)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu().view(torch.int16), O.merge_heads_ref(ctx, b).view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b,s,heads,masked", [(2, 128, 12, True), (1, 32, 3, True), (3, 96, 2, False),
                                               (1, 512, 2, True), (2, 288, 1, True), (2, 192, 4, True),
                                               (1, 160, 3, False)])
def test_attention_fwd(gpu, dtype, b, s, heads, masked):
    """icpp_attention_fwd against fp32 attention on the CPU: the BERT layer's causal mask
    (-10000 above the diagonal), sequence lengths for both kernels (direct up to 128 keys,
    staged from 160 to 512, including 160 and 192 where one 128-key chunk is partial),
    a partial last 64-query block (96, 160, 288) and no mask.
    The unmasked cases use scale 1.0: scores of std ~2.7 give a peaked softmax, so the
    output depends on which key each probability belongs to (at the BERT scale 0.125 an
    unmasked softmax over U(-1, 1) inputs is nearly uniform and the output ~ mean(V)
    whatever the key order).
    Tolerance 1e-2 + 1e-2 |ref| (P is rounded to the data type before P V)."""
    g = torch.Generator().manual_seed(b * 7 + s + heads)
    q = (torch.rand(b * heads, s, 64, generator=g) * 2 - 1).to(dtype)
    k = (torch.rand(b * heads, s, 64, generator=g) * 2 - 1).to(dtype)
    v = (torch.rand(b * heads, s, 64, generator=g) * 2 - 1).to(dtype)
    mask = torch.triu(torch.full((s, s), -10000.0), 1).to(dtype) if masked else None
    scale = 0.125 if masked else 1.0
    want = O.attention_ref(q, k, v, b, scale, mask)
    print(f"[parity] attention_fwd b={b} s={s} heads={heads} {dtype} masked={masked} scale={scale}", flush=True)
    got = runtime.attention_fwd(q.cuda(), k.cuda(), v.transpose(1, 2).contiguous().cuda(), b, scale,
                                mask.cuda() if mask is not None else None)
    torch.cuda.synchronize()
    _close(got.float().cpu(), want, 1e-2, 1e-2, f"attention b={b} s={s} {dtype}")
