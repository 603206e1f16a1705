"""GPU parity of the BERT-layer building blocks and of the whole layer.

  GEMM + bias + residual + LayerNorm (every LN instance, all three strategies):
      atol 2e-2, rtol 2e-2 as the GEMM+bias+LN rows (x is stored as f16 before the
      two-pass normalisation)
  GEMM + bias + GELU-erf (f16): rtol 1e-2, atol 1e-2 as the reference's GEMM+act check
  BERT layer (end2end.py bert_fwd_std, f16 storage between blocks, U(-0.4, 0.4)
  parameters as the reference): max |err| <= 6e-2 and mean |err| <= 6e-3 against the
  fp32 oracle; the layer output is LayerNorm-scaled by gamma in (-0.4, 0.4)
"""

import math

import pytest
import torch

from icpp_tuning_amd import inputs as I
from icpp_tuning_amd import runtime
from icpp_tuning_amd.bert import BertLayer, BertLayerWeights, bert_forward
from icpp_tuning_amd.kernels import gemm_bias_act as gba_mod
from icpp_tuning_amd.kernels import gemm_bias_layernorm as ln_mod
from icpp_tuning_amd.kernels._base import family_instances, raw_from_inst
from oracle import ops as O

pytestmark = pytest.mark.gpu


def _close(y, ref, rtol, atol, what):
    y = y.float().cpu()
    ref = ref.float().cpu()
    assert torch.isfinite(y).all(), f"{what}: non-finite"
    err = (y - ref).abs()
    bad = err > atol + rtol * ref.abs()
    assert not bad.any(), f"{what}: {int(bad.sum())} / {y.numel()} outside tol, max err {err.max().item():.4g}"


@pytest.mark.parametrize("strategy", ["row", "two_pass", "gemm_ln", "coresident"])
def test_residual_layernorm_every_instance(gpu, strategy):
    M, N, K = 200, 768, 512
    d = I.gemm_inputs(M, N, K, torch.float16, 60, b_std=1 / math.sqrt(K), bias=True)
    g = torch.Generator().manual_seed(61)
    gamma, beta = torch.rand(N, generator=g).half(), torch.rand(N, generator=g).half()
    R = torch.randn(M, N, generator=g).half()
    ref = O.gemm_bias_layernorm_ref(d["A"], d["B"], d["bias"], gamma, beta, 1e-5, residual=R)
    dev = [t.cuda() for t in (d["A"], d["B"], d["bias"], gamma, beta)]
    fam = ln_mod.STRATEGY_FAMILY[strategy]
    for inst in family_instances(fam):
        if K % inst.bk or (strategy == "row" and N > inst.bn) or inst.dtype != "f16":
            continue
        if strategy == "coresident" and not ln_mod.coresident_fits(inst, N):
            continue
        raw = raw_from_inst(inst)
        raw["strategy"] = strategy
        print(f"[parity] residual LN {inst.name}", flush=True)
        k = ln_mod.build_fused_kernel(M, N, K, gemm_config=raw)
        y = k(*dev, residual=R.cuda())
        torch.cuda.synchronize()
        _close(y, ref, 2e-2, 2e-2, f"{inst.name} residual")
        # in place: the residual is the output buffer
        y2 = R.cuda().clone()
        k(*dev, out=y2, residual=y2)
        torch.cuda.synchronize()
        _close(y2, ref, 2e-2, 2e-2, f"{inst.name} residual in place")


def test_gemm_bias_gelu_erf(gpu):
    M, N, K = 256, 3072, 768
    d = I.gemm_inputs(M, N, K, torch.float16, 62, b_std=1 / math.sqrt(K), bias=True)
    ref = O.gemm_bias_act_ref(d["A"], d["B"], d["bias"], "gelu_erf")
    k = gba_mod.build_kernel(M, N, K, act="gelu_erf", dtype="f16")
    y = k(d["A"].cuda(), d["B"].cuda(), d["bias"].cuda())
    torch.cuda.synchronize()
    _close(y, ref, 1e-2, 1e-2, f"gelu_erf {k.config}")
    # GELU-erf and GELU-tanh differ by up to ~1e-3 x |x|: the kernel must compute the erf form
    tanh_ref = O.gemm_bias_act_ref(d["A"], d["B"], d["bias"], "gelu_tanh")
    assert (y.float().cpu() - ref).abs().mean() < (tanh_ref - ref).abs().mean()


# (1, 128) and (4, 64): the fused attention kernel; (1, 416): its LDS-staged variant (over
# 256 keys); (2, 40): a length off the 32-key step, the batched-product path
@pytest.mark.parametrize("batch,seq,layers", [(1, 128, 2), (4, 64, 1), (1, 416, 1), (2, 40, 1)])
def test_bert_layers(gpu, batch, seq, layers):
    heads, hsize = 12, 64
    H = heads * hsize
    ws = [BertLayerWeights.random(H, seed=70 + i) for i in range(layers)]
    g = torch.Generator().manual_seed(80)
    x0 = (torch.rand(batch, seq, H, generator=g) * 0.8 - 0.4).half()
    qkvs = [(torch.rand(batch, seq, 3 * H, generator=g) * 0.8 - 0.4).half() for _ in range(layers)]
    ref = x0
    for w, q in zip(ws, qkvs):
        ref = O.bert_layer_ref(q, ref.half(), w, heads, hsize)
    mods = [BertLayer(w.to("cuda"), batch, seq, heads, hsize) for w in ws]
    print(f"[parity] bert b={batch} s={seq} layers={layers}", flush=True)
    out = bert_forward(mods, x0.cuda(), [q.cuda() for q in qkvs])
    torch.cuda.synchronize()
    err = (out.float().cpu() - ref).abs()
    assert torch.isfinite(out).all()
    assert err.max() <= 6e-2 and err.mean() <= 6e-3, (float(err.max()), float(err.mean()))
