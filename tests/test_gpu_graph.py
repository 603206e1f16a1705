"""HIP graph capture of the launchers: bench.py and tune() time kernels by
replaying a captured graph, so every op path must record into a graph and
give the eager result on every replay.

Each replay is preceded by eager work on the outputs (a fill with NaN) and a
synchronisation, and its outputs are compared bit-for-bit with the eager run of
the same kernels (same instance, same split: the kernels are deterministic).
"""

import pytest
import torch

from icpp_tuning_amd import inputs as I
from icpp_tuning_amd.kernels import conv2d as conv_mod
from icpp_tuning_amd.kernels import fp8_gemm_bias_act as fp8_mod
from icpp_tuning_amd.kernels import gemm as gemm_mod
from icpp_tuning_amd.kernels import gemm_bias_layernorm as ln_mod
from icpp_tuning_amd.kernels._base import raw_from_inst, family_instances

pytestmark = pytest.mark.gpu

REPLAYS = 3


def _replay_check(run, outs, what):
    """run() launches into the current stream and writes the tensors in outs."""
    for o in outs:
        o.fill_(float("nan"))
    run()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    torch.cuda.synchronize()
    for r in range(REPLAYS):
        for o in outs:
            o.fill_(float("nan"))       # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o.view(torch.uint8), e.view(torch.uint8)), f"{what}: replay {r} differs from eager"
    print(f"[graph] {what}: {REPLAYS} replays match", flush=True)


def test_graph_gemm_splitk(gpu):
    M, N, K = 61, 2304, 768
    d = I.gemm_inputs(M, N, K, torch.float16, 95)
    A, B = d["A"].cuda(), d["B"].cuda()
    C = torch.empty((M, N), dtype=torch.float16, device="cuda")
    for sk in (1, 4):
        raw = next(r for r in gemm_mod.get_configs(M, K, split_k_values=(sk,), N=N) if r.get("split_k", 1) == sk)
        k = gemm_mod.build_kernel(M, N, K, config=raw)
        _replay_check(lambda: k(A, B, out=C), [C], f"gemm {gemm_mod.DESCRIPTOR.format_config(raw)}")


def test_graph_gemm_ln_two_pass(gpu):
    M, N, K = 300, 1024, 512
    d = I.config3(M, N, K)
    raw = raw_from_inst(family_instances("gemm_ln_stats")[0])
    raw["strategy"] = "two_pass"
    k = ln_mod.build_fused_kernel(M, N, K, gemm_config=raw)
    args = [d[t].cuda() for t in ("A", "B", "bias", "gamma", "beta")]
    Y = torch.empty((M, N), dtype=torch.float16, device="cuda")
    _replay_check(lambda: k(*args, out=Y), [Y], "gemm+ln two-pass")


def test_graph_gemm_ln_coresident(gpu):
    """The co-resident LayerNorm's counters return to zero at the end of every launch,
    so graph replays (one launch in two rounds, the second ragged) give the eager result
    each time."""
    M, N, K = 5000, 4096, 256
    d = I.config3(M, N, K)
    inst = next(i for i in family_instances("gemm") if i.name == "gemm_f16_256x256x64_w2x4_m16_s2_pp")
    raw = raw_from_inst(inst)
    raw["strategy"] = "coresident"
    k = ln_mod.build_fused_kernel(M, N, K, gemm_config=raw)
    args = [d[t].cuda() for t in ("A", "B", "bias", "gamma", "beta")]
    Y = torch.empty((M, N), dtype=torch.float16, device="cuda")
    _replay_check(lambda: k(*args, out=Y), [Y], "gemm+ln co-resident")


def test_graph_conv_splitk(gpu):
    Nb, H, W, C, F = 2, 14, 14, 256, 256
    d = I.config4(Nb, H, W, C, F)
    X, Wt = d["X"].cuda(), d["W"].cuda()
    Y = torch.empty((Nb, H, W, F), dtype=torch.float16, device="cuda")
    for sk in (1, 2):
        cfgs = [c for c in conv_mod.get_configs(C, 3, 3) if c.get("split_k", 1) == sk]
        k = conv_mod.build_conv2d_kernel(Nb, C, H, W, F, 3, 3, 1, 1, 1, config=cfgs[0])
        _replay_check(lambda: k(X, Wt, Y), [Y], f"conv sk={sk}")


def test_graph_fp8(gpu):
    M, N, K = 16, 4096, 4096
    d = I.config5(M, N, K)
    k = fp8_mod.build_kernel(M, N, K)
    a, b, bias = d["A"].cuda(), d["B"].cuda(), d["bias"].cuda()
    Y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    _replay_check(lambda: k(a, b, d["scale_a"], d["scale_b"], bias, out=Y), [Y], f"fp8 {k.config}")
