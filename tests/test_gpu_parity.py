"""GPU parity: every compiled instance against the CPU oracle on seeded inputs.

Tolerances (stated per op, checked elementwise as |y - y_ref| <= atol + rtol*|y_ref|):
  GEMM / GEMM+bias+act (fp16, bf16)     rtol 1e-2, atol 1e-2  (reference gemm_bias_act.py:160)
  conv2d (fp16)                          rtol 1e-2, atol 1e-2  (reference conv2d.py:310)
  GEMM+bias+LayerNorm (fp16 out)         atol 2e-2, rtol 2e-2
  fp8 e4m3 GEMM+bias+SiLU (bf16 out)     rtol 1e-2, atol 1e-2 against the oracle run on
                                         the same dequantised fp8 values (scale = amax/448)
"""

import math

import pytest
import torch

from icpp_tuning_amd import inputs as I
from icpp_tuning_amd import runtime
from icpp_tuning_amd.kernels import conv2d as conv_mod
from icpp_tuning_amd.kernels import fp8_gemm_bias_act as fp8_mod
from icpp_tuning_amd.kernels import gemm as gemm_mod
from icpp_tuning_amd.kernels import gemm_bias_act as gba_mod
from icpp_tuning_amd.kernels import gemm_bias_layernorm as ln_mod
from icpp_tuning_amd.kernels._base import family_instances, raw_from_inst
from oracle import ops as O

pytestmark = pytest.mark.gpu


def _close(y, ref, rtol, atol, what):
    y = y.float().cpu()
    ref = ref.float().cpu()
    assert y.shape == ref.shape, what
    assert torch.isfinite(y).all(), f"{what}: non-finite output"
    err = (y - ref).abs()
    bound = atol + rtol * ref.abs()
    bad = (err > bound)
    if bad.any():
        idx = bad.nonzero()[0].tolist()
        raise AssertionError(f"{what}: {int(bad.sum())} / {y.numel()} outside tol; max err {err.max().item():.4g}; "
                             f"first at {idx}: got {y[tuple(idx)].item():.5g} want {ref[tuple(idx)].item():.5g}")


def _gemm_inst_ids(dtype):
    return [(i, inst.name) for i, inst in enumerate(family_instances("gemm")) if inst.dtype == dtype]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_every_gemm_instance(gpu, dtype):
    """All compiled GEMM tiles at a ragged shape: M not a tile multiple, bias + act."""
    M, N, K = 200, 328, 512
    tdt = runtime.TORCH_DTYPE[dtype]
    d = I.gemm_inputs(M, N, K, tdt, 90, b_std=1 / math.sqrt(K), bias=True)
    for act in ("none", "relu", "gelu_tanh", "silu"):
        ref = O.gemm_bias_act_ref(d["A"], d["B"], d["bias"], act)
        A, B, bias = d["A"].cuda(), d["B"].cuda(), d["bias"].cuda()
        for idx, name in _gemm_inst_ids(dtype):
            inst = family_instances("gemm")[idx]
            if K % inst.bk:
                continue
            print(f"[parity] {name} act={act} M={M} N={N} K={K}", flush=True)
            y = runtime.gemm(idx, dtype, A, B, bias=bias, act=act)
            torch.cuda.synchronize()
            _close(y, ref, 1e-2, 1e-2, f"{name} act={act}")


def test_pingpong_twins_bitwise(gpu):
    """A ping-pong instance issues, per accumulator, the same MFMAs in the same K
    order as its default-schedule twin, so the outputs are bit-identical: odd K-tile
    counts, ragged M / N, split-K partials (uneven slices), fp8 with scales."""
    fam = family_instances("gemm")
    key = lambda t: (t.dtype, t.bm, t.bn, t.bk, t.wm, t.wn, t.mf, t.stages)
    pairs = [(i, next(j for j, u in enumerate(fam) if not u.sched and key(u) == key(t)))
             for i, t in enumerate(fam) if t.sched == "pp"]
    assert pairs
    for i, j in pairs:
        inst = fam[i]
        for M, N, nkt, sk in [(300, 528, 19, 1), (130, 272, 5, 2), (256, 256, 1, 1)]:
            K = nkt * inst.bk
            if inst.dtype == "fp8":
                d = I.config5(M, N, K)
                kw = dict(scale_a=d["scale_a"], scale_b=d["scale_b"], act="silu")
                A, B = d["A"].cuda(), d["B"].cuda()
            else:
                d = I.gemm_inputs(M, N, K, runtime.TORCH_DTYPE[inst.dtype], 95, b_std=1 / math.sqrt(K), bias=True)
                kw = dict(act="gelu_tanh")
                A, B = d["A"].cuda(), d["B"].cuda()
            bias = d["bias"].cuda()
            print(f"[parity] {inst.name} vs {fam[j].name} M={M} N={N} K={K} sk={sk}", flush=True)
            y_pp = runtime.gemm(i, inst.dtype, A, B, bias=bias, split_k=sk, **kw)
            y_ref = runtime.gemm(j, inst.dtype, A, B, bias=bias, split_k=sk, **kw)
            torch.cuda.synchronize()
            assert torch.equal(y_pp.view(torch.int16) if y_pp.element_size() == 2 else y_pp,
                               y_ref.view(torch.int16) if y_ref.element_size() == 2 else y_ref), \
                f"{inst.name} differs from {fam[j].name} at M={M} N={N} K={K} sk={sk}"


@pytest.mark.parametrize("M", [1, 6, 61, 126])
def test_reference_eval_shapes_splitk(gpu, M):
    """The reference's evaluation shapes (M=1..126, N=2304, K=768), fp16, split-K 1/2/4."""
    N, K = 2304, 768
    d = I.gemm_inputs(M, N, K, torch.float16, 91)
    ref = O.gemm_ref(d["A"], d["B"])
    A, B = d["A"].cuda(), d["B"].cuda()
    for raw in gemm_mod.get_configs(M, K, split_k_values=(1, 2, 4), N=N):
        k = gemm_mod.build_kernel(M, N, K, config=raw)
        print(f"[parity] gemm {gemm_mod.DESCRIPTOR.format_config(raw)} M={M}", flush=True)
        y = k(A, B)
        torch.cuda.synchronize()
        _close(y, ref, 1e-2, 1e-2, f"gemm {raw} M={M}")


def test_config1_gemm_1024(gpu):
    M = N = K = 1024
    d = I.config1()
    ref = O.gemm_ref(d["A"], d["B"])
    k = gemm_mod.build_kernel(M, N, K)
    y = k(d["A"].cuda(), d["B"].cuda())
    torch.cuda.synchronize()
    _close(y, ref, 1e-2, 1e-2, f"config1 {k.config}")


@pytest.mark.parametrize("act", ["gelu_tanh", "relu", "silu"])
def test_config2_gemm_bias_act_4096(gpu, act):
    M = N = K = 4096
    d = I.config2()
    ref = O.gemm_bias_act_ref(d["A"], d["B"], d["bias"], act)
    k = gba_mod.build_kernel(M, N, K, act=act, dtype="bf16")
    print(f"[parity] config2 {act} {k.config}", flush=True)
    y = k(d["A"].cuda(), d["B"].cuda(), d["bias"].cuda())
    torch.cuda.synchronize()
    _close(y, ref, 1e-2, 1e-2, f"config2 {act} {k.config}")


@pytest.mark.parametrize("strategy", ["row", "two_pass"])
def test_every_ln_instance(gpu, strategy):
    M, K = 333, 512
    fam = ln_mod.STRATEGY_FAMILY[strategy]
    for idx, inst in enumerate(family_instances(fam)):
        N = 768 if (strategy == "row" and inst.bn == 768) else (1024 if strategy == "row" else 776)
        d = I.config3(M, N, K)
        ref = O.gemm_bias_layernorm_ref(d["A"], d["B"], d["bias"], d["gamma"], d["beta"])
        raw = raw_from_inst(inst)
        raw["strategy"] = strategy
        print(f"[parity] {inst.name} M={M} N={N} K={K}", flush=True)
        k = ln_mod.build_fused_kernel(M, N, K, gemm_config=raw)
        y = k(*(d[t].cuda() for t in ("A", "B", "bias", "gamma", "beta")))
        torch.cuda.synchronize()
        _close(y, ref, 2e-2, 2e-2, inst.name)


@pytest.mark.parametrize("N", [768, 1024, 4096])
def test_config3_gemm_bias_layernorm(gpu, N):
    M, K = 8192, 4096
    d = I.config3(M, N, K)
    ref = O.gemm_bias_layernorm_ref(d["A"], d["B"], d["bias"], d["gamma"], d["beta"])
    k = ln_mod.build_fused_kernel(M, N, K)
    print(f"[parity] config3 N={N} {k.config}", flush=True)
    y = k(*(d[t].cuda() for t in ("A", "B", "bias", "gamma", "beta")))
    torch.cuda.synchronize()
    _close(y, ref, 2e-2, 2e-2, f"config3 N={N} {k.config}")


C3_OFFSETS = I.C3_OFFSETS


@pytest.mark.parametrize("kind", C3_OFFSETS)
@pytest.mark.parametrize("strategy", ["row", "two_pass", "gemm_ln", "coresident"])
def test_every_ln_instance_offset_rows(gpu, strategy, kind):
    """Every instance of each LayerNorm strategy on rows far from zero (ragged M and N;
    N = the row tile's width for whole-row instances)."""
    M, K = 333, 512
    fam = ln_mod.STRATEGY_FAMILY[strategy]
    refs = {}
    for inst in family_instances(fam):
        if inst.dtype != "f16" or K % inst.bk:
            continue
        N = inst.bn if strategy == "row" else 776
        if strategy == "coresident" and not ln_mod.coresident_fits(inst, N):
            continue
        if N not in refs:
            d = I.config3_offset(M, N, K, kind)
            refs[N] = (d, O.gemm_bias_layernorm_ref(d["A"], d["B"], d["bias"], d["gamma"], d["beta"]))
        d, ref = refs[N]
        raw = raw_from_inst(inst)
        raw["strategy"] = strategy
        print(f"[parity] {inst.name} {strategy} {kind} M={M} N={N} K={K}", flush=True)
        k = ln_mod.build_fused_kernel(M, N, K, gemm_config=raw)
        y = k(*(d[t].cuda() for t in ("A", "B", "bias", "gamma", "beta")))
        torch.cuda.synchronize()
        _close(y, ref, 2e-2, 2e-2, f"{inst.name} {strategy} {kind}")


@pytest.mark.parametrize("kind", C3_OFFSETS)
@pytest.mark.parametrize("N", [768, 1024, 4096])
def test_config3_offset_rows_every_strategy(gpu, N, kind):
    """Full config-3 size (M = 8192, K = 4096) on rows far from zero: the tuner's pick and
    the formula's best config of each strategy that serves N."""
    from icpp_tuning_amd.autotuner.interface import rank_all

    M, K = 8192, 4096
    d = I.config3_offset(M, N, K, kind)
    ref = O.gemm_bias_layernorm_ref(d["A"], d["B"], d["bias"], d["gamma"], d["beta"])
    dev = {t: d[t].cuda() for t in ("A", "B", "bias", "gamma", "beta")}
    configs, seen = [], set()
    ranked = rank_all(ln_mod.DESCRIPTOR, M=M, N=N, K=K)
    for strategy in ("row", "two_pass", "gemm_ln", "coresident"):
        top = next((e["raw_config"] for e in ranked if e["raw_config"].get("strategy") == strategy), None)
        if top is not None:
            configs.append(top)
    configs.append(ln_mod.build_fused_kernel(M, N, K).config)
    ran = 0
    for raw in configs:
        name = ln_mod.DESCRIPTOR.format_config(raw)
        if name in seen:
            continue
        seen.add(name)
        print(f"[parity] config3 offset {kind} N={N} {name}", flush=True)
        k = ln_mod.build_fused_kernel(M, N, K, gemm_config=raw)
        y = k(dev["A"], dev["B"], dev["bias"], dev["gamma"], dev["beta"])
        torch.cuda.synchronize()
        _close(y, ref, 2e-2, 2e-2, f"config3 offset {kind} N={N} {name}")
        ran += 1
    assert ran >= (4 if N <= 1024 else 3)


def _cr_counters(k, M, N):
    """(wait-failed flag, counter block) of a co-resident LayerNorm kernel's workspace, read
    through the runtime's layout of it."""
    _, ctr, n = runtime.coresident_layout(k.inst, M, N)
    return k.wait_failed(), k._ws.view(torch.int32).cpu()[ctr: ctr + n]


def test_coresident_every_instance(gpu):
    """Every f16 GEMM tile with the co-resident LayerNorm kernel on ragged M and N, called
    twice in a row (the counters must return to zero and the error flag stay clear)."""
    M, N, K = 333, 776, 512
    d = I.config3(M, N, K)
    ref = O.gemm_bias_layernorm_ref(d["A"], d["B"], d["bias"], d["gamma"], d["beta"])
    dev = [d[t].cuda() for t in ("A", "B", "bias", "gamma", "beta")]
    ran = 0
    for inst in family_instances("gemm"):
        if K % inst.bk or not ln_mod.coresident_fits(inst, N):
            continue
        raw = raw_from_inst(inst)
        raw["strategy"] = "coresident"
        print(f"[parity] co-resident {inst.name} M={M} N={N} K={K}", flush=True)
        k = ln_mod.build_fused_kernel(M, N, K, gemm_config=raw)
        for call in range(2):
            y = k(*dev)
            torch.cuda.synchronize()
            _close(y, ref, 2e-2, 2e-2, f"{inst.name} co-resident call {call}")
            err, ctr = _cr_counters(k, M, N)
            assert err == 0 and not ctr.any(), f"{inst.name}: error flag {err}, counters {ctr.tolist()}"
        ran += 1
    assert ran >= 10


def test_coresident_statistics_across_two_stages(gpu):
    """Tiles whose row block's (mean, M2) pairs outgrow one LDS stage array at N = 2312
    (37 tile columns of 64, 19 of 128): the kernel puts an even number of rows in the
    first array and the rest in the second.  The last row block has an odd row count
    and the tile-column count is odd, so the odd last pair lands in the second array."""
    N, K = 2312, 256
    ran = 0
    for inst in family_instances("gemm"):
        tiles_n = -(-N // inst.bn)
        stage = (inst.bm + inst.bn) * inst.bk * 2
        if K % inst.bk or not ln_mod.coresident_fits(inst, N) or inst.bm * tiles_n * 8 <= stage:
            continue
        M = 2 * inst.bm - 5
        d = I.config3(M, N, K)
        ref = O.gemm_bias_layernorm_ref(d["A"], d["B"], d["bias"], d["gamma"], d["beta"])
        raw = raw_from_inst(inst)
        raw["strategy"] = "coresident"
        print(f"[parity] co-resident two-stage statistics {inst.name} M={M} N={N} K={K}", flush=True)
        k = ln_mod.build_fused_kernel(M, N, K, gemm_config=raw)
        y = k(*(d[t].cuda() for t in ("A", "B", "bias", "gamma", "beta")))
        torch.cuda.synchronize()
        _close(y, ref, 2e-2, 2e-2, f"{inst.name} two-stage statistics")
        err, ctr = _cr_counters(k, M, N)
        assert not err and not ctr.any(), f"{inst.name}: wait failed {err}, counters {ctr.tolist()}"
        ran += 1
    assert ran >= 3


@pytest.mark.parametrize("M,N,tile", [(8192, 4096, "gemm_f16_256x256x64_w2x4_m16_s2_pp"),
                                       (5000, 4096, "gemm_f16_256x256x64_w2x4_m16_s2_pp"),
                                       (11000, 768, "gemm_f16_256x128x64_w2x4_m16_s2")])
def test_coresident_rounds_and_chunks(gpu, M, N, tile):
    """Row blocks beyond what the device holds at once: the 256 x 256 tile at N = 4096 runs
    one launch in rounds of 16 row blocks (8 x 4 tiles per XCD), the last round ragged at
    M = 5000 (its spare workgroups exit); at N = 768 the 256 x 128 tile's 6 tile columns do
    not split over 8 XCDs, so its 43 row blocks go out in even chunks, one launch each."""
    K = 128
    d = I.config3(M, N, K)
    ref = O.gemm_bias_layernorm_ref(d["A"], d["B"], d["bias"], d["gamma"], d["beta"])
    inst = next(i for i in family_instances("gemm") if i.name == tile)
    raw = raw_from_inst(inst)
    raw["strategy"] = "coresident"
    print(f"[parity] co-resident rounds / chunks {inst.name} M={M} N={N} K={K}", flush=True)
    k = ln_mod.build_fused_kernel(M, N, K, gemm_config=raw)
    y = k(*(d[t].cuda() for t in ("A", "B", "bias", "gamma", "beta")))
    torch.cuda.synchronize()
    _close(y, ref, 2e-2, 2e-2, f"co-resident rounds / chunks {tile} M={M}")
    err, ctr = _cr_counters(k, M, N)
    assert err == 0 and not ctr.any()


def test_every_conv_instance(gpu):
    Nb, H, W, C, F = 2, 9, 7, 64, 64
    d = I.config4(Nb, H, W, C, F)
    ref = O.conv2d_nhwc_ref(d["X"], d["W"], 1, 1)
    X, Wt = d["X"].cuda(), d["W"].cuda()
    for idx, inst in enumerate(family_instances("conv2d")):
        for sk in (1, 3):
            if (9 * C) % (inst.bk * sk):
                continue
            raw = raw_from_inst(inst, sk)
            print(f"[parity] {inst.name} sk={sk}", flush=True)
            k = conv_mod.build_conv2d_kernel(Nb, C, H, W, F, 3, 3, 1, 1, 1, config=raw)
            Y = torch.full((Nb, H, W, F), float("nan"), dtype=torch.float16, device="cuda")
            k(X, Wt, Y)
            torch.cuda.synchronize()
            _close(Y, ref, 1e-2, 1e-2, f"{inst.name} sk={sk}")


@pytest.mark.parametrize("shape", [(32, 56, 56, 64, 64), (32, 14, 14, 256, 256), (32, 7, 7, 512, 512),
                                   (3, 5, 5, 64, 24)])
def test_config4_conv(gpu, shape):
    Nb, H, W, C, F = shape
    d = I.config4(Nb, H, W, C, F)
    ref = O.conv2d_nhwc_ref(d["X"], d["W"], 1, 1)
    k = conv_mod.build_conv2d_kernel(Nb, C, H, W, F, 3, 3, 1, 1, 1)
    print(f"[parity] config4 {shape} {k.config}", flush=True)
    Y = torch.empty((Nb, H, W, F), dtype=torch.float16, device="cuda")
    k(d["X"].cuda(), d["W"].cuda(), Y)
    torch.cuda.synchronize()
    _close(Y, ref, 1e-2, 1e-2, f"config4 {shape} {k.config}")


def test_every_fp8_instance(gpu):
    M, N, K = 40, 512, 1024
    d = I.config5(M, N, K)
    ref = O.fp8_gemm_bias_act_ref(d["A"], d["B"], d["scale_a"], d["scale_b"], d["bias"], "silu")
    A, B, bias = d["A"].cuda(), d["B"].cuda(), d["bias"].cuda()
    for idx, inst in enumerate(family_instances("gemm")):
        if inst.dtype != "fp8":
            continue
        for sk in (1, 2):
            if K % (inst.bk * sk):
                continue
            print(f"[parity] {inst.name} sk={sk}", flush=True)
            y = runtime.gemm(idx, "fp8", A, B, bias=bias, act="silu", scale_a=d["scale_a"], scale_b=d["scale_b"],
                             split_k=sk)
            torch.cuda.synchronize()
            _close(y, ref, 1e-2, 1e-2, f"{inst.name} sk={sk}")


@pytest.mark.parametrize("M", [16, 256, 4096])
@pytest.mark.parametrize("NK", [(4096, 4096), (11008, 4096), (4096, 11008)])
def test_config5_fp8(gpu, M, NK):
    N, K = NK
    d = I.config5(M, N, K)
    ref = O.fp8_gemm_bias_act_ref(d["A"], d["B"], d["scale_a"], d["scale_b"], d["bias"], "silu")
    k = fp8_mod.build_kernel(M, N, K)
    print(f"[parity] config5 M={M} N={N} K={K} {k.config}", flush=True)
    y = k(d["A"].cuda(), d["B"].cuda(), d["scale_a"], d["scale_b"], d["bias"].cuda())
    torch.cuda.synchronize()
    _close(y, ref, 1e-2, 1e-2, f"config5 M={M} N={N} K={K}")


@pytest.mark.parametrize("dtype,M,N,K,sk", [("fp8", 16, 512, 11008, 4), ("fp8", 40, 256, 11008, 8),
                                            ("f16", 61, 384, 11008, 8), ("bf16", 7, 256, 1216, 3)])
def test_uneven_split_k(gpu, dtype, M, N, K, sk):
    """split_k slices of ceil(K tiles / split_k) tiles, the last one shorter
    (K = 11008 = 86 x 128 = 172 x 64 tiles; 1216 = 19 x 64), every instance whose
    split plan is exactly sk slices."""
    from icpp_tuning_amd.kernels._base import InstanceDescriptor  # noqa: F401
    if dtype == "fp8":
        d = I.config5(M, N, K)
        ref = O.fp8_gemm_bias_act_ref(d["A"], d["B"], d["scale_a"], d["scale_b"], d["bias"], "silu")
        args = dict(act="silu", scale_a=d["scale_a"], scale_b=d["scale_b"])
    else:
        d = I.gemm_inputs(M, N, K, runtime.TORCH_DTYPE[dtype], 97, b_std=1 / math.sqrt(K), bias=True)
        ref = O.gemm_bias_act_ref(d["A"], d["B"], d["bias"], "relu")
        args = dict(act="relu")
    A, B, bias = d["A"].cuda(), d["B"].cuda(), d["bias"].cuda()
    ran = 0
    for idx, inst in enumerate(family_instances("gemm")):
        if inst.dtype != dtype or K % inst.bk:
            continue
        nkt = K // inst.bk
        per = -(-nkt // sk)
        if sk > nkt or -(-nkt // per) != sk or nkt % per == 0:
            continue  # only plans whose last slice is shorter
        print(f"[parity] {inst.name} M={M} N={N} K={K} sk={sk}", flush=True)
        y = runtime.gemm(idx, dtype, A, B, bias=bias, split_k=sk, **args)
        torch.cuda.synchronize()
        _close(y, ref, 1e-2, 1e-2, f"{inst.name} uneven sk={sk}")
        ran += 1
    assert ran > 0


@pytest.mark.parametrize("shape,sk", [((32, 56, 56, 64, 64), 1), ((32, 14, 14, 256, 256), 2),
                                      ((32, 14, 14, 256, 256), 1), ((32, 7, 7, 512, 512), 1)])
def test_conv_every_instance_full_size(gpu, shape, sk):
    """Every conv tile at two benchmark sizes (many workgroup rounds for the small
    tiles), alone and with split-K."""
    Nb, H, W, C, F = shape
    d = I.config4(Nb, H, W, C, F)
    ref = O.conv2d_nhwc_ref(d["X"], d["W"], 1, 1)
    X, Wt = d["X"].cuda(), d["W"].cuda()
    for inst in family_instances("conv2d"):
        if (9 * C) % (inst.bk * sk):
            continue
        raw = raw_from_inst(inst, sk)
        print(f"[parity] {inst.name} {shape} sk={sk}", flush=True)
        k = conv_mod.build_conv2d_kernel(Nb, C, H, W, F, 3, 3, 1, 1, 1, config=raw)
        Y = torch.full((Nb, H, W, F), float("nan"), dtype=torch.float16, device="cuda")
        k(X, Wt, Y)
        torch.cuda.synchronize()
        _close(Y, ref, 1e-2, 1e-2, f"{inst.name} {shape} sk={sk}")


@pytest.mark.parametrize("geom", [
    # (N, H, W, C, F, KH, KW, stride, pad, dilation)
    (2, 9, 7, 128, 64, 3, 3, 1, 1, 1),   # 3x3 stride 1, C = 2 x 64: per-tile-tap gather, two tiles per tap
    (3, 5, 5, 192, 72, 3, 3, 1, 1, 1),   # C = 3 x 64, F not a multiple of the tile
    (2, 7, 6, 16, 64, 2, 2, 1, 0, 1),    # K tile spans 4 filter taps (general gather path)
    (2, 9, 9, 64, 64, 3, 3, 2, 1, 1),    # stride 2
    (2, 8, 8, 64, 128, 3, 3, 1, 2, 2),   # dilation 2
    (1, 5, 5, 128, 72, 1, 1, 1, 0, 1),   # 1x1, F not a multiple of the tile
    # input halo (3x3 stride 1 pad 1, C = 64): MFMA row bands that straddle image rows
    # and images, taps outside the image redirected to the zero pixel
    (3, 9, 11, 64, 72, 3, 3, 1, 1, 1),   # W = 11, F not a multiple of the tile
    (2, 13, 5, 64, 64, 3, 3, 1, 1, 1),   # W = 5: a 256-row tile spans both images
    (1, 56, 56, 64, 64, 3, 3, 1, 1, 1),  # one image, the widest the halo holds
    (2, 6, 80, 64, 64, 3, 3, 1, 1, 1),   # W = 80: past the halo capacity of every tile, the gathers take it
])
def test_conv_geometries(gpu, geom):
    Nb, H, W, C, F, KH, KW, S, P, D = geom
    d = I.config4(Nb, H, W, C, F, KH, KW)
    ref = O.conv2d_nhwc_ref(d["X"], d["W"], S, P, D)
    X, Wt = d["X"].cuda(), d["W"].cuda()
    for idx, inst in enumerate(family_instances("conv2d")):
        for sk in (1, 2):          # split-K slices the same gathers at a K offset
            if (KH * KW * C) % (inst.bk * sk):
                continue
            raw = raw_from_inst(inst, sk)
            print(f"[parity] conv {geom} {inst.name} sk={sk}", flush=True)
            k = conv_mod.build_conv2d_kernel(Nb, C, H, W, F, KH, KW, S, P, D, config=raw)
            Y = torch.full(tuple(ref.shape), float("nan"), dtype=torch.float16, device="cuda")
            k(X, Wt, Y)
            torch.cuda.synchronize()
            _close(Y, ref, 1e-2, 1e-2, f"conv {geom} {inst.name} sk={sk}")
