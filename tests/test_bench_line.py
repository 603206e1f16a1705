"""bench.py's last stdout line: compact, parseable, carrying the driver's keys.

The driver reads only the tail of stdout, so the headline record must stay a
short final line even with every per-op row summarised in it."""

import json

import bench


def _head():
    return {
        "metric": bench.METRIC, "value": 1130.5, "unit": "TFLOP/s", "n_gpus": 1, "steps": 20, "warmup": 5,
        "ms_per_step": 0.12155, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) / N(0,1/sqrt(K)))",
        "config": {"workload": "gemm_bias_gelu_tanh_4096x4096x4096_bf16", "M": 4096, "N": 4096, "K": 4096,
                   "op": "gemm+bias+gelu_tanh", "tile": "BM256_BN256_BK64_S2_T512_W2x4_M16_PP",
                   "input_copies": 7, "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "achieved": 1135.7, "peak": 2516.6, "unit": "TFLOP/s", "frac": 0.4513,
                     "traffic": 235180000, "traffic_source": "t" * 260, "kernel_us": 121.02, "peak_sclk_mhz": 2400.0, "sclk_mhz": 1650.3,
                     "peak_at_sclk": 1730.5, "frac_at_sclk": 0.6563, "sclk_window_s": 0.2},
        "tuner": {"time_to_best_s": 1.234, "prune_rank_s": 0.0123, "compile_s": 0.0011, "bench_s": 1.2,
                  "formula_top1": "BM256_BN256_BK64_S2_T512_W2x4_M32", "formula_top1_ms": 0.1234,
                  "select_best_s": 0.0101, "candidates": 4},
    }


def _rows():
    rows = []
    def g(op, shape, bound="mfma", cfg="BM128_BN128_BK64_SK4_S2_T256_W2x2_M16_PP"):
        rows.append({"op": op, "shape": shape, "dtype": "f16", "config": cfg, "raw_config": {"block_M": 128},
                     "ms": 0.0123456, "tflops": 1234.56, "pct_mfma_peak": 49.06, "gbps": 4567.8,
                     "pct_hbm": 57.1, "bound": bound, "tuner": {"time_to_best_s": 0.5}})
    g("gemm", {"M": 1024, "N": 1024, "K": 1024})
    for a in ("gelu_tanh", "relu", "silu"):
        g(f"gemm_bias_{a}", {"M": 4096, "N": 4096, "K": 4096})
    for n in (768, 1024, 4096):
        g("gemm_bias_layernorm", {"M": 8192, "N": n, "K": 4096})
    for (h, c) in ((56, 64), (14, 256), (7, 512)):
        for op in ("conv2d", "conv2d_bn_relu", "conv_bn_add_relu"):
            g(op, dict(N=32, C=c, H=h, W=h, OC=c, KH=3, KW=3, stride=1, padding=1))
    for n in (1024, 4096, 12288):
        rows.append({"op": "softmax", "shape": {"M": 4096, "N": n}, "dtype": "f32", "input_copies": 16,
                     "ms": 0.0123, "gbps": 5000.1, "pct_hbm": 62.5, "bound": "hbm"})
    for n in (1024, 4096, 8192, 15872):
        for op in ("layernorm_fwd", "layernorm_bwd"):
            rows.append({"op": op, "shape": {"M": 4096, "N": n}, "dtype": "f16", "input_copies": 16,
                         "ms": 0.0123, "gbps": 5000.1, "pct_hbm": 62.5, "bound": "hbm"})
    for (b, s) in ((1, 128), (32, 128), (8, 512)):
        rows.append({"op": "bert_base_e2e", "shape": {"batch": b, "seq": s, "layers": 12}, "dtype": "f16",
                     "ms": 1.2345, "torch_composition_ms": 2.3456, "speedup": 1.9, "tflops": 123.4})
    for m in (16, 256, 4096):
        for (n, k) in ((4096, 4096), (11008, 4096), (4096, 11008)):
            g("fp8_gemm_bias_silu", {"M": m, "N": n, "K": k}, bound="hbm" if m < 4096 else "mfma",
              cfg="BM16_BN128_BK512_SK8_S2_T256_W1x4_M16")
    return rows


def _cpu():
    per = {k: {"tflops": 1.2345, "seconds": 1.0, "sample": "x" * 90} for k in
           ("gemm_1024_f16", "gemm_bias_gelu_tanh_4096_bf16", "gemm_bias_layernorm_8192x1024x4096_f16",
            "conv2d_b32_56x56x64_f16", "fp8_gemm_bias_silu_256x4096x4096")}
    return {"value": 1.2345, "unit": "TFLOP/s", "cores": 16, "kind": "port",
            "cpu_model": "AMD EPYC 9575F 64-Core Processor", "sample": "y" * 160, "per_op": per}


def test_final_line_is_compact_and_complete():
    line = bench.final_line(_head(), _rows(), _cpu())
    assert "\n" not in line
    assert len(line) <= bench.FINAL_LINE_MAX, len(line)
    d = json.loads(line)
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline", "tuner"):
        assert k in d, k
    assert d["config"]["workload"] == "gemm_bias_gelu_tanh_4096x4096x4096_bf16"
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic", "kernel_us", "sclk_mhz", "frac_at_sclk"):
        assert k in d["roofline"], k
    cb = d["cpu_baseline"]
    for k in ("value", "unit", "cores", "kind", "sample", "cpu_model"):
        assert k in cb, k
    assert len(cb["per_op_tflops"]) == 5
    # every per-op row is summarised, configs kept while the line fits
    assert len(d["ops"]) == len(_rows())
    assert all("us" in e for e in d["ops"])


def test_final_line_without_ops_or_cpu():
    d = json.loads(bench.final_line(_head()))
    assert d["value"] == 1130.5 and "ops" not in d and "cpu_baseline" not in d


def test_final_line_drops_detail_before_exceeding_the_limit():
    rows = _rows() * 3
    line = bench.final_line(_head(), rows, _cpu())
    assert len(line) <= bench.FINAL_LINE_MAX
    assert json.loads(line)["roofline"]["frac"] == 0.4513


def test_untimed_formula_pick_is_null_not_nan():
    # the tuner reports NaN for a formula pick it did not time; the line must stay strict JSON
    assert bench._finite(float("nan"), 5) is None and bench._finite(None, 5) is None
    assert bench._finite(0.123456789, 5) == 0.12346
    h = _head()
    h["tuner"]["formula_top1_ms"] = bench._finite(float("nan"), 5)
    line = bench.final_line(h, _rows(), _cpu())
    assert "NaN" not in line
    assert json.loads(line)["tuner"]["formula_top1_ms"] is None


def test_traffic_is_reported_only_for_the_profiled_tile():
    from pathlib import Path
    prof = json.loads((Path(bench.__file__).parent / "profiles" /
                       "traffic_gemm_bias_gelu_tanh_4096x4096x4096_bf16.json").read_text())
    b, src = bench._load_traffic("gemm_bias_gelu_tanh_4096x4096x4096_bf16", prof["tile"])
    assert b == prof["bytes_per_launch"] and prof["tile"] in src and "FETCH_SIZE" in src
    b, src = bench._load_traffic("gemm_bias_gelu_tanh_4096x4096x4096_bf16", "BM64_BN64_BK64_S2_T256_W2x2_M16")
    assert b is None and "profiled on tile" in src
    b, src = bench._load_traffic("no_such_workload", "x")
    assert b is None and "absent" in src
