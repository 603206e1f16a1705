"""PerformanceDB built from device measurements, then served by AdaptiveTuner.

The table must hand back, for each profiled shape, the fastest candidate that
was measured for it, and a config it serves for an unprofiled shape must run
and match the CPU oracle (GEMM+bias+GELU-tanh bf16: rtol 1e-2, atol 1e-2, as
the reference's gemm_bias_act.py:160).
"""

import math

import pytest
import torch

from icpp_tuning_amd import inputs as I
from icpp_tuning_amd.autotuner import get_gpu_spec
from icpp_tuning_amd.autotuner.perfdb import AdaptiveTuner, PerformanceDB, build_db, op_key
from icpp_tuning_amd.kernels import gemm_bias_act as gba_mod
from oracle import ops as O

pytestmark = pytest.mark.gpu


def test_db_from_device_measurements(gpu, tmp_path):
    desc = gba_mod.descriptor("gelu_tanh", "bf16")
    shapes = [dict(M=m, N=1024, K=1024) for m in (64, 512, 2048)]
    print(f"[perfdb] profiling {shapes}", flush=True)
    db = build_db(desc, shapes, top_k=3, budget_ms=10.0, reps=5)
    db.save(tmp_path / "db.json")
    db = PerformanceDB.load(tmp_path / "db.json")
    assert db.hw == get_gpu_spec().name and db.op == op_key(desc)
    tuner = AdaptiveTuner(desc, db)
    for s in shapes:
        recs = [r for r in db.records if r.shape == s]
        assert len(recs) >= 3
        r = tuner.select(**s)
        assert r.level == "table"
        assert r.config == min(recs, key=lambda r: r.ms).config
    # an unprofiled M inside the profiled range is served from the table and computes correctly
    M, N, K = 300, 1024, 1024
    r = tuner.select(M=M, N=N, K=K)
    assert r.level == "table"
    d = I.gemm_inputs(M, N, K, torch.bfloat16, 77, b_std=1 / math.sqrt(K), bias=True)
    ref = O.gemm_bias_act_ref(d["A"], d["B"], d["bias"], "gelu_tanh")
    k = gba_mod.build_kernel(M, N, K, config=r.config, act="gelu_tanh", dtype="bf16")
    print(f"[perfdb] M={M} table config {desc.format_config(r.config)}", flush=True)
    y = k(d["A"].cuda(), d["B"].cuda(), d["bias"].cuda())
    torch.cuda.synchronize()
    err = (y.float().cpu() - ref.float()).abs()
    assert bool((err <= 1e-2 + 1e-2 * ref.float().abs()).all()), float(err.max())
    assert tuner.select(M=1 << 15, N=N, K=K).level == "formula"
