"""The reference's candidate grids and descriptor adjustments, restated.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Used to run the restated
cost model (icpp_tuning_amd.autotuner.cost_model) in A100 reference mode and
compare its argmax and scores with the published evaluation CSVs.
"""

from __future__ import annotations

import itertools
import math
import re

from icpp_tuning_amd.autotuner.cost_model import TuneConfig, make_conv2d_spec, make_matmul_spec


def gemm_configs(M, K, split_k_values=(2,)):
    """reference kernel/tilelang/gemm/gemm.py:24-48"""
    out = []
    for bm, bn, bk, sk, ns, tn in itertools.product([16, 32, 64], [128, 256], [32, 64, 128], split_k_values,
                                                   [1, 2, 4, 8], [64, 128, 256]):
        if K % sk or (K // sk) % bk:
            continue
        out.append({"block_M": bm, "block_N": bn, "block_K": bk, "split_k": sk, "num_stages": ns, "thread_num": tn})
    return out


def bias_act_configs(M, K):
    """reference gemm_bias_act.py:20-41 (identical grid in gemm_bias_layernorm.py:19-40)"""
    out = []
    for bm, bn, bk, ns, tn in itertools.product([16, 32, 64], [64, 128, 256], [32, 64], [1, 2], [128, 256]):
        if K % bk:
            continue
        out.append({"block_M": bm, "block_N": bn, "block_K": bk, "num_stages": ns, "thread_num": tn})
    return out


def conv_configs():
    """reference conv2d.py:186-205 (no filtering)"""
    return [{"block_M": bm, "block_N": bn, "block_K": bk, "num_stages": ns, "thread_num": tn}
            for bm, bn, bk, ns, tn in itertools.product([16, 32, 64], [64, 128, 256], [32, 64], [1, 2], [128, 256])]


def to_tune_config(raw):
    """reference interface.py:92-103 (thread_num // 32 warps)"""
    return TuneConfig(block_M=raw["block_M"], block_N=raw["block_N"], block_K=raw["block_K"],
                      num_stages=raw["num_stages"], num_warps=raw["thread_num"] // 32)


def op_spec(op, raw, M, N, K):
    """reference descriptors: gemm.py:102-104 (K // split_k), gemm_bias_act.py:109-110,
    gemm_bias_layernorm.py:201-202"""
    if op == "gemm":
        return make_matmul_spec(M=M, N=N, K=K // raw.get("split_k", 2))
    if op == "gemm_bias_act":
        return make_matmul_spec(M=M, N=N, K=K, primitives=["bias_add", "relu"])
    if op == "gemm_bias_layernorm":
        return make_matmul_spec(M=M, N=N, K=K, primitives=["bias_add", "row_layernorm"])
    raise ValueError(op)


def adjust(op, raw, score):
    """reference gemm.py:109-111 (score * sqrt(sk) / sk); identity elsewhere (interface.py:105-115)"""
    if op == "gemm":
        sk = raw.get("split_k", 2)
        return score * math.sqrt(sk) / sk
    return score


def configs_for(op, M, K):
    return gemm_configs(M, K) if op == "gemm" else bias_act_configs(M, K)


def conv_spec(N, C, H, W, F, KH, KW, stride, pad):
    """reference conv2d.py:472-473"""
    return make_conv2d_spec(N, C, H, W, F, KH, KW, stride=stride, padding=pad)


def format_config(raw):
    """reference interface.py:117-128"""
    parts = [f"BM{raw['block_M']}", f"BN{raw['block_N']}", f"BK{raw['block_K']}"]
    if "split_k" in raw:
        parts.append(f"SK{raw['split_k']}")
    parts += [f"S{raw['num_stages']}", f"T{raw['thread_num']}"]
    return "_".join(parts)


def parse_config(s):
    d = {}
    for key, val in re.findall(r"(BM|BN|BK|SK|S|T)(\d+)", s):
        d[{"BM": "block_M", "BN": "block_N", "BK": "block_K", "SK": "split_k", "S": "num_stages",
           "T": "thread_num"}[key]] = int(val)
    return d
