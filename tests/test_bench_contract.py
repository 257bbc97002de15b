"""bench.py's contract, checked on the CPU: the workload it measures, the algorithmic-flop
definitions behind its figures, and its refusal of more than one GPU."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def test_headline_workload_is_the_wan14b_block():
    # q, k, v, o 5120 -> 5120 and ffn 5120 -> 13824 -> 5120 at 32760 tokens, rank 32
    # (src/models/wan21/config.jl:36-45)
    assert bench.TOKENS == 32760 and bench.RANK == 32
    assert [(K, N) for (_, K, N) in bench.PROJECTIONS] == [(5120, 5120)] * 4 + [(5120, 13824), (13824, 5120)]
    assert [(K, N) for (_, K, N) in bench.PROJECTIONS_13B] == [(1536, 1536)] * 4 + [(1536, 8960), (8960, 1536)]


def test_flop_definitions():
    # forward 2MNK + 2Mr(K+N); dX 2MNK + 2Mr(N+K); dA 2MrK; dB 2MrN: 4MNK + 6Mr(K+N) in all
    M, K, N, r = 7, 11, 13, 3
    assert bench.linear_flops(M, K, N, r) == 4 * M * N * K + 6 * M * r * (K + N)
    # the GEMM launches carry the base product and the fused up-projection of their direction
    assert bench.gemm_flops("fwd", M, K, N, r) == 2 * M * N * K + 2 * M * r * N
    assert bench.gemm_flops("dx", M, K, N, r) == 2 * M * N * K + 2 * M * r * K
    # the headline step: 3.2786e13 flops (six projections at 32760 tokens, rank 32)
    step = sum(bench.linear_flops(bench.TOKENS, K, N, bench.RANK) for (_, K, N) in bench.PROJECTIONS)
    assert abs(step - 3.2786e13) / 3.2786e13 < 1e-4
    f, b = bench.attention_flops(1, 32760, 32760, 40, 128)
    assert f == 4.0 * 40 * 32760 * 32760 * 128 and b == 2.5 * f


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "exactly one GPU" in r.stderr
