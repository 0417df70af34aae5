"""bench.py's contract on the CPU: the single-GPU refusal and argument checks run before anything touches a GPU,
and the FLOP and byte counts behind `roofline` equal the workload's published figures (per token-head, chunk 64:
F_fwd = 2C(3K+2V) + 6KV = 180,224 at K = V = 128, 311,296 at K = 128, V = 256, 65,536 at K = V = 64; the
fwd+bwd step counts 3 F_fwd; its minimum HBM traffic is 2,840 bytes at K = V = 128 bf16)."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def run_bench(*args, env_extra=None):
    env = dict(os.environ, **(env_extra or {}))
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          env=env, timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = run_bench("--gpus", "2")
    assert r.returncode == 2
    assert "single GPU" in r.stderr and "--gpus 1" in r.stderr
    assert r.stdout == ""  # no JSON line for a run that did not happen


def test_world_size_above_one_is_refused():
    r = run_bench(env_extra={"WORLD_SIZE": "8"})
    assert r.returncode == 2 and "single GPU" in r.stderr


def test_unknown_workload_is_an_argument_error():
    r = run_bench("--only", "train,bogus")
    assert r.returncode != 0 and "bogus" in r.stderr


@pytest.mark.parametrize("K,V,expected", [(128, 128, 180_224), (128, 256, 311_296), (64, 64, 65_536)])
def test_forward_flops_per_token_head(K, V, expected):
    assert bench.f_fwd(K, V) == expected


def test_step_counts_match_the_published_figures():
    assert 3 * bench.f_fwd(128, 128) == 540_672
    assert 3 * bench.f_fwd(128, 256) == 933_888
    assert bench.algo_bytes_step(128, 128) == 2_840
    # B8 T4096 H16: 2.835e11 FLOPs and 1.489e9 bytes per step
    th = 8 * 4096 * 16
    assert 3 * bench.f_fwd(128, 128) * th == 283_467_841_536
    assert bench.algo_bytes_step(128, 128) * th == 1_488_977_920

