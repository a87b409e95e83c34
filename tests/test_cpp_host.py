"""The C++ host API (nano-vllm-rs_amd/host/gpu.hpp, the mirror of
src/gpu.rs) through its test binary tests/cpp/test_gpu_host: the argument
checks on the CPU, and the reference's own GPU tests (src/gpu.rs:1148-1472)
restated in C++ on a GPU."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_gpu_host")


def _run(suite: str) -> str:
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is missing: build it with __graft_entry__.build()")
    result = subprocess.run([BIN, suite], capture_output=True, text=True, timeout=600)
    assert result.returncode == 0, result.stdout + result.stderr
    return result.stdout


def test_cpp_host_argument_checks():
    out = _run("cpu")
    assert "FAILED" not in out and " passed" in out


@pytest.mark.gpu
def test_cpp_host_reference_gpu_tests():
    out = _run("gpu")
    assert "FAILED" not in out
    for name in ("gpu_views_keep_allocations_and_reject_overlap", "gpu_parallel_sampler_matches_serial",
                 "gpu_cached_rope_matches_direct_at_context_boundary", "gpu_gemm_rms_sampling_graph",
                 "gpu_causal_paged_attention_and_rope", "gpu_ragged_gqa_matches_cpu"):
        assert name in out
