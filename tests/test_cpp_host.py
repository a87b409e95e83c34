"""The C++ host side through its test binaries:

- tests/cpp/test_gpu_host: the host API (nano-vllm-rs_amd/host/gpu.hpp, the
  mirror of src/gpu.rs): argument checks on the CPU, and the reference's own
  GPU tests (src/gpu.rs:1148-1472) restated in C++ on a GPU;
- tests/cpp/test_model: the Qwen3 runner (host/model.hpp, the mirror of
  src/model.rs): the packed-metadata test of src/model.rs:1232-1297 and config
  checks on the CPU; batch validation, graph replay against the eager forward
  and decode against prefill on a GPU."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(binary: str, suite: str) -> str:
    path = os.path.join(ROOT, "tests", "cpp", "_build", binary)
    if not os.path.exists(path):
        pytest.fail(f"{path} is missing: build it with __graft_entry__.build()")
    result = subprocess.run([path, suite], capture_output=True, text=True, timeout=600)
    assert result.returncode == 0, result.stdout + result.stderr
    return result.stdout


def test_cpp_host_argument_checks():
    out = _run("test_gpu_host", "cpu")
    assert "FAILED" not in out and " passed" in out


def test_cpp_model_metadata_and_config():
    out = _run("test_model", "cpu")
    assert "FAILED" not in out
    assert "packed_metadata_preserves_values_alignment_and_clears_table_padding ... ok" in out


@pytest.mark.gpu
def test_cpp_host_reference_gpu_tests():
    out = _run("test_gpu_host", "gpu")
    assert "FAILED" not in out
    for name in ("gpu_views_keep_allocations_and_reject_overlap", "gpu_parallel_sampler_matches_serial",
                 "gpu_cached_rope_matches_direct_at_context_boundary", "gpu_gemm_rms_sampling_graph",
                 "gpu_causal_paged_attention_and_rope", "gpu_ragged_gqa_matches_cpu"):
        assert name in out


@pytest.mark.gpu
def test_cpp_model_forward():
    out = _run("test_model", "gpu")
    assert "FAILED" not in out
    for name in ("model_rejects_invalid_batches_like_the_reference", "decode_graphs_replay_the_eager_forward",
                 "decode_step_matches_prefill_of_the_longer_prompt",
                 "model_reports_memory_and_keeps_graphs_per_batch_size"):
        assert name + " ..." in out
