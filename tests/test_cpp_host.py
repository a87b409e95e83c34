"""The C++ host side through its test binaries:

- tests/cpp/test_gpu_host: the host API (nano-vllm-rs_amd/host/gpu.hpp):
  its argument contract on the CPU, and the reference's own GPU tests
  (src/gpu.rs:1148-1472) restated in C++ on a GPU;
- tests/cpp/test_model: the Qwen3 runner (host/model.hpp): the step record and
  config checks on the CPU; on a GPU the batch contract, the fused-attention
  choice, the forward against the CPU oracle stage by stage, fused against
  split attention, graph replay against the eager forward and decode against
  prefill;
- tests/cpp/candidate_floor_check: the sampler's direct candidate floor
  against the binary search it replaces (host only)."""
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


def test_candidate_floor_direct_form_equals_search():
    """sample.hip's candidate floor from bound * T and a few predicate steps
    gives the same bits as the binary search over every bf16 key."""
    out = _run("candidate_floor_check", "2000000")
    assert " 0 mismatches" in out, out


def test_cpp_model_metadata_and_config():
    out = _run("test_model", "cpu")
    assert "FAILED" not in out
    assert "step_record_layout_fill_and_table_padding ... ok" in out


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
    for name in ("plan_rejects_invalid_batches", "plan_fuses_attention_only_for_independent_rows",
                 "forward_matches_the_oracle_stage_by_stage", "decode_graphs_replay_the_eager_forward",
                 "fused_and_split_attention_give_identical_steps", "decode_step_matches_prefill_of_the_longer_prompt",
                 "model_reports_memory_and_keeps_graphs_per_batch_size"):
        assert name + " ..." in out
