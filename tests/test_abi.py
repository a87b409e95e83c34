"""C-ABI surface and host-mirror checks that need no GPU.

- libnano_hip.so loads and exports every function include/nano_hip.h declares,
  and the host wrapper (nvr.py) declares a signature for each of them;
- host-only entry points (nv_sampling_seed, nv_last_error) work without a GPU;
- the wrapper's validation (extents, alignment, aliasing, capture rules)
  mirrors src/gpu.rs:222-509 and rejects what the reference rejects.
"""
import os
import re
import subprocess

import numpy as np
import pytest

import nvr
import oracle as ora

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nano_hip.h")

# The reference's Rust side binds exactly these (src/gpu.rs:17-178).
REFERENCE_SYMBOLS = {
    "nv_stream", "nv_sm_count", "nv_last_error", "nv_create", "nv_destroy", "nv_alloc", "nv_free", "nv_upload",
    "nv_download", "nv_sync", "nv_mem_info", "nv_capture_begin", "nv_capture_end", "nv_capture_abort",
    "nv_graph_replay", "nv_graph_destroy", "nv_gemm", "nv_embedding", "nv_rms", "nv_add_rms", "nv_qkv_rope",
    "nv_rope_cache", "nv_qkv_rope_cached", "nv_attention", "nv_silu", "nv_gather", "nv_sample",
    "nv_sample_parallel",
}


def header_functions() -> set[str]:
    text = open(HEADER).read()
    return set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*(nv_[a-z0-9_]+)\s*\(", text, re.M))


def test_header_covers_reference_abi():
    declared = header_functions()
    assert REFERENCE_SYMBOLS <= declared
    assert declared == set(nvr.SIGNATURES)


def test_library_exports_every_declared_symbol():
    assert os.path.exists(nvr.LIB_PATH), "build with __graft_entry__.build() first"
    out = subprocess.run(["nm", "-D", "--defined-only", nvr.LIB_PATH], capture_output=True, text=True, check=True)
    exported = {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}
    missing = header_functions() - exported
    assert not missing, missing
    lib = nvr.library()  # declares every argtype; fails if a symbol is absent
    assert lib.nv_last_error() is not None


def test_host_seed_function_matches_oracle():
    for args in [(0, 0, 0), (0, 5, 3), (1234, 17, 100), (2**64 - 1, 1, 2)]:
        assert nvr.sampling_seed(*args) == ora.sampling_seed(*args)


def test_library_has_no_oracle_dependency():
    out = subprocess.run(["ldd", nvr.LIB_PATH], capture_output=True, text=True, check=True).stdout
    assert "oracle" not in out
    uses = re.compile(r"import\s+oracle|from\s+oracle|liboracle|oracle\.h|oracle/")
    src = os.path.join(ROOT, "nano-vllm-rs_amd")
    for dirpath, _, files in os.walk(src):
        for f in files:
            if f.endswith((".hip", ".h", ".py", ".cpp", "Makefile")):
                assert not uses.search(open(os.path.join(dirpath, f)).read()), f


# -------------------------------------------------- host-side validation ----
class _FakeContext:
    def __init__(self):
        self.capturing = False
        self.captured = []

    def outside_capture(self):
        if self.capturing:
            raise ValueError("allocation, transfer and synchronization are forbidden during graph capture")


def _fake_gpu():
    g = object.__new__(nvr.Gpu)
    g.context = _FakeContext()
    g.lib = None
    return g


def _fake_buffer(ctx, nbytes, ptr=0x10000):
    alloc = object.__new__(nvr._Allocation)
    alloc.context, alloc.ptr, alloc.bytes = ctx, None, nbytes  # ptr None: __del__ frees nothing
    alloc.ptr_value = ptr
    return nvr.Buffer(alloc, 0, nbytes)


def test_views_alignment_and_aliasing_rules():
    """Host half of src/gpu.rs:1169-1192."""
    gpu = _fake_gpu()
    packed = _fake_buffer(gpu.context, 32)
    tokens = packed.slice(0, 8)
    adjacent = packed.slice(8, 8)
    nvr.Gpu.distinct(tokens, [adjacent])  # adjacent views do not overlap
    with pytest.raises(ValueError):
        nvr.Gpu.distinct(tokens, [packed.slice(4, 8)])
    with pytest.raises(ValueError):
        tokens.slice(4, 8)  # past the end of the view
    with pytest.raises(ValueError):
        packed.slice(2**64 - 1, 1)
    with pytest.raises(ValueError):
        gpu.tensor(packed.slice(1, 8), [1], 4)  # misaligned i32 view
    gpu.tensor(packed.slice(4, 8), [2], 4)
    with pytest.raises(ValueError):
        gpu.tensor(packed, [0], 4)  # zero dimension
    with pytest.raises(ValueError):
        gpu.tensor(packed, [9], 4)  # extent beyond the buffer
    other = _fake_buffer(_FakeContext(), 32)
    with pytest.raises(ValueError):
        gpu.tensor(other, [1], 4)  # different context


def test_kernel_wrappers_reject_bad_arguments_before_calling():
    gpu = _fake_gpu()
    ctx = gpu.context
    x = _fake_buffer(ctx, 8 * 1024 * 2)
    w = _fake_buffer(ctx, 1024 * 2)
    with pytest.raises(ValueError):
        gpu.rms_norm(x, w, x, 8, 1024, 1e-6)  # out aliases x
    out = _fake_buffer(ctx, 8 * 1024 * 2)
    for eps in (0.0, -1.0, float("nan"), float("inf")):
        with pytest.raises(ValueError):
            gpu.rms_norm(x, w, out, 8, 1024, eps)
    with pytest.raises(ValueError):
        gpu.rms_norm(x, w, out, 9, 1024, 1e-6)  # x too small for 9 rows
    with pytest.raises(ValueError):
        nvr.Gpu._heads(16, 3, 128)  # qh % kvh != 0
    with pytest.raises(ValueError):
        nvr.Gpu._heads(16, 8, 129)  # odd head dim
    with pytest.raises(ValueError):
        nvr.Gpu._heads(16, 8, 258)
    logits = _fake_buffer(ctx, 2 * 151936 * 2)
    small = _fake_buffer(ctx, 16)
    with pytest.raises(ValueError):  # scratch needs batch * ceil(vocab / 2048) entries
        gpu.sample_parallel(logits, small, small, _fake_buffer(ctx, 8), small, small, 2, 151936)


def test_capture_forbids_transfers():
    ctx = _FakeContext()
    ctx.capturing = True
    with pytest.raises(ValueError):
        ctx.outside_capture()


def test_bf16_helpers_round_trip():
    x = np.array([1.0, -2.5, 3.140625, 65536.0], np.float32)
    assert np.array_equal(nvr.bf16_values(nvr.bf16_bits(x)), x)
    assert nvr.bf16_bits(np.float32(1.0 + 2**-8)).item() == 0x3F80
