"""C-ABI surface and host-mirror checks that need no GPU.

- libnano_hip.so loads and exports every function include/nano_hip.h declares,
  and the host wrapper (nvr.py) declares a signature for each of them;
- host-only entry points (nv_sampling_seed, nv_last_error) work without a GPU;
- the wrapper's argument contract (dimensions, extents, alignment, buffer
  ownership, overlapping outputs, scalars, head layouts), each rejection by
  the rule it breaks.
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


def test_rust_build_snippet_compiles_every_source():
    """The build.rs that INTEGRATION.md gives the Rust host lists its .hip
    files by name; it must name exactly the library's sources, or a symbol
    the header declares would be missing from a Rust build."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    listed = re.search(r"let sources = \[([^\]]*)\]", text)
    assert listed, "INTEGRATION.md has no build.rs source list"
    names = set(re.findall(r'"([a-z_]+)"', listed.group(1)))
    csrc = os.path.join(ROOT, "nano-vllm-rs_amd", "csrc")
    sources = {f[:-4] for f in os.listdir(csrc) if f.endswith(".hip")}
    assert names == sources


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
def _fake_gpu():
    """A Gpu with no device behind it: argument admission only (no kernel runs)."""
    g = object.__new__(nvr.Gpu)
    g._device = nvr._Device(None, 0)
    g.lib = None
    return g


def _fake_buffer(gpu, nbytes):
    return nvr.Buffer(nvr._Memory(gpu._device, None, nbytes), 0, nbytes)  # address None: nothing is freed


def _fault(fault, fn, *args):
    with pytest.raises(nvr.ArgumentError) as e:
        fn(*args)
    assert e.value.fault == fault, str(e.value)


def test_views_and_argument_admission():
    gpu = _fake_gpu()
    packed = _fake_buffer(gpu, 32)
    tokens, adjacent, straddling = packed.slice(0, 8), packed.slice(8, 8), packed.slice(4, 8)
    assert not tokens.overlaps(adjacent) and tokens.overlaps(straddling)
    _fault("extent", tokens.slice, 4, 8)  # past the end of the view
    _fault("extent", packed.slice, 2**64 - 1, 1)
    weights, out = _fake_buffer(gpu, 8), _fake_buffer(gpu, 4)
    _fault("alignment", gpu.embedding, packed.slice(1, 8), weights, out, 2, 1, 4)
    _fault("overlap", gpu.embedding, tokens, weights, weights.slice(0, 4), 2, 1, 4)
    _fault("extent", gpu.embedding, tokens, weights, out, 3, 1, 4)
    _fault("dimension", gpu.embedding, tokens, weights, out, 0, 1, 4)
    _fault("dimension", gpu.embedding, tokens, weights, out, 2**31, 1, 4)
    _fault("foreign", gpu.embedding, tokens, weights, _fake_buffer(_fake_gpu(), 4), 2, 1, 4)
    # Only the bytes an argument covers count: a written view that shares the
    # allocation, but not the bytes, of an input is accepted up to the C call.
    with pytest.raises(AttributeError):  # the fake Gpu has no library to call
        gpu.embedding(tokens, weights, packed.slice(16, 4), 2, 1, 4)


def test_kernel_wrappers_reject_bad_scalars_and_layouts():
    gpu = _fake_gpu()
    x, w, out = _fake_buffer(gpu, 8 * 1024 * 2), _fake_buffer(gpu, 1024 * 2), _fake_buffer(gpu, 8 * 1024 * 2)
    for eps in (0.0, -1.0, float("nan"), float("inf")):
        _fault("value", gpu.rms_norm, x, w, out, 8, 1024, eps)
    _fault("overlap", gpu.rms_norm, x, w, x, 8, 1024, 1e-6)  # out is x
    _fault("value", nvr.require_head_layout, 16, 3, 128)  # q heads do not group over KV heads
    _fault("value", nvr.require_head_layout, 16, 8, 129)  # odd head dim
    _fault("value", nvr.require_head_layout, 16, 8, 258)  # above 256
    _fault("value", nvr.require_head_layout, 65535, 1, 128)
    logits = _fake_buffer(gpu, 2 * 151936 * 2)
    small = _fake_buffer(gpu, 16)
    # scratch needs batch * ceil(vocab / 2048) entries
    _fault("extent", gpu.sample_parallel, logits, small, small.slice(0, 16), _fake_buffer(gpu, 8), _fake_buffer(gpu, 16),
           _fake_buffer(gpu, 16), 2, 151936)
    kc = _fake_buffer(gpu, 1 << 20)
    _fault("value", gpu.paged_attention, x, kc, kc, small, small, small, out, 1, 16, 8, 128, 16, 1, 1, 1, 5000)


def test_capture_state_is_tracked_per_gpu():
    gpu = _fake_gpu()
    gpu._device.recording = {}
    _fault("value", gpu.capture, lambda: None)  # a capture inside a capture


def test_bf16_helpers_round_trip():
    x = np.array([1.0, -2.5, 3.140625, 65536.0], np.float32)
    assert np.array_equal(nvr.bf16_values(nvr.bf16_bits(x)), x)
    assert nvr.bf16_bits(np.float32(1.0 + 2**-8)).item() == 0x3F80


def test_tile_gate_up_rows_order():
    """Tile t of the reordered weight holds gate rows 8t..8t+7, then up rows 8t..8t+7."""
    inter, k = 24, 3
    w = np.arange(2 * inter * k, dtype=np.uint16).reshape(2 * inter, k)
    t = nvr.tile_gate_up_rows(w, inter)
    for tile in range(inter // 8):
        for e in range(8):
            assert (t[16 * tile + e] == w[8 * tile + e]).all()
            assert (t[16 * tile + 8 + e] == w[inter + 8 * tile + e]).all()
