"""C-ABI surface and host-mirror checks that need no GPU.

- libnano_hip.so loads and exports every function include/nano_hip.h declares,
  and the host wrapper (nvr.py) declares a signature for each of them;
- host-only entry points (nv_sampling_seed, nv_last_error) work without a GPU;
- the wrapper's argument contract (dimensions, extents, alignment, buffer
  ownership, overlapping outputs, scalars, head layouts), each rejection by
  the rule it breaks.
"""
import ctypes
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


# Argument and return types of every extern the reference's Rust side
# declares (src/gpu.rs:17-178), transcribed by hand: `*mut c_void` context ->
# ctx, `*const c_void` -> const void*, `*mut c_void` -> void*,
# `*mut *mut c_void` -> void**, `*mut c_int` -> int*, `*mut usize` -> size_t*,
# c_int -> int, f32 -> float, usize -> size_t, `*const c_char` -> const char*.
_C, _M = "const void*", "void*"
REFERENCE_EXTERNS = {
    "nv_stream": ("int", ["ctx", "void**"]),                          # src/gpu.rs:18
    "nv_sm_count": ("int", ["ctx", "int*"]),                          # :19
    "nv_last_error": ("const char*", []),                             # :20
    "nv_create": ("int", ["int", "void**"]),                          # :21
    "nv_destroy": ("void", ["ctx"]),                                  # :22
    "nv_alloc": ("int", ["ctx", "size_t", "void**"]),                 # :23
    "nv_free": ("void", ["ctx", _M]),                                 # :24
    "nv_upload": ("int", ["ctx", _M, _C, "size_t"]),                  # :25-26
    "nv_download": ("int", ["ctx", _C, _M, "size_t"]),                # :27-32
    "nv_sync": ("int", ["ctx"]),                                      # :33
    "nv_mem_info": ("int", ["ctx", "size_t*", "size_t*"]),            # :34
    "nv_capture_begin": ("int", ["ctx"]),                             # :35
    "nv_capture_end": ("int", ["ctx", "void**"]),                     # :36
    "nv_capture_abort": ("void", ["ctx"]),                            # :37
    "nv_graph_replay": ("int", ["ctx", _M]),                          # :38
    "nv_graph_destroy": ("void", ["ctx", _M]),                        # :39
    "nv_gemm": ("int", ["ctx", _C, _C, _M, "int", "int", "int"]),     # :40-48
    "nv_embedding": ("int", ["ctx", _C, _C, _M, "int", "int", "int"]),  # :49-57
    "nv_rms": ("int", ["ctx", _C, _C, _M, "int", "int", "float"]),    # :58-66
    "nv_add_rms": ("int", ["ctx", _C, _M, _C, _M, "int", "int", "float"]),  # :67-76
    "nv_qkv_rope": ("int", ["ctx"] + [_C] * 5 + [_M] * 3 + ["int"] * 6 + ["float", "float"]),  # :77-95
    "nv_rope_cache": ("int", ["ctx", _M, "int", "int", "float"]),     # :96-102
    "nv_qkv_rope_cached": ("int", ["ctx"] + [_C] * 5 + [_M] * 3 + ["int"] * 6 + ["float", _C, "int"]),  # :103-122
    "nv_attention": ("int", ["ctx"] + [_C] * 6 + [_M] + ["int"] * 9),  # :123-141
    "nv_silu": ("int", ["ctx", _C, _M, "int", "int"]),                # :142-148
    "nv_gather": ("int", ["ctx", _C, _C, _M, "int", "int", "int"]),   # :149-157
    "nv_sample": ("int", ["ctx", _C, _C, _C, _M, "int", "int"]),      # :158-166
    "nv_sample_parallel": ("int", ["ctx", _C, _C, _C, _M, _M, _M, "int", "int"]),  # :167-177
}


def header_signatures() -> dict[str, tuple[str, list[str]]]:
    """{name: (return type, [parameter types])} of every nv_* declaration in the
    header, parameter names dropped, `nv_context*` written as ctx."""
    text = re.sub(r"/\*.*?\*/", " ", open(HEADER).read(), flags=re.S)
    out = {}
    for ret, name, params in re.findall(r"((?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**)\s*(nv_[a-z0-9_]+)\s*\(([^)]*)\)\s*;",
                                        text):
        types = []
        for param in [q.strip() for q in params.split(",")]:
            if param in ("", "void"):
                continue
            t = re.sub(r"\s*\b[A-Za-z_][A-Za-z0-9_]*$", "", param)  # drop the parameter name
            t = re.sub(r"\s*\*", "*", t).strip()
            types.append({"nv_context*": "ctx", "nv_context**": "void**"}.get(t, t))
        out[name] = (re.sub(r"\s*\*", "*", ret).strip(), types)
    return out


CTYPE_OF = {"ctx": ctypes.c_void_p, "void*": ctypes.c_void_p, "const void*": ctypes.c_void_p,
            "void**": ctypes.POINTER(ctypes.c_void_p), "int*": ctypes.POINTER(ctypes.c_int),
            "size_t*": ctypes.POINTER(ctypes.c_size_t), "int": ctypes.c_int, "float": ctypes.c_float,
            "size_t": ctypes.c_size_t, "uint64_t": ctypes.c_uint64, "const char*": ctypes.c_char_p, "void": None}


def test_header_types_match_the_reference_externs():
    """Every reference extern keeps its argument count, order and C types
    (const-ness included) in include/nano_hip.h."""
    declared = header_signatures()
    for name, (ret, args) in REFERENCE_EXTERNS.items():
        assert name in declared, name
        assert declared[name] == (ret, args), f"{name}: header {declared[name]} != reference {(ret, args)}"


def test_wrapper_types_match_the_header():
    """nvr.SIGNATURES declares each function with the header's C types."""
    sigs = header_signatures()
    assert set(sigs) == header_functions() == set(nvr.SIGNATURES)
    for name, (ret, args) in sigs.items():
        restype, argtypes = nvr.SIGNATURES[name]
        assert restype == CTYPE_OF[ret], name
        assert argtypes == [CTYPE_OF[a] for a in args], name


def test_header_signature_parser_sees_a_swapped_argument():
    """The parser behind the two tests above tells int from float and a
    pointer from a value (a swapped pair is caught)."""
    sigs = header_signatures()
    ret, args = sigs["nv_rope_cache"]
    assert args == ["ctx", "void*", "int", "int", "float"]
    assert REFERENCE_EXTERNS["nv_rope_cache"][1] != ["ctx", "void*", "int", "float", "int"]
    assert sigs["nv_sampling_seed"] == ("uint64_t", ["uint64_t"] * 3)


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
