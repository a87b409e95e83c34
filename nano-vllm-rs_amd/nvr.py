"""Checked host wrapper over the nano-vllm-rs HIP library (libnano_hip.so).

This mirrors the reference's safe FFI layer, src/gpu.rs:214-1146: the same
`Gpu`, `Buffer` and `Graph` objects, the same method names and argument
meaning, and the same validation before every C call (positive i32 dimensions,
finite positive eps/theta, buffer extents and element alignment, context
identity, no output aliasing, no allocation/transfer/sync during capture).
Violations raise `ValueError`; a non-zero status from the library raises
`BackendError` carrying nv_last_error() and the status, as
`check()` at src/gpu.rs:214-221 turns them into an error.

The library is loaded from this directory. There is no fallback: if the
shared object is missing, every entry point raises.
"""
from __future__ import annotations

import atexit
import ctypes
import math
import os
import sys
from typing import Callable, Iterable, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnano_hip.so")

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); every symbol include/nano_hip.h declares.
SIGNATURES = {
    "nv_last_error": (ctypes.c_char_p, []),
    "nv_stream": (_i, [_vp, ctypes.POINTER(_vp)]),
    "nv_sm_count": (_i, [_vp, ctypes.POINTER(_i)]),
    "nv_create": (_i, [_i, ctypes.POINTER(_vp)]),
    "nv_destroy": (None, [_vp]),
    "nv_alloc": (_i, [_vp, _sz, ctypes.POINTER(_vp)]),
    "nv_free": (None, [_vp, _vp]),
    "nv_upload": (_i, [_vp, _vp, _vp, _sz]),
    "nv_download": (_i, [_vp, _vp, _vp, _sz]),
    "nv_sync": (_i, [_vp]),
    "nv_mem_info": (_i, [_vp, ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    "nv_capture_begin": (_i, [_vp]),
    "nv_capture_end": (_i, [_vp, ctypes.POINTER(_vp)]),
    "nv_capture_abort": (None, [_vp]),
    "nv_graph_replay": (_i, [_vp, _vp]),
    "nv_graph_destroy": (None, [_vp, _vp]),
    "nv_gemm": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "nv_embedding": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "nv_rms": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f]),
    "nv_add_rms": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _f]),
    "nv_qkv_rope": (_i, [_vp] * 9 + [_i] * 6 + [_f, _f]),
    "nv_rope_cache": (_i, [_vp, _vp, _i, _i, _f]),
    "nv_qkv_rope_cached": (_i, [_vp] * 9 + [_i] * 6 + [_f, _vp, _i]),
    "nv_attention": (_i, [_vp] * 8 + [_i] * 9),
    "nv_attention_qkv_rope": (_i, [_vp] * 11 + [_i] * 9 + [_f, _vp, _i]),
    "nv_silu": (_i, [_vp, _vp, _vp, _i, _i]),
    "nv_gather": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "nv_sample": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "nv_sample_parallel": (_i, [_vp] * 7 + [_i, _i]),
    "nv_sample_parallel_static": (_i, [_vp] * 5 + [_i, _i]),
    "nv_kv_write": (_i, [_vp] * 6 + [_i] * 5),
    "nv_sampling_seed": (ctypes.c_uint64, [ctypes.c_uint64] * 3),
}

_LIB = None
_EXITING = False


def _mark_exiting() -> None:
    # Runs before interpreter finalization: from here on, finalizers stop
    # calling into the library, because module teardown destroys objects in
    # an arbitrary order and the process exit releases device memory anyway.
    global _EXITING
    _EXITING = True


atexit.register(_mark_exiting)


def _native_ok() -> bool:
    return not _EXITING and not sys.is_finalizing()


class BackendError(RuntimeError):
    """A non-zero status returned by the HIP library."""

    def __init__(self, message: str, status: int):
        super().__init__(f"HIP backend: {message} (status {status})")
        self.status = status


def library(path: str | None = None) -> ctypes.CDLL:
    """Loads libnano_hip.so once and declares every C signature."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    target = path or LIB_PATH
    if not os.path.exists(target):
        raise FileNotFoundError(f"{target} is missing: build it with `make -C nano-vllm-rs_amd` "
                                "(or __graft_entry__.build()); there is no fallback path")
    lib = ctypes.CDLL(target)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def _check(code: int, lib: ctypes.CDLL | None = None) -> None:
    if code != 0:
        msg = (lib or library()).nv_last_error().decode(errors="replace")
        raise BackendError(msg, code)


def _dimension(value: int) -> int:
    if value <= 0:
        raise ValueError("tensor dimensions must be positive")
    if value > 0x7FFFFFFF:
        raise ValueError(f"dimension {value} exceeds i32")
    return int(value)


def _extent(dims: Sequence[int], element_size: int) -> int:
    n = element_size
    for d in dims:
        n *= _dimension(d)
    return n


def _positive(value: float, name: str) -> None:
    if not (math.isfinite(value) and value > 0.0):
        raise ValueError(f"{name} must be positive and finite")


def sampling_seed(base: int, request_id: int, generated: int) -> int:
    """src/runtime.rs:780-790, computed by the library's host function."""
    return int(library().nv_sampling_seed(base, request_id, generated))


class _Context:
    def __init__(self, handle: int, lib: ctypes.CDLL):
        self.handle = handle
        self.capturing = False
        self.captured: list[Buffer] = []
        self.lib = lib

    def outside_capture(self) -> None:
        if self.capturing:
            raise ValueError("allocation, transfer and synchronization are forbidden during graph capture")

    def __del__(self):
        if getattr(self, "handle", None) and _native_ok():
            self.lib.nv_destroy(self.handle)
        self.handle = None


class _Allocation:
    def __init__(self, context: _Context, ptr: int, nbytes: int):
        self.context = context
        self.ptr = ptr
        self.bytes = nbytes

    def __del__(self):
        if getattr(self, "ptr", None) and _native_ok() and self.context.handle:
            self.context.lib.nv_free(self.context.handle, self.ptr)
        self.ptr = None


class Buffer:
    """Owned device bytes; views share the allocation (src/gpu.rs:278-392)."""

    def __init__(self, allocation: _Allocation, offset: int, nbytes: int):
        self.allocation = allocation
        self.offset = offset
        self.bytes = nbytes

    @property
    def ptr(self) -> int:
        return self.allocation.ptr + self.offset

    def __len__(self) -> int:
        return self.bytes

    def _bounds(self, nbytes: int) -> None:
        if nbytes > self.bytes:
            raise ValueError(f"buffer needs {nbytes} bytes, allocation has {self.bytes}")

    def slice(self, offset: int, nbytes: int) -> "Buffer":
        if offset < 0 or nbytes < 0:
            raise ValueError("buffer view extent overflow")
        self._bounds(offset + nbytes)
        start = self.offset + offset
        if start > self.allocation.bytes or nbytes > self.allocation.bytes - start:
            raise ValueError("buffer view exceeds allocation")
        return Buffer(self.allocation, start, nbytes)

    def overlaps(self, other: "Buffer") -> bool:
        return (self.bytes > 0 and other.bytes > 0 and self.allocation is other.allocation
                and self.offset < other.offset + other.bytes and other.offset < self.offset + self.bytes)

    def upload(self, values: np.ndarray) -> None:
        ctx = self.allocation.context
        ctx.outside_capture()
        arr = np.ascontiguousarray(values)
        self._bounds(arr.nbytes)
        if arr.nbytes == 0:
            return
        _check(ctx.lib.nv_upload(ctx.handle, self.ptr, arr.ctypes.data, arr.nbytes))

    def download(self, dtype, count: int) -> np.ndarray:
        ctx = self.allocation.context
        ctx.outside_capture()
        out = np.empty(count, dtype=dtype)
        self._bounds(out.nbytes)
        if out.nbytes:
            _check(ctx.lib.nv_download(ctx.handle, self.ptr, out.ctypes.data, out.nbytes))
        return out

    def download_bytes(self, count: int | None = None) -> bytes:
        return self.download(np.uint8, self.bytes if count is None else count).tobytes()


class Graph:
    """Executable graph; keeps every captured allocation alive (src/gpu.rs:1128-1146)."""

    def __init__(self, context: _Context, handle: int, buffers: list[Buffer]):
        self.context = context
        self.handle = handle
        self._buffers = buffers

    def replay(self) -> None:
        self.context.outside_capture()
        _check(self.context.lib.nv_graph_replay(self.context.handle, self.handle))

    def __del__(self):
        if getattr(self, "handle", None) and _native_ok() and self.context.handle:
            self.context.lib.nv_graph_destroy(self.context.handle, self.handle)
        self.handle = None


class Gpu:
    """One device, one stream, one hipBLAS handle (src/gpu.rs:394-1112)."""

    def __init__(self, device: int = 0, library_path: str | None = None):
        """library_path selects another build of libnano_hip.so (default: this directory's)."""
        if device < 0:
            raise ValueError("device index must be nonnegative")
        lib = library(library_path)
        handle = _vp()
        code = lib.nv_create(device, ctypes.byref(handle))
        if code != 0:
            raise BackendError(lib.nv_last_error().decode(errors="replace"), code)
        if not handle.value:
            raise BackendError("library returned a null context", -1)
        self.context = _Context(handle.value, lib)
        self.lib = lib

    @property
    def handle(self) -> int:
        return self.context.handle

    # ------------------------------------------------------------ runtime --
    def alloc(self, nbytes: int) -> Buffer:
        self.context.outside_capture()
        if nbytes <= 0:
            raise ValueError(f"invalid allocation size {nbytes}")
        ptr = _vp()
        _check(self.lib.nv_alloc(self.handle, nbytes, ctypes.byref(ptr)))
        if not ptr.value:
            raise BackendError("library returned a null allocation", -1)
        return Buffer(_Allocation(self.context, ptr.value, nbytes), 0, nbytes)

    def upload_array(self, values: np.ndarray) -> Buffer:
        arr = np.ascontiguousarray(values)
        buf = self.alloc(max(arr.nbytes, 1))
        buf.upload(arr)
        return buf.slice(0, arr.nbytes) if arr.nbytes else buf

    def sync(self) -> None:
        self.context.outside_capture()
        _check(self.lib.nv_sync(self.handle))

    def mem_info(self) -> tuple[int, int]:
        self.context.outside_capture()
        free, total = _sz(), _sz()
        _check(self.lib.nv_mem_info(self.handle, ctypes.byref(free), ctypes.byref(total)))
        return free.value, total.value

    def sm_count(self) -> int:
        n = _i()
        _check(self.lib.nv_sm_count(self.handle, ctypes.byref(n)))
        if n.value <= 0:
            raise BackendError("invalid compute-unit count", -1)
        return n.value

    def stream(self) -> int:
        s = _vp()
        _check(self.lib.nv_stream(self.handle, ctypes.byref(s)))
        return s.value or 0

    def tensor(self, buffer: Buffer, dims: Sequence[int], element_size: int) -> None:
        if buffer.allocation.context is not self.context:
            raise ValueError("buffer belongs to a different context")
        buffer._bounds(_extent(dims, element_size))
        if buffer.offset % element_size != 0:
            raise ValueError("tensor view is not aligned to its element size")
        if self.context.capturing and not any(b.allocation is buffer.allocation for b in self.context.captured):
            self.context.captured.append(buffer)

    @staticmethod
    def distinct(output: Buffer, inputs: Iterable[Buffer]) -> None:
        if any(output.overlaps(i) for i in inputs):
            raise ValueError("kernel output aliases an input or another output")

    def capture(self, forward: Callable[[], None]) -> Graph:
        """Captures only device operations; captured buffers live with the Graph."""
        self.context.outside_capture()
        _check(self.lib.nv_capture_begin(self.handle))
        self.context.capturing = True
        try:
            forward()
        except BaseException:
            self.lib.nv_capture_abort(self.handle)
            self.context.capturing = False
            self.context.captured = []
            raise
        graph = _vp()
        code = self.lib.nv_capture_end(self.handle, ctypes.byref(graph))
        self.context.capturing = False
        buffers, self.context.captured = self.context.captured, []
        _check(code)
        if not graph.value:
            raise BackendError("null graph", -1)
        return Graph(self.context, graph.value, buffers)

    # -------------------------------------------------------------- GEMM ---
    def gemm(self, x: Buffer, w: Buffer, y: Buffer, m: int, n: int, k: int) -> None:
        self.tensor(x, [m, k], 2)
        self.tensor(w, [n, k], 2)
        self.tensor(y, [m, n], 2)
        self.distinct(y, [x, w])
        _check(self.lib.nv_gemm(self.handle, x.ptr, w.ptr, y.ptr, _dimension(m), _dimension(n), _dimension(k)))

    # ----------------------------------------------------------- kernels ---
    def embedding(self, tokens: Buffer, weight: Buffer, out: Buffer, rows: int, hidden: int, vocab: int) -> None:
        self.tensor(tokens, [rows], 4)
        self.tensor(weight, [vocab, hidden], 2)
        self.tensor(out, [rows, hidden], 2)
        self.distinct(out, [tokens, weight])
        _check(self.lib.nv_embedding(self.handle, tokens.ptr, weight.ptr, out.ptr, _dimension(rows),
                                     _dimension(hidden), _dimension(vocab)))

    def rms_norm(self, x: Buffer, weight: Buffer, out: Buffer, rows: int, hidden: int, eps: float) -> None:
        _positive(eps, "RMS epsilon")
        self.tensor(x, [rows, hidden], 2)
        self.tensor(weight, [hidden], 2)
        self.tensor(out, [rows, hidden], 2)
        self.distinct(out, [x, weight])
        _check(self.lib.nv_rms(self.handle, x.ptr, weight.ptr, out.ptr, _dimension(rows), _dimension(hidden), eps))

    def add_rms_norm(self, x: Buffer, residual: Buffer, weight: Buffer, out: Buffer, rows: int, hidden: int,
                     eps: float) -> None:
        """residual <- bf16(x + residual); out <- RMSNorm(f32(x) + f32(residual))."""
        _positive(eps, "RMS epsilon")
        self.tensor(x, [rows, hidden], 2)
        self.tensor(residual, [rows, hidden], 2)
        self.tensor(weight, [hidden], 2)
        self.tensor(out, [rows, hidden], 2)
        self.distinct(out, [x, residual, weight])
        self.distinct(residual, [x, weight])
        _check(self.lib.nv_add_rms(self.handle, x.ptr, residual.ptr, weight.ptr, out.ptr, _dimension(rows),
                                   _dimension(hidden), eps))

    @staticmethod
    def _heads(qheads: int, kvheads: int, head_dim: int) -> None:
        _dimension(qheads)
        _dimension(kvheads)
        _dimension(head_dim)
        if qheads % kvheads != 0:
            raise ValueError("query heads must be a multiple of KV heads")
        if head_dim % 2 != 0 or head_dim > 256:
            raise ValueError("head dimension must be even and at most 256")
        if qheads + kvheads > 65535:
            raise ValueError("too many heads for one launch")

    def _check_qkv_rope(self, qkv, qweight, kweight, positions, slots, qout, kcache, vcache, rows, qheads, kvheads,
                        head_dim, block_size, num_blocks, eps) -> None:
        self._heads(qheads, kvheads, head_dim)
        _positive(eps, "RMS epsilon")
        self.tensor(qkv, [rows, qheads + 2 * kvheads, head_dim], 2)
        for w in (qweight, kweight):
            self.tensor(w, [head_dim], 2)
        for meta in (positions, slots):
            self.tensor(meta, [rows], 4)
        self.tensor(qout, [rows, qheads, head_dim], 2)
        for cache in (kcache, vcache):
            self.tensor(cache, [num_blocks, block_size, kvheads, head_dim], 2)
        inputs = [qkv, qweight, kweight, positions, slots]
        for out in (qout, kcache, vcache):
            self.distinct(out, inputs)
        self.distinct(qout, [kcache, vcache])
        self.distinct(kcache, [vcache])

    def qkv_rope(self, qkv, qweight, kweight, positions, slots, qout, kcache, vcache, rows, qheads, kvheads,
                 head_dim, block_size, num_blocks, eps, theta) -> None:
        _positive(theta, "RoPE theta")
        self._check_qkv_rope(qkv, qweight, kweight, positions, slots, qout, kcache, vcache, rows, qheads, kvheads,
                             head_dim, block_size, num_blocks, eps)
        _check(self.lib.nv_qkv_rope(self.handle, qkv.ptr, qweight.ptr, kweight.ptr, positions.ptr, slots.ptr,
                                    qout.ptr, kcache.ptr, vcache.ptr, _dimension(rows), _dimension(qheads),
                                    _dimension(kvheads), _dimension(head_dim), _dimension(block_size),
                                    _dimension(num_blocks), eps, theta))

    def rope_cache(self, cache: Buffer, max_positions: int, head_dim: int, theta: float) -> None:
        """fp32 [positions, cos(head_dim/2) | sin(head_dim/2)], built once at load time."""
        self._heads(1, 1, head_dim)
        _positive(theta, "RoPE theta")
        self.tensor(cache, [max_positions, head_dim], 4)
        _check(self.lib.nv_rope_cache(self.handle, cache.ptr, _dimension(max_positions), _dimension(head_dim),
                                      theta))

    def qkv_rope_cached(self, qkv, qweight, kweight, positions, slots, qout, kcache, vcache, rows, qheads, kvheads,
                        head_dim, block_size, num_blocks, eps, rope_cache, max_positions) -> None:
        self._check_qkv_rope(qkv, qweight, kweight, positions, slots, qout, kcache, vcache, rows, qheads, kvheads,
                             head_dim, block_size, num_blocks, eps)
        self.tensor(rope_cache, [max_positions, head_dim], 4)
        for output in (qout, kcache, vcache):
            self.distinct(output, [rope_cache])
        _check(self.lib.nv_qkv_rope_cached(self.handle, qkv.ptr, qweight.ptr, kweight.ptr, positions.ptr,
                                           slots.ptr, qout.ptr, kcache.ptr, vcache.ptr, _dimension(rows),
                                           _dimension(qheads), _dimension(kvheads), _dimension(head_dim),
                                           _dimension(block_size), _dimension(num_blocks), eps, rope_cache.ptr,
                                           _dimension(max_positions)))

    def paged_attention(self, q: Buffer, kcache: Buffer, vcache: Buffer, positions: Buffer, seq_indices: Buffer,
                        block_tables: Buffer, out: Buffer, rows: int, qheads: int, kvheads: int, head_dim: int,
                        block_size: int, num_blocks: int, table_stride: int, batch_size: int,
                        max_context: int) -> None:
        """Causal paged GQA over flattened ragged prefill and decode rows
        (src/gpu.rs:826-887). KV layout [blocks, block_size, kvheads, head_dim];
        each row attends to positions[row] + 1 keys of sequence seq_indices[row]."""
        self._heads(qheads, kvheads, head_dim)
        if not 0 < max_context <= 4096:
            raise ValueError("paged attention supports at most 4096 context tokens")
        self.tensor(q, [rows, qheads, head_dim], 2)
        self.tensor(out, [rows, qheads, head_dim], 2)
        for cache in (kcache, vcache):
            self.tensor(cache, [num_blocks, block_size, kvheads, head_dim], 2)
        for meta in (positions, seq_indices):
            self.tensor(meta, [rows], 4)
        self.tensor(block_tables, [batch_size, table_stride], 4)
        self.distinct(out, [q, kcache, vcache, positions, seq_indices, block_tables])
        _check(self.lib.nv_attention(self.handle, q.ptr, kcache.ptr, vcache.ptr, positions.ptr, seq_indices.ptr,
                                     block_tables.ptr, out.ptr, _dimension(rows), _dimension(qheads),
                                     _dimension(kvheads), _dimension(head_dim), _dimension(block_size),
                                     _dimension(num_blocks), _dimension(table_stride), _dimension(batch_size),
                                     _dimension(max_context)))

    def attention_qkv_rope(self, qkv: Buffer, qweight: Buffer, kweight: Buffer, positions: Buffer, slots: Buffer,
                           kcache: Buffer, vcache: Buffer, seq_indices: Buffer, block_tables: Buffer, out: Buffer,
                           rows: int, qheads: int, kvheads: int, head_dim: int, block_size: int, num_blocks: int,
                           table_stride: int, batch_size: int, max_context: int, eps: float, rope_cache: Buffer,
                           max_positions: int) -> None:
        """qkv_rope_cached followed by paged_attention in one launch (head dim
        128), for decode batches: no row may read a KV slot that another row
        writes. The rotated q is not written to memory."""
        if head_dim != 128:
            raise ValueError("fused attention needs head_dim 128")
        if not 0 < max_context <= 4096:
            raise ValueError("paged attention supports at most 4096 context tokens")
        self.tensor(out, [rows, qheads, head_dim], 2)
        self.tensor(seq_indices, [rows], 4)
        self.tensor(block_tables, [batch_size, table_stride], 4)
        self.tensor(rope_cache, [max_positions, head_dim], 4)
        self._check_qkv_rope(qkv, qweight, kweight, positions, slots, out, kcache, vcache, rows, qheads, kvheads,
                             head_dim, block_size, num_blocks, eps)
        self.distinct(out, [qkv, kcache, vcache, positions, seq_indices, block_tables, rope_cache])
        for cache in (kcache, vcache):
            self.distinct(cache, [rope_cache, seq_indices, block_tables])
        _check(self.lib.nv_attention_qkv_rope(self.handle, qkv.ptr, qweight.ptr, kweight.ptr, positions.ptr,
                                              slots.ptr, kcache.ptr, vcache.ptr, seq_indices.ptr, block_tables.ptr,
                                              out.ptr, _dimension(rows), _dimension(qheads), _dimension(kvheads),
                                              _dimension(head_dim), _dimension(block_size), _dimension(num_blocks),
                                              _dimension(table_stride), _dimension(batch_size),
                                              _dimension(max_context), eps, rope_cache.ptr,
                                              _dimension(max_positions)))

    def kv_write(self, k: Buffer, v: Buffer, slots: Buffer, kcache: Buffer, vcache: Buffer, rows: int,
                 kvheads: int, head_dim: int, block_size: int, num_blocks: int) -> None:
        """Standalone paged KV-cache slot write (no counterpart method in src/gpu.rs)."""
        for t in (k, v):
            self.tensor(t, [rows, kvheads, head_dim], 2)
        self.tensor(slots, [rows], 4)
        for cache in (kcache, vcache):
            self.tensor(cache, [num_blocks, block_size, kvheads, head_dim], 2)
        for out in (kcache, vcache):
            self.distinct(out, [k, v, slots])
        self.distinct(kcache, [vcache])
        _check(self.lib.nv_kv_write(self.handle, k.ptr, v.ptr, slots.ptr, kcache.ptr, vcache.ptr, _dimension(rows),
                                    _dimension(kvheads), _dimension(head_dim), _dimension(block_size),
                                    _dimension(num_blocks)))

    def silu_mul(self, gateup: Buffer, out: Buffer, rows: int, intermediate: int) -> None:
        self.tensor(gateup, [rows, 2, intermediate], 2)
        self.tensor(out, [rows, intermediate], 2)
        if intermediate > 0x7FFFFFFF // 2:
            raise ValueError("intermediate size too large")
        self.distinct(out, [gateup])
        _check(self.lib.nv_silu(self.handle, gateup.ptr, out.ptr, _dimension(rows), _dimension(intermediate)))

    def gather(self, x: Buffer, indices: Buffer, out: Buffer, rows: int, hidden: int, input_rows: int) -> None:
        self.tensor(x, [input_rows, hidden], 2)
        self.tensor(indices, [rows], 4)
        self.tensor(out, [rows, hidden], 2)
        self.distinct(out, [x, indices])
        _check(self.lib.nv_gather(self.handle, x.ptr, indices.ptr, out.ptr, _dimension(rows), _dimension(hidden),
                                  _dimension(input_rows)))

    def sample(self, logits: Buffer, temperatures: Buffer, seeds: Buffer, out: Buffer, batch: int,
               vocab: int) -> None:
        """bf16 logits; f32 temperatures (<= 0 greedy); u64 seeds; i32 output."""
        self.tensor(logits, [batch, vocab], 2)
        self.tensor(temperatures, [batch], 4)
        self.tensor(seeds, [batch], 8)
        self.tensor(out, [batch], 4)
        self.distinct(out, [logits, temperatures, seeds])
        _check(self.lib.nv_sample(self.handle, logits.ptr, temperatures.ptr, seeds.ptr, out.ptr, _dimension(batch),
                                  _dimension(vocab)))

    def sample_parallel(self, logits: Buffer, temperatures: Buffer, seeds: Buffer, out: Buffer,
                        partial_scores: Buffer, partial_ids: Buffer, batch: int, vocab: int) -> None:
        """Two-stage vocabulary reduction; scratch holds batch x ceil(vocab/2048) entries."""
        self.tensor(logits, [batch, vocab], 2)
        self.tensor(temperatures, [batch], 4)
        self.tensor(seeds, [batch], 8)
        self.tensor(out, [batch], 4)
        parts = -(-vocab // 2048)
        self.tensor(partial_scores, [batch, parts], 4)
        self.tensor(partial_ids, [batch, parts], 4)
        for output in (out, partial_scores, partial_ids):
            self.distinct(output, [logits, temperatures, seeds])
        self.distinct(out, [partial_scores, partial_ids])
        self.distinct(partial_scores, [partial_ids])
        _check(self.lib.nv_sample_parallel(self.handle, logits.ptr, temperatures.ptr, seeds.ptr, out.ptr,
                                           partial_scores.ptr, partial_ids.ptr, _dimension(batch),
                                           _dimension(vocab)))


    STATIC_PARTIALS = 1 << 17

    def sample_parallel_static(self, logits: Buffer, temperatures: Buffer, seeds: Buffer, out: Buffer, batch: int,
                               vocab: int) -> None:
        """sample_parallel with the library's static partials instead of caller
        scratch (no allocation): batch * ceil(vocab / 2048) <= 131072."""
        self.tensor(logits, [batch, vocab], 2)
        self.tensor(temperatures, [batch], 4)
        self.tensor(seeds, [batch], 8)
        self.tensor(out, [batch], 4)
        self.distinct(out, [logits, temperatures, seeds])
        _check(self.lib.nv_sample_parallel_static(self.handle, logits.ptr, temperatures.ptr, seeds.ptr, out.ptr,
                                                  _dimension(batch), _dimension(vocab)))


def bf16_bits(values) -> np.ndarray:
    """fp32 values -> bf16 bit patterns, round to nearest even (NaN stays NaN)."""
    f = np.ascontiguousarray(values, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    quiet = ((u >> 16) | 0x40) & 0xFFFF
    return np.where(nan, quiet, rounded).astype(np.uint16)


def bf16_values(bits) -> np.ndarray:
    """bf16 bit patterns -> fp32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
