"""Python host API over libnano_hip.so (ctypes), used by the tests and bench.py.

Class and method names follow the Rust host of nano-vllm-rs (src/gpu.rs: Gpu,
Buffer, Graph, one method per kernel, with the same argument order). The
argument contract is this library's own, the same one the C++ host API
(host/gpu.hpp) enforces:

* Tensor arguments. Every kernel method lists its tensor arguments as
  (name, buffer, element width, shape, written?) and ``Gpu._admit`` checks
  them together: every dimension in [1, 2^31 - 1]; the view holds the byte
  count; the view starts at a multiple of the element width; the buffer was
  allocated by this Gpu; the bytes a written argument covers share nothing
  with the bytes of any other argument.
* Scalars. eps and theta finite and positive; q heads a multiple of KV heads,
  head_dim even and at most 256, q + KV heads at most 65535.
* Capture. The library itself refuses allocation, transfers and
  synchronisation while its stream is captured (status -2). A capture here
  only records the allocations its kernels use; the Graph keeps them alive.

A broken rule raises ``ArgumentError`` (a ValueError) whose ``fault`` names the
rule: "dimension", "extent", "alignment", "foreign", "overlap" or "value". A
non-zero library status raises ``BackendError`` with nv_last_error().

The library is loaded from this directory. There is no fallback: if the shared
object is missing, every entry point raises.
"""
from __future__ import annotations

import atexit
import ctypes
import math
import os
import sys
from typing import Callable, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnano_hip.so")
INT_MAX = 0x7FFFFFFF

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
    "nv_add_rms_gather": (_i, [_vp] * 6 + [_i, _i, _i, _f]),
    "nv_rms_gemm": (_i, [_vp] * 8 + [_i, _i, _i, _f]),
    "nv_gemm_rows": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "nv_rms_gemm_silu": (_i, [_vp] * 9 + [_i, _i, _i, _f]),
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
_SHUTDOWN = False


def _shutting_down() -> None:
    # Runs before interpreter finalization: from then on, finalizers make no
    # library calls (module teardown order is arbitrary, and the process exit
    # releases device memory anyway).
    global _SHUTDOWN
    _SHUTDOWN = True


atexit.register(_shutting_down)


def _live() -> bool:
    return not _SHUTDOWN and not sys.is_finalizing()


class BackendError(RuntimeError):
    """A non-zero status returned by the HIP library."""

    def __init__(self, message: str, status: int):
        super().__init__(f"libnano_hip status {status}: {message}")
        self.status = status


class ArgumentError(ValueError):
    """An argument broke the host contract; ``fault`` names the rule."""

    def __init__(self, fault: str, message: str):
        super().__init__(f"{fault}: {message}")
        self.fault = fault


def library(path: str | None = None) -> ctypes.CDLL:
    """Loads libnano_hip.so (once for the default path) and declares every C signature."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    target = path or LIB_PATH
    if not os.path.exists(target):
        raise FileNotFoundError(f"{target} is missing: build it with `make -C nano-vllm-rs_amd` "
                                "(or __graft_entry__.build()); there is no fallback path")
    lib = ctypes.CDLL(target)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = restype, argtypes
    if path is None:
        _LIB = lib
    return lib


def tile_gate_up_rows(gate_up: np.ndarray, intermediate: int) -> np.ndarray:
    """The [2 * intermediate, k] gate_up weight (gate rows, then up rows) in the
    tile row order nv_rms_gemm_silu reads: tile t = gate rows 8t..8t+7, then up
    rows 8t..8t+7."""
    w = np.asarray(gate_up).reshape(2, intermediate // 8, 8, -1)
    return np.ascontiguousarray(w.transpose(1, 0, 2, 3).reshape(2 * intermediate, -1))


def check_status(status: int, lib: ctypes.CDLL | None = None) -> None:
    """Raises BackendError for a non-zero library status."""
    if status != 0:
        raise BackendError((lib or library()).nv_last_error().decode(errors="replace"), status)


def as_dim(value: int) -> int:
    """value as a kernel dimension in [1, 2^31 - 1]."""
    if not 1 <= value <= INT_MAX:
        raise ArgumentError("dimension", f"{value} outside [1, 2^31 - 1]")
    return int(value)


def byte_count(dims: Sequence[int], width: int) -> int:
    """width * prod(dims), every dimension checked by as_dim."""
    n = width
    for d in dims:
        n *= as_dim(d)
    return n


def require_positive(value: float, what: str) -> None:
    if not (math.isfinite(value) and value > 0.0):
        raise ArgumentError("value", f"{what} = {value} is not a positive finite number")


def require_head_layout(qheads: int, kvheads: int, head_dim: int) -> None:
    as_dim(qheads), as_dim(kvheads), as_dim(head_dim)
    if qheads % kvheads:
        raise ArgumentError("value", f"{qheads} query heads do not group evenly over {kvheads} KV heads")
    if head_dim % 2 or head_dim > 256:
        raise ArgumentError("value", f"head_dim {head_dim} is not an even number up to 256")
    if qheads + kvheads > 65535:
        raise ArgumentError("value", f"{qheads + kvheads} q + KV heads exceed one launch's 65535 grid rows")


def sampling_seed(base: int, request_id: int, generated: int) -> int:
    """src/runtime.rs:780-790, computed by the library's host function."""
    return int(library().nv_sampling_seed(base, request_id, generated))


# --------------------------------------------------------------- objects ---
class _Device:
    """A library context; while a capture runs, the allocations its kernels use."""

    def __init__(self, lib: ctypes.CDLL, ctx: int):
        self.lib, self.ctx = lib, ctx
        self.recording: dict[int, "_Memory"] | None = None

    def __del__(self):
        if getattr(self, "ctx", None) and _live():
            self.lib.nv_destroy(self.ctx)  # waits for the stream first
        self.ctx = None


class _Memory:
    """One device allocation; freed when the last view goes."""

    def __init__(self, device: _Device, address: int, size: int):
        self.device, self.address, self.size = device, address, size

    def __del__(self):
        if getattr(self, "address", None) and _live() and self.device.ctx:
            self.device.lib.nv_free(self.device.ctx, self.address)
        self.address = None


class Buffer:
    """A view (offset, length) of a device allocation; views keep the allocation alive."""

    def __init__(self, memory: _Memory, offset: int, length: int):
        self._memory, self._offset, self._length = memory, offset, length

    @property
    def ptr(self) -> int:
        return self._memory.address + self._offset

    @property
    def bytes(self) -> int:
        return self._length

    def __len__(self) -> int:
        return self._length

    def slice(self, offset: int, nbytes: int) -> "Buffer":
        """The sub-view [offset, offset + nbytes) of this view."""
        if offset < 0 or nbytes < 0 or offset > self._length or nbytes > self._length - offset:
            raise ArgumentError("extent", f"sub-view [{offset}, +{nbytes}) of a {self._length}-byte view")
        return Buffer(self._memory, self._offset + offset, nbytes)

    def overlaps(self, other: "Buffer") -> bool:
        if self._memory is not other._memory or not self._length or not other._length:
            return False
        return max(self._offset, other._offset) < min(self._offset + self._length, other._offset + other._length)

    def upload(self, values: np.ndarray) -> None:
        """Synchronous host -> device copy of `values` to the start of the view."""
        arr = np.ascontiguousarray(values)
        if arr.nbytes > self._length:
            raise ArgumentError("extent", f"upload of {arr.nbytes} bytes into a {self._length}-byte view")
        if arr.nbytes:
            d = self._memory.device
            check_status(d.lib.nv_upload(d.ctx, self.ptr, arr.ctypes.data, arr.nbytes), d.lib)

    def download(self, dtype, count: int) -> np.ndarray:
        """Synchronous device -> host copy of `count` elements from the start of the view."""
        out = np.empty(count, dtype=dtype)
        if out.nbytes > self._length:
            raise ArgumentError("extent", f"download of {out.nbytes} bytes from a {self._length}-byte view")
        if out.nbytes:
            d = self._memory.device
            check_status(d.lib.nv_download(d.ctx, self.ptr, out.ctypes.data, out.nbytes), d.lib)
        return out

    def download_bytes(self, count: int | None = None) -> bytes:
        return self.download(np.uint8, self._length if count is None else count).tobytes()


class Graph:
    """An executable graph; holds the allocations its kernels use."""

    def __init__(self, device: _Device, exec_handle: int, held: list[_Memory]):
        self._device, self._exec, self._held = device, exec_handle, held

    def replay(self) -> None:
        check_status(self._device.lib.nv_graph_replay(self._device.ctx, self._exec), self._device.lib)

    def __del__(self):
        if getattr(self, "_exec", None) and _live() and self._device.ctx:
            self._device.lib.nv_graph_destroy(self._device.ctx, self._exec)
        self._exec = None


def _r(name: str, buf: Buffer, width: int, *dims: int):
    return name, buf, width, dims, False


def _w(name: str, buf: Buffer, width: int, *dims: int):
    return name, buf, width, dims, True


class Gpu:
    """One device, one stream, one hipBLAS handle."""

    def __init__(self, device: int = 0, library_path: str | None = None):
        """library_path selects another build of libnano_hip.so (default: this directory's)."""
        if device < 0:
            raise ArgumentError("value", f"device index {device} is negative")
        lib = library(library_path)
        ctx = _vp()
        check_status(lib.nv_create(device, ctypes.byref(ctx)), lib)
        self._device = _Device(lib, ctx.value)
        self.lib = lib

    @property
    def handle(self) -> int:
        return self._device.ctx

    # ------------------------------------------------------------ runtime --
    def alloc(self, nbytes: int) -> Buffer:
        """Zero-filled device memory."""
        if nbytes <= 0:
            raise ArgumentError("extent", f"allocation of {nbytes} bytes")
        address = _vp()
        check_status(self.lib.nv_alloc(self.handle, nbytes, ctypes.byref(address)), self.lib)
        return Buffer(_Memory(self._device, address.value, nbytes), 0, nbytes)

    def upload_array(self, values: np.ndarray) -> Buffer:
        arr = np.ascontiguousarray(values)
        buf = self.alloc(max(arr.nbytes, 1))
        buf.upload(arr)
        return buf.slice(0, arr.nbytes) if arr.nbytes else buf

    def sync(self) -> None:
        check_status(self.lib.nv_sync(self.handle), self.lib)

    def mem_info(self) -> tuple[int, int]:
        free, total = _sz(), _sz()
        check_status(self.lib.nv_mem_info(self.handle, ctypes.byref(free), ctypes.byref(total)), self.lib)
        return free.value, total.value

    def sm_count(self) -> int:
        n = _i()
        check_status(self.lib.nv_sm_count(self.handle, ctypes.byref(n)), self.lib)
        return as_dim(n.value)

    def stream(self) -> int:
        s = _vp()
        check_status(self.lib.nv_stream(self.handle, ctypes.byref(s)), self.lib)
        return s.value or 0

    def capture(self, forward: Callable[[], None]) -> Graph:
        """Records the device work `forward` enqueues into a graph."""
        if self._device.recording is not None:
            raise ArgumentError("value", "a capture is already running on this Gpu")
        check_status(self.lib.nv_capture_begin(self.handle), self.lib)
        self._device.recording = {}
        try:
            forward()
        except BaseException:
            self.lib.nv_capture_abort(self.handle)
            self._device.recording = None
            raise
        exec_handle = _vp()
        status = self.lib.nv_capture_end(self.handle, ctypes.byref(exec_handle))  # over whatever the status
        held, self._device.recording = list(self._device.recording.values()), None
        check_status(status, self.lib)
        return Graph(self._device, exec_handle.value, held)

    def _admit(self, op: str, args) -> None:
        """Checks the tensor arguments of kernel `op` (the module's contract)."""
        spans = []
        for name, buf, width, dims, _ in args:
            who = f"{op}: argument '{name}'"
            if buf._memory.device is not self._device:
                raise ArgumentError("foreign", f"{who} was not allocated by this Gpu")
            need = byte_count(dims, width)
            if need > buf._length:
                raise ArgumentError("extent", f"{who} needs {need} bytes; its view holds {buf._length}")
            if buf._offset % width:
                raise ArgumentError("alignment", f"{who} starts at byte {buf._offset}, not a multiple of {width}")
            spans.append((buf._memory, buf._offset, buf._offset + need))
        for i, (name, _, _, _, written) in enumerate(args):
            if not written:
                continue
            mem, lo, hi = spans[i]
            for j, (other, olo, ohi) in enumerate(spans):
                if j != i and other is mem and max(lo, olo) < min(hi, ohi):
                    raise ArgumentError("overlap", f"{op}: written argument '{name}' shares bytes with "
                                                   f"argument '{args[j][0]}'")
        if self._device.recording is not None:
            for _, buf, _, _, _ in args:
                self._device.recording.setdefault(id(buf._memory), buf._memory)

    def _call(self, status: int) -> None:
        check_status(status, self.lib)

    # -------------------------------------------------------------- GEMM ---
    def gemm(self, x: Buffer, w: Buffer, y: Buffer, m: int, n: int, k: int) -> None:
        """Y[m, n] = X[m, k] W[n, k]^T, bf16 in/out, fp32 accumulation."""
        self._admit("gemm", [_r("x", x, 2, m, k), _r("w", w, 2, n, k), _w("y", y, 2, m, n)])
        self._call(self.lib.nv_gemm(self.handle, x.ptr, w.ptr, y.ptr, m, n, k))

    # ----------------------------------------------------------- kernels ---
    def embedding(self, tokens: Buffer, weight: Buffer, out: Buffer, rows: int, hidden: int, vocab: int) -> None:
        self._admit("embedding", [_r("tokens", tokens, 4, rows), _r("weight", weight, 2, vocab, hidden),
                                  _w("out", out, 2, rows, hidden)])
        self._call(self.lib.nv_embedding(self.handle, tokens.ptr, weight.ptr, out.ptr, rows, hidden, vocab))

    def rms_norm(self, x: Buffer, weight: Buffer, out: Buffer, rows: int, hidden: int, eps: float) -> None:
        require_positive(eps, "rms_norm eps")
        self._admit("rms_norm", [_r("x", x, 2, rows, hidden), _r("weight", weight, 2, hidden),
                                 _w("out", out, 2, rows, hidden)])
        self._call(self.lib.nv_rms(self.handle, x.ptr, weight.ptr, out.ptr, rows, hidden, eps))

    def add_rms_norm(self, x: Buffer, residual: Buffer, weight: Buffer, out: Buffer, rows: int, hidden: int,
                     eps: float) -> None:
        """residual <- bf16(x + residual); out <- RMSNorm(f32(x) + f32(residual)) * weight."""
        require_positive(eps, "add_rms_norm eps")
        self._admit("add_rms_norm", [_r("x", x, 2, rows, hidden), _w("residual", residual, 2, rows, hidden),
                                     _r("weight", weight, 2, hidden), _w("out", out, 2, rows, hidden)])
        self._call(self.lib.nv_add_rms(self.handle, x.ptr, residual.ptr, weight.ptr, out.ptr, rows, hidden, eps))

    RMS_GEMM_MAX_ROWS = 32

    def gemm_rows(self, x: Buffer, w: Buffer, y: Buffer, m: int, n: int, k: int) -> None:
        """Y[m, n] = X[m, k] W[n, k]^T for 1 <= m <= 32 rows on this library's MFMA kernel."""
        if not 1 <= m <= self.RMS_GEMM_MAX_ROWS or n % 16 or k not in (1024, 2048, 3072, 4096):
            raise ArgumentError("value", f"gemm_rows: unsupported shape m {m}, n {n}, k {k}")
        self._admit("gemm_rows", [_r("x", x, 2, m, k), _r("w", w, 2, n, k), _w("y", y, 2, m, n)])
        self._call(self.lib.nv_gemm_rows(self.handle, x.ptr, w.ptr, y.ptr, m, n, k))

    def rms_gemm(self, x: Buffer, residual: Buffer | None, residual_out: Buffer | None, norm_weight: Buffer,
                 w: Buffer, y: Buffer, normed: Buffer | None, m: int, n: int, k: int, eps: float) -> None:
        """y = bf16(RMSNorm(x [+ residual]) W^T) for 1 <= m <= 32 rows; residual_out <- bf16(x + residual)
        (another buffer) and normed <- the normalised rows when given."""
        require_positive(eps, "rms_gemm eps")
        if residual is None and residual_out is not None:
            raise ArgumentError("value", "rms_gemm: residual_out needs a residual to add")
        if not 1 <= m <= self.RMS_GEMM_MAX_ROWS or n % 16 or k not in (512, 1024, 2048):
            raise ArgumentError("value", f"rms_gemm: unsupported shape m {m}, n {n}, k {k}")
        args = [_r("x", x, 2, m, k), _r("norm_weight", norm_weight, 2, k), _r("w", w, 2, n, k), _w("y", y, 2, m, n)]
        if residual is not None:
            args.append(_r("residual", residual, 2, m, k))
        if residual_out is not None:
            args.append(_w("residual_out", residual_out, 2, m, k))
        if normed is not None:
            args.append(_w("normed", normed, 2, m, k))
        self._admit("rms_gemm", args)
        ptr = lambda b: None if b is None else b.ptr  # noqa: E731
        self._call(self.lib.nv_rms_gemm(self.handle, x.ptr, ptr(residual), ptr(residual_out), norm_weight.ptr, w.ptr,
                                        y.ptr, ptr(normed), m, n, k, eps))

    def rms_gemm_silu(self, x: Buffer, residual: Buffer | None, residual_out: Buffer | None, norm_weight: Buffer,
                      w_tiled: Buffer, gate_up: Buffer | None, act: Buffer, normed: Buffer | None, m: int,
                      intermediate: int, k: int, eps: float) -> None:
        """rms_gemm with SiLU·up as the epilogue: w_tiled is the gate_up weight in tile row order
        (tile_gate_up_rows), act [m, intermediate] receives silu(gate) * up, gate_up (optional) the GEMM
        output in [gate | up] order."""
        require_positive(eps, "rms_gemm_silu eps")
        if residual is None and residual_out is not None:
            raise ArgumentError("value", "rms_gemm_silu: residual_out needs a residual to add")
        if not 1 <= m <= self.RMS_GEMM_MAX_ROWS or intermediate % 8 or k not in (512, 1024, 2048):
            raise ArgumentError("value", f"rms_gemm_silu: unsupported shape m {m}, intermediate {intermediate}, k {k}")
        args = [_r("x", x, 2, m, k), _r("norm_weight", norm_weight, 2, k),
                _r("w_tiled", w_tiled, 2, 2 * intermediate, k), _w("act", act, 2, m, intermediate)]
        for name, buf, dims, writes in (("residual", residual, (m, k), False), ("residual_out", residual_out, (m, k), True),
                                        ("gate_up", gate_up, (m, 2 * intermediate), True),
                                        ("normed", normed, (m, k), True)):
            if buf is not None:
                args.append((_w if writes else _r)(name, buf, 2, *dims))
        self._admit("rms_gemm_silu", args)
        ptr = lambda b: None if b is None else b.ptr  # noqa: E731
        self._call(self.lib.nv_rms_gemm_silu(self.handle, x.ptr, ptr(residual), ptr(residual_out), norm_weight.ptr,
                                             w_tiled.ptr, ptr(gate_up), act.ptr, ptr(normed), m, intermediate, k, eps))

    def add_rms_norm_gather(self, x: Buffer, residual: Buffer, weight: Buffer, indices: Buffer, out: Buffer,
                            rows: int, hidden: int, input_rows: int, eps: float) -> None:
        """The output of add_rms_norm for input rows indices[r] in output row r (a +0 row for an index
        outside [0, input_rows)); residual is read, not updated."""
        require_positive(eps, "add_rms_norm_gather eps")
        self._admit("add_rms_norm_gather", [
            _r("x", x, 2, input_rows, hidden), _r("residual", residual, 2, input_rows, hidden),
            _r("weight", weight, 2, hidden), _r("indices", indices, 4, rows), _w("out", out, 2, rows, hidden)])
        self._call(self.lib.nv_add_rms_gather(self.handle, x.ptr, residual.ptr, weight.ptr, indices.ptr, out.ptr,
                                              rows, hidden, input_rows, eps))

    @staticmethod
    def _rope_args(qkv, qweight, kweight, positions, slots, qout, kcache, vcache, rows, qheads, kvheads, head_dim,
                   block_size, num_blocks):
        args = [_r("qkv", qkv, 2, rows, qheads + 2 * kvheads, head_dim), _r("qweight", qweight, 2, head_dim),
                _r("kweight", kweight, 2, head_dim), _r("positions", positions, 4, rows), _r("slots", slots, 4, rows),
                _w("kcache", kcache, 2, num_blocks, block_size, kvheads, head_dim),
                _w("vcache", vcache, 2, num_blocks, block_size, kvheads, head_dim)]
        if qout is not None:
            args.append(_w("qout", qout, 2, rows, qheads, head_dim))
        return args

    def qkv_rope(self, qkv, qweight, kweight, positions, slots, qout, kcache, vcache, rows, qheads, kvheads,
                 head_dim, block_size, num_blocks, eps, theta) -> None:
        """Per-head q/k RMSNorm + NeoX RoPE (angle computed inline) + KV write."""
        require_positive(eps, "qkv_rope eps")
        require_positive(theta, "qkv_rope theta")
        require_head_layout(qheads, kvheads, head_dim)
        self._admit("qkv_rope", self._rope_args(qkv, qweight, kweight, positions, slots, qout, kcache, vcache, rows,
                                                qheads, kvheads, head_dim, block_size, num_blocks))
        self._call(self.lib.nv_qkv_rope(self.handle, qkv.ptr, qweight.ptr, kweight.ptr, positions.ptr, slots.ptr,
                                        qout.ptr, kcache.ptr, vcache.ptr, rows, qheads, kvheads, head_dim, block_size,
                                        num_blocks, eps, theta))

    def rope_cache(self, cache: Buffer, max_positions: int, head_dim: int, theta: float) -> None:
        """f32 [max_positions, head_dim]: cos of the head_dim/2 pairs, then sin."""
        require_positive(theta, "rope_cache theta")
        require_head_layout(1, 1, head_dim)
        self._admit("rope_cache", [_w("cache", cache, 4, max_positions, head_dim)])
        self._call(self.lib.nv_rope_cache(self.handle, cache.ptr, max_positions, head_dim, theta))

    def qkv_rope_cached(self, qkv, qweight, kweight, positions, slots, qout, kcache, vcache, rows, qheads, kvheads,
                        head_dim, block_size, num_blocks, eps, rope_cache, max_positions) -> None:
        """As qkv_rope with cos/sin from the table; positions outside [0, max_positions) rotate by 0."""
        require_positive(eps, "qkv_rope_cached eps")
        require_head_layout(qheads, kvheads, head_dim)
        args = self._rope_args(qkv, qweight, kweight, positions, slots, qout, kcache, vcache, rows, qheads, kvheads,
                               head_dim, block_size, num_blocks)
        self._admit("qkv_rope_cached", args + [_r("rope_cache", rope_cache, 4, max_positions, head_dim)])
        self._call(self.lib.nv_qkv_rope_cached(self.handle, qkv.ptr, qweight.ptr, kweight.ptr, positions.ptr,
                                               slots.ptr, qout.ptr, kcache.ptr, vcache.ptr, rows, qheads, kvheads,
                                               head_dim, block_size, num_blocks, eps, rope_cache.ptr, max_positions))

    @staticmethod
    def _context_limit(max_context: int) -> None:
        if not 1 <= max_context <= 4096:
            raise ArgumentError("value", f"max_context {max_context} outside [1, 4096]")

    def paged_attention(self, q: Buffer, kcache: Buffer, vcache: Buffer, positions: Buffer, seq_indices: Buffer,
                        block_tables: Buffer, out: Buffer, rows: int, qheads: int, kvheads: int, head_dim: int,
                        block_size: int, num_blocks: int, table_stride: int, batch_size: int,
                        max_context: int) -> None:
        """Causal paged GQA over flattened ragged rows; row r reads positions[r] + 1 keys."""
        require_head_layout(qheads, kvheads, head_dim)
        self._context_limit(max_context)
        self._admit("paged_attention", [
            _r("q", q, 2, rows, qheads, head_dim), _r("kcache", kcache, 2, num_blocks, block_size, kvheads, head_dim),
            _r("vcache", vcache, 2, num_blocks, block_size, kvheads, head_dim), _r("positions", positions, 4, rows),
            _r("seq_indices", seq_indices, 4, rows), _r("block_tables", block_tables, 4, batch_size, table_stride),
            _w("out", out, 2, rows, qheads, head_dim)])
        self._call(self.lib.nv_attention(self.handle, q.ptr, kcache.ptr, vcache.ptr, positions.ptr, seq_indices.ptr,
                                         block_tables.ptr, out.ptr, rows, qheads, kvheads, head_dim, block_size,
                                         num_blocks, table_stride, batch_size, max_context))

    def attention_qkv_rope(self, qkv: Buffer, qweight: Buffer, kweight: Buffer, positions: Buffer, slots: Buffer,
                           kcache: Buffer, vcache: Buffer, seq_indices: Buffer, block_tables: Buffer, out: Buffer,
                           rows: int, qheads: int, kvheads: int, head_dim: int, block_size: int, num_blocks: int,
                           table_stride: int, batch_size: int, max_context: int, eps: float, rope_cache: Buffer,
                           max_positions: int) -> None:
        """qkv_rope_cached + paged_attention in one launch for decode batches (head dim 128);
        no row may read a KV slot that another row writes."""
        require_positive(eps, "attention_qkv_rope eps")
        require_head_layout(qheads, kvheads, head_dim)
        if head_dim != 128:
            raise ArgumentError("value", "attention_qkv_rope takes head_dim 128 only")
        self._context_limit(max_context)
        args = self._rope_args(qkv, qweight, kweight, positions, slots, None, kcache, vcache, rows, qheads, kvheads,
                               head_dim, block_size, num_blocks)
        self._admit("attention_qkv_rope", args + [
            _r("seq_indices", seq_indices, 4, rows), _r("block_tables", block_tables, 4, batch_size, table_stride),
            _r("rope_cache", rope_cache, 4, max_positions, head_dim), _w("out", out, 2, rows, qheads, head_dim)])
        self._call(self.lib.nv_attention_qkv_rope(self.handle, qkv.ptr, qweight.ptr, kweight.ptr, positions.ptr,
                                                  slots.ptr, kcache.ptr, vcache.ptr, seq_indices.ptr,
                                                  block_tables.ptr, out.ptr, rows, qheads, kvheads, head_dim,
                                                  block_size, num_blocks, table_stride, batch_size, max_context, eps,
                                                  rope_cache.ptr, max_positions))

    def kv_write(self, k: Buffer, v: Buffer, slots: Buffer, kcache: Buffer, vcache: Buffer, rows: int,
                 kvheads: int, head_dim: int, block_size: int, num_blocks: int) -> None:
        """kcache[slots[r]] = k[r], vcache[slots[r]] = v[r] for slots in [0, block_size * num_blocks)."""
        if as_dim(kvheads) * as_dim(head_dim) > INT_MAX:
            raise ArgumentError("dimension", "kv_write: kvheads * head_dim exceeds 2^31 - 1")
        self._admit("kv_write", [
            _r("k", k, 2, rows, kvheads, head_dim), _r("v", v, 2, rows, kvheads, head_dim),
            _r("slots", slots, 4, rows), _w("kcache", kcache, 2, num_blocks, block_size, kvheads, head_dim),
            _w("vcache", vcache, 2, num_blocks, block_size, kvheads, head_dim)])
        self._call(self.lib.nv_kv_write(self.handle, k.ptr, v.ptr, slots.ptr, kcache.ptr, vcache.ptr, rows, kvheads,
                                        head_dim, block_size, num_blocks))

    def silu_mul(self, gateup: Buffer, out: Buffer, rows: int, intermediate: int) -> None:
        """out[r] = bf16(silu(gate) * up) with gateup = [rows, 2, intermediate]."""
        if intermediate > INT_MAX // 2:
            raise ArgumentError("dimension", "silu_mul: 2 * intermediate exceeds 2^31 - 1")
        self._admit("silu_mul", [_r("gateup", gateup, 2, rows, 2, intermediate),
                                 _w("out", out, 2, rows, intermediate)])
        self._call(self.lib.nv_silu(self.handle, gateup.ptr, out.ptr, rows, intermediate))

    def gather(self, x: Buffer, indices: Buffer, out: Buffer, rows: int, hidden: int, input_rows: int) -> None:
        self._admit("gather", [_r("x", x, 2, input_rows, hidden), _r("indices", indices, 4, rows),
                               _w("out", out, 2, rows, hidden)])
        self._call(self.lib.nv_gather(self.handle, x.ptr, indices.ptr, out.ptr, rows, hidden, input_rows))

    @staticmethod
    def _sampler_args(logits, temperatures, seeds, out, batch, vocab):
        return [_r("logits", logits, 2, batch, vocab), _r("temperatures", temperatures, 4, batch),
                _r("seeds", seeds, 8, batch), _w("out", out, 4, batch)]

    def sample(self, logits: Buffer, temperatures: Buffer, seeds: Buffer, out: Buffer, batch: int,
               vocab: int) -> None:
        """bf16 logits; f32 temperatures (<= 0 greedy); u64 seeds; i32 output."""
        self._admit("sample", self._sampler_args(logits, temperatures, seeds, out, batch, vocab))
        self._call(self.lib.nv_sample(self.handle, logits.ptr, temperatures.ptr, seeds.ptr, out.ptr, batch, vocab))

    def sample_parallel(self, logits: Buffer, temperatures: Buffer, seeds: Buffer, out: Buffer,
                        partial_scores: Buffer, partial_ids: Buffer, batch: int, vocab: int) -> None:
        """Vocabulary-parallel sampling; scratch holds batch x ceil(vocab/2048) entries."""
        parts = -(-vocab // 2048)
        self._admit("sample_parallel", self._sampler_args(logits, temperatures, seeds, out, batch, vocab) + [
            _w("partial_scores", partial_scores, 4, batch, parts), _w("partial_ids", partial_ids, 4, batch, parts)])
        self._call(self.lib.nv_sample_parallel(self.handle, logits.ptr, temperatures.ptr, seeds.ptr, out.ptr,
                                               partial_scores.ptr, partial_ids.ptr, batch, vocab))

    STATIC_PARTIALS = 1 << 17

    def sample_parallel_static(self, logits: Buffer, temperatures: Buffer, seeds: Buffer, out: Buffer, batch: int,
                               vocab: int) -> None:
        """sample_parallel with the library's static partials instead of caller
        scratch (no allocation): batch * ceil(vocab / 2048) <= 131072."""
        self._admit("sample_parallel_static", self._sampler_args(logits, temperatures, seeds, out, batch, vocab))
        self._call(self.lib.nv_sample_parallel_static(self.handle, logits.ptr, temperatures.ptr, seeds.ptr, out.ptr,
                                                      batch, vocab))


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
