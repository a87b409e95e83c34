"""ctypes binding of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, as the checker of the HIP library. The product
(nano-vllm-rs_amd/) never imports it.

Arrays are numpy: bf16 tensors are uint16 bit patterns, ints are int32,
seeds uint64, temperatures and RoPE tables float32.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

_p = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_u64 = ctypes.c_uint64

_SIGS = {
    "ora_bf16_from_f32": (ctypes.c_uint16, [_f]),
    "ora_f32_from_bf16": (_f, [ctypes.c_uint16]),
    "ora_splitmix64": (_u64, [_u64]),
    "ora_sampling_seed": (_u64, [_u64, _u64, _u64]),
    "ora_logf": (_f, [_f]),
    "ora_logf_n": (None, [_p, _p, ctypes.c_size_t]),
    "ora_expf": (_f, [_f]),
    "ora_expf_n": (None, [_p, _p, ctypes.c_size_t]),
    "ora_attention": (None, [_p] * 7 + [_i] * 10),
    "ora_gumbel_score": (_f, [_f, _f, _u64, ctypes.c_uint32]),
    "ora_rope_cos_sin": (None, [_i, _i, _i, _f, ctypes.POINTER(_f), ctypes.POINTER(_f)]),
    "ora_block_sum_sq": (_f, [_p, _i]),
    "ora_embedding": (None, [_p, _p, _p, _i, _i, _i, _i]),
    "ora_gather": (None, [_p, _p, _p, _i, _i, _i, _i]),
    "ora_rms": (None, [_p, _p, _p, _i, _i, _f, _i]),
    "ora_add_rms": (None, [_p, _p, _p, _p, _i, _i, _f, _i]),
    "ora_rope_cache": (None, [_p, _i, _i, _f, _i]),
    "ora_qkv_rope": (None, [_p] * 8 + [_i] * 6 + [_f, _f, _p, _i, _i]),
    "ora_kv_write": (None, [_p] * 5 + [_i] * 6),
    "ora_silu": (None, [_p, _p, _i, _i, _i]),
    "ora_sample": (None, [_p, _p, _p, _p, _i, _i, _i]),
    "ora_sample_partitioned": (None, [_p] * 6 + [_i, _i, _i]),
    "ora_fill_normal_bf16": (None, [_p, ctypes.c_size_t, _u64, ctypes.c_double, ctypes.c_double]),
}

_LIB = None


def build() -> None:
    """Compiles liboracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            build()
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = l
    return _LIB


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------------ data ----
def normal_bf16(shape, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """Seeded bf16 normals (SplitMix64 stream + Box-Muller), as uint16 bits."""
    out = np.empty(shape, dtype=np.uint16)
    lib().ora_fill_normal_bf16(out.ctypes.data, out.size, seed & (2**64 - 1), mean, std)
    return out


# --------------------------------------------------------------- scalars ----
def logf(x: float) -> float:
    return lib().ora_logf(x)


def logf_array(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib().ora_logf_n(x.ctypes.data, out.ctypes.data, x.size)
    return out


def expf(x: float) -> float:
    return lib().ora_expf(x)


def expf_array(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib().ora_expf_n(x.ctypes.data, out.ctypes.data, x.size)
    return out


def splitmix64(v: int) -> int:
    return int(lib().ora_splitmix64(v & (2**64 - 1)))


def sampling_seed(base: int, request_id: int, generated: int) -> int:
    return int(lib().ora_sampling_seed(base, request_id, generated))


def gumbel_score(logit: float, temperature: float, seed: int, token: int) -> float:
    return lib().ora_gumbel_score(logit, temperature, seed, token)


def rope_cos_sin(position: int, pair: int, dim: int, theta: float) -> tuple[float, float]:
    c, s = _f(), _f()
    lib().ora_rope_cos_sin(position, pair, dim, theta, ctypes.byref(c), ctypes.byref(s))
    return c.value, s.value


def block_sum_sq(values: np.ndarray) -> float:
    v = _c(values, np.float32)
    return lib().ora_block_sum_sq(v.ctypes.data, v.size)


# --------------------------------------------------------------- kernels ----
def embedding(tokens, weight, rows, hidden, vocab, threads=1):
    tokens, weight = _c(tokens, np.int32), _c(weight, np.uint16)
    out = np.empty((rows, hidden), np.uint16)
    lib().ora_embedding(_ptr(tokens), _ptr(weight), _ptr(out), rows, hidden, vocab, threads)
    return out


def gather(x, indices, rows, hidden, input_rows, threads=1):
    x, indices = _c(x, np.uint16), _c(indices, np.int32)
    out = np.empty((rows, hidden), np.uint16)
    lib().ora_gather(_ptr(x), _ptr(indices), _ptr(out), rows, hidden, input_rows, threads)
    return out


def rms(x, weight, rows, hidden, eps, threads=1):
    x, weight = _c(x, np.uint16), _c(weight, np.uint16)
    out = np.empty((rows, hidden), np.uint16)
    lib().ora_rms(_ptr(x), _ptr(weight), _ptr(out), rows, hidden, eps, threads)
    return out


def add_rms(x, residual, weight, rows, hidden, eps, threads=1):
    """Returns (new residual, out)."""
    x, weight = _c(x, np.uint16), _c(weight, np.uint16)
    res = np.array(residual, dtype=np.uint16, copy=True, order="C")
    out = np.empty((rows, hidden), np.uint16)
    lib().ora_add_rms(_ptr(x), _ptr(res), _ptr(weight), _ptr(out), rows, hidden, eps, threads)
    return res, out


def rope_cache(positions, dim, theta, threads=1):
    out = np.empty((positions, dim), np.float32)
    lib().ora_rope_cache(_ptr(out), positions, dim, theta, threads)
    return out


def qkv_rope(qkv, qw, kw, positions, slots, kc, vc, rows, qh, kvh, dim, bs, blocks, eps, theta=1.0, table=None,
             max_positions=0, threads=1):
    """Returns (qout, kcache, vcache); kc/vc are the caches before the write."""
    qkv, qw, kw = _c(qkv, np.uint16), _c(qw, np.uint16), _c(kw, np.uint16)
    positions, slots = _c(positions, np.int32), _c(slots, np.int32)
    kc = np.array(kc, dtype=np.uint16, copy=True, order="C")
    vc = np.array(vc, dtype=np.uint16, copy=True, order="C")
    qout = np.zeros((rows, qh, dim), np.uint16)
    tab = None if table is None else _c(table, np.float32)
    lib().ora_qkv_rope(_ptr(qkv), _ptr(qw), _ptr(kw), _ptr(positions), _ptr(slots), _ptr(qout), _ptr(kc), _ptr(vc),
                       rows, qh, kvh, dim, bs, blocks, eps, theta, _ptr(tab), max_positions, threads)
    return qout, kc, vc


def kv_write(k, v, slots, kc, vc, rows, kvh, dim, bs, blocks, threads=1):
    k, v, slots = _c(k, np.uint16), _c(v, np.uint16), _c(slots, np.int32)
    kc = np.array(kc, dtype=np.uint16, copy=True, order="C")
    vc = np.array(vc, dtype=np.uint16, copy=True, order="C")
    lib().ora_kv_write(_ptr(k), _ptr(v), _ptr(slots), _ptr(kc), _ptr(vc), rows, kvh, dim, bs, blocks, threads)
    return kc, vc


def silu(packed, rows, intermediate, threads=1):
    packed = _c(packed, np.uint16)
    out = np.empty((rows, intermediate), np.uint16)
    lib().ora_silu(_ptr(packed), _ptr(out), rows, intermediate, threads)
    return out


def sample(logits, temps, seeds, batch, vocab, threads=1):
    logits, temps, seeds = _c(logits, np.uint16), _c(temps, np.float32), _c(seeds, np.uint64)
    out = np.empty(batch, np.int32)
    lib().ora_sample(_ptr(logits), _ptr(temps), _ptr(seeds), _ptr(out), batch, vocab, threads)
    return out


def sample_partitioned(logits, temps, seeds, batch, vocab, width=2048):
    """Returns (out, partial_scores, partial_ids)."""
    logits, temps, seeds = _c(logits, np.uint16), _c(temps, np.float32), _c(seeds, np.uint64)
    parts = -(-vocab // width)
    out = np.empty(batch, np.int32)
    ps = np.empty((batch, parts), np.float32)
    pi = np.empty((batch, parts), np.int32)
    lib().ora_sample_partitioned(_ptr(logits), _ptr(temps), _ptr(seeds), _ptr(out), _ptr(ps), _ptr(pi), batch,
                                 vocab, width)
    return out, ps, pi


def attention(q, kc, vc, positions, seqs, tables, rows, qh, kvh, dim, bs, blocks, stride, batch, max_context,
              threads=1):
    """Paged causal GQA attention; returns out [rows, qh, dim] bf16 bits."""
    q, kc, vc = _c(q, np.uint16), _c(kc, np.uint16), _c(vc, np.uint16)
    positions, seqs, tables = _c(positions, np.int32), _c(seqs, np.int32), _c(tables, np.int32)
    out = np.empty((rows, qh, dim), np.uint16)
    lib().ora_attention(_ptr(q), _ptr(kc), _ptr(vc), _ptr(positions), _ptr(seqs), _ptr(tables), _ptr(out), rows, qh,
                        kvh, dim, bs, blocks, stride, batch, max_context, threads)
    return out
