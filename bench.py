#!/usr/bin/env python3
"""Benchmark of the nano-vllm-rs fused per-layer kernels on one MI355X.

Step (the `value` workload): the fused, non-GEMM kernels of one Qwen3-0.6B
forward pass over T = 8192 prompt tokens, in the reference's order
(src/model.rs:649-789):

    embedding(tokens -> residual)
    layer 0: rms(residual -> normed)            layers 1..27: add_rms(mlp_out[l-1], residual -> normed)
             qkv_rope_cached(qkv[l] -> query, kcache[l], vcache[l])
             add_rms(attn_out[l], residual -> normed)
             silu(gate_up[l] -> act)
    add_rms(mlp_out[27], residual -> normed)     (final norm)

The GEMM/attention outputs that feed these kernels (qkv[l], attn_out[l],
gate_up[l], mlp_out[l]) are synthetic bf16 tensors, one per layer, resident
in HBM before timing starts. The step is captured once as a HIP graph and
replayed; `value` is tokens per second of that step.

Per-kernel lines reproduce the kernel workloads (RMSNorm 8x1024, q/k norm +
RoPE at 2048 and 8192 tokens, add-RMSNorm 8192x1024, SiLU 8192x6144, embedding
and KV write at 16384 tokens, sampling 256x151936). Each is launched over
several distinct buffer sets totalling more than 512 MB so that no launch finds
its data in the 256 MB Infinity Cache; time is HIP events on the library's
stream around the whole loop, divided by the launch count.

The CPU baseline runs the oracle's multithreaded C restatement of the same
step (all 28 layers, T = 8192) on the host cores.

`decode` reports the whole Qwen3-0.6B forward (GEMMs and attention included,
random weights) as the C++ runner serves it: 1024 prompt tokens, then decode
steps of 8 and 32 rows, each step one HIP graph replay (decode_bench).

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-kernels] [--no-decode]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nano-vllm-rs_amd"))

import nvr  # noqa: E402

METRIC = "achieved HBM GB/s and % roofline per fused kernel; tokens/s at T=8192, 1 MI355X"
HBM_PEAK_GBS = 8000.0

# Qwen3-0.6B shapes (src/model.rs:1407-1411).
H, I, QH, KVH, D, V, LAYERS = 1024, 3072, 16, 8, 128, 151936, 28
HEADS = QH + 2 * KVH
EPS, THETA, MAX_POS, BS = 1e-6, 1e6, 4096, 256
MALL_DEFEAT_BYTES = 640 << 20


# ------------------------------------------------------------ HIP plumbing --
class Hip:
    """Events and device copies from the HIP runtime the library already loaded."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        vp = ctypes.c_void_p
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        self.lib.hipEventRecord.argtypes = [vp, vp]
        self.lib.hipEventSynchronize.argtypes = [vp]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        self.lib.hipEventDestroy.argtypes = [vp]
        self.lib.hipMemcpyAsync.argtypes = [vp, vp, ctypes.c_size_t, ctypes.c_int, vp]
        self.lib.hipStreamSynchronize.argtypes = [vp]
        self.lib.hipDeviceSynchronize.argtypes = []

    def check(self, code, what):
        if code != 0:
            raise RuntimeError(f"{what} failed with HIP status {code}")

    def event(self):
        e = ctypes.c_void_p()
        self.check(self.lib.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e

    def destroy(self, e):
        self.check(self.lib.hipEventDestroy(e), "hipEventDestroy")

    def record(self, e, stream):
        self.check(self.lib.hipEventRecord(e, stream), "hipEventRecord")

    def elapsed_ms(self, a, b):
        self.check(self.lib.hipEventSynchronize(b), "hipEventSynchronize")
        ms = ctypes.c_float()
        self.check(self.lib.hipEventElapsedTime(ctypes.byref(ms), a, b), "hipEventElapsedTime")
        return float(ms.value)

    def copy_d2d(self, dst, src, nbytes, stream):
        self.check(self.lib.hipMemcpyAsync(dst, src, nbytes, 3, stream), "hipMemcpyAsync")

    def device_sync(self):
        self.check(self.lib.hipDeviceSynchronize(), "hipDeviceSynchronize")


class Filler:
    """Fills device buffers with seeded bf16 normals: one host-generated pool per
    distribution is uploaded once, then tiled with device-to-device copies."""

    POOL = 16 << 20  # elements (32 MiB of bf16)

    def __init__(self, gpu: nvr.Gpu, hip: Hip):
        self.gpu, self.hip, self.pools = gpu, hip, {}
        self.stream = gpu.stream()

    def pool(self, mean, std):
        key = (mean, std)
        if key not in self.pools:
            rng = np.random.default_rng(abs(hash(key)) % (2**32))
            vals = (mean + std * rng.standard_normal(self.POOL, dtype=np.float32)).astype(np.float32)
            self.pools[key] = self.gpu.upload_array(nvr.bf16_bits(vals))
        return self.pools[key]

    def normal(self, nbytes, mean=0.0, std=1.0):
        buf = self.gpu.alloc(nbytes)
        src = self.pool(mean, std)
        off = 0
        # Start each buffer at a different pool offset so tiles are not identical.
        shift = int(np.random.default_rng(nbytes ^ int(std * 1000)).integers(0, src.bytes // 2)) & ~15
        while off < nbytes:
            n = min(src.bytes - shift, nbytes - off)
            self.hip.copy_d2d(buf.ptr + off, src.ptr + shift, n, self.stream)
            off += n
            shift = 0
        return buf

    def ints(self, values: np.ndarray):
        return self.gpu.upload_array(np.ascontiguousarray(values, dtype=np.int32))


# ----------------------------------------------------- algorithmic bytes --
def bytes_rms(rows, hidden):
    return 2 * rows * hidden * 2 + hidden * 2


def bytes_add_rms(rows, hidden):
    return 4 * rows * hidden * 2 + hidden * 2


def bytes_qkv_rope(rows, distinct_positions):
    return rows * HEADS * D * 2 * 2 + rows * 8 + 2 * D * 2 + distinct_positions * D * 4


def bytes_silu(rows, inter):
    return rows * 3 * inter * 2


def bytes_embedding(rows, hidden):
    return rows * 4 + 2 * rows * hidden * 2


def bytes_kv_write(rows):
    return rows * 4 + 2 * 2 * rows * KVH * D * 2


def bytes_attention(rows, context, table_stride):
    """K and V rows of every context token of each (row, kv head), q, out and
    the row's metadata."""
    return rows * (2 * context * KVH * D * 2 + 2 * QH * D * 2 + 8 + table_stride * 4)


def bytes_sampling(batch, vocab):
    return batch * vocab * 2 + batch * (4 + 8 + 4)


# ------------------------------------------------------------- the step ----
class Chain:
    def __init__(self, gpu: nvr.Gpu, fill: Filler, tokens: int, layers: int, seed: int = 0):
        self.gpu, self.T, self.L = gpu, tokens, layers
        T = tokens
        rng = np.random.default_rng(seed)
        self.blocks = -(-T // BS)
        self.tok = fill.ints(rng.integers(0, V, T))
        self.table = fill.normal(V * H * 2, 0.0, 0.02)
        self.residual = gpu.alloc(T * H * 2)
        self.normed = gpu.alloc(T * H * 2)
        self.query = gpu.alloc(T * QH * D * 2)
        self.act = gpu.alloc(T * I * 2)
        # Prefill batch of sequences of MAX_POS tokens: positions restart per
        # sequence; slots come from a random permutation of cache blocks.
        pos = (np.arange(T) % MAX_POS).astype(np.int32)
        perm = rng.permutation(self.blocks)
        slots = (perm[np.arange(T) // BS] * BS + np.arange(T) % BS).astype(np.int32)
        self.distinct_positions = int(len(np.unique(pos)))
        self.pos, self.slots = fill.ints(pos), fill.ints(slots)
        self.rope = gpu.alloc(MAX_POS * D * 4)
        gpu.rope_cache(self.rope, MAX_POS, D, THETA)
        self.final_norm = fill.normal(H * 2, 1.0, 0.02)
        self.layers = []
        for _ in range(layers):
            self.layers.append(dict(
                in_norm=fill.normal(H * 2, 1.0, 0.02), post_norm=fill.normal(H * 2, 1.0, 0.02),
                q_norm=fill.normal(D * 2, 1.0, 0.02), k_norm=fill.normal(D * 2, 1.0, 0.02),
                qkv=fill.normal(T * HEADS * D * 2), attn_out=fill.normal(T * H * 2),
                gate_up=fill.normal(T * 2 * I * 2, 0.0, 2.0), mlp_out=fill.normal(T * H * 2),
                kc=gpu.alloc(self.blocks * BS * KVH * D * 2), vc=gpu.alloc(self.blocks * BS * KVH * D * 2)))

    def step(self):
        g, T = self.gpu, self.T
        g.embedding(self.tok, self.table, self.residual, T, H, V)
        for i, l in enumerate(self.layers):
            if i == 0:
                g.rms_norm(self.residual, l["in_norm"], self.normed, T, H, EPS)
            else:
                g.add_rms_norm(self.layers[i - 1]["mlp_out"], self.residual, l["in_norm"], self.normed, T, H, EPS)
            g.qkv_rope_cached(l["qkv"], l["q_norm"], l["k_norm"], self.pos, self.slots, self.query, l["kc"], l["vc"],
                              T, QH, KVH, D, BS, self.blocks, EPS, self.rope, MAX_POS)
            g.add_rms_norm(l["attn_out"], self.residual, l["post_norm"], self.normed, T, H, EPS)
            g.silu_mul(l["gate_up"], self.act, T, I)
        g.add_rms_norm(self.layers[-1]["mlp_out"], self.residual, self.final_norm, self.normed, T, H, EPS)

    def bytes(self):
        T, L = self.T, self.L
        return (bytes_embedding(T, H) + bytes_rms(T, H) + (2 * L - 1) * bytes_add_rms(T, H) + bytes_add_rms(T, H)
                + L * bytes_qkv_rope(T, self.distinct_positions) + L * bytes_silu(T, I))

    def launches(self):
        return {"embedding": 1, "rms": 1, "add_rms": 2 * self.L, "qkv_rope_cached": self.L, "silu": self.L}


def time_graph(gpu, hip, graph, reps, warmup):
    stream = gpu.stream()
    for _ in range(warmup):
        graph.replay()
    gpu.sync()
    hip.device_sync()
    a, b = hip.event(), hip.event()
    try:
        hip.record(a, stream)
        for _ in range(reps):
            graph.replay()
        hip.record(b, stream)
        ms = hip.elapsed_ms(a, b)
    finally:
        # Events hold runtime resources; a timing loop that never released
        # them ended in a crash inside hipGraphLaunch after ~10^3 calls.
        hip.destroy(a)
        hip.destroy(b)
    gpu.sync()
    hip.device_sync()
    return ms / reps


# ------------------------------------------------------ per-kernel loops ---
LAYOUT_SEEDS = (1, 2, 3, 4, 5)


def add_spikes(buf, rows, vocab, count, amount, rng):
    """Adds `amount` to one random logit in each of `count` random rows of a
    bf16 [rows, vocab] device buffer (rounded once to bf16)."""
    for r in rng.choice(rows, count, replace=False):
        off = (int(r) * vocab + int(rng.integers(0, vocab))) * 2
        cell = buf.slice(off, 2)
        value = nvr.bf16_values(cell.download(np.uint16, 1))[0]
        cell.upload(nvr.bf16_bits(np.array([value + amount], np.float32)))


def slot_layouts(tokens, cache_blocks):
    """Slot layouts of the sweep: identity slots, then the block permutations
    of LAYOUT_SEEDS (slot = perm[t // 256] * 256 + t % 256)."""
    t = np.arange(tokens)
    out = [("@identity", t.astype(np.int32))]
    for seed in LAYOUT_SEEDS:
        perm = np.random.default_rng(seed).permutation(cache_blocks)
        out.append((f"@perm{seed}", (perm[t // BS] * BS + t % BS).astype(np.int32)))
    return out


def kernel_cases(gpu: nvr.Gpu, hip: Hip, fill: Filler, chain: Chain, only=(), sweep_layouts=True):
    """(name, workload, launch closures over rotating sets, bytes per launch, rows per launch) per case."""
    cases = []

    def want(*names):
        return not only or any(n in only for n in names)

    def sets_for(per_set_bytes):
        return max(3, -(-MALL_DEFEAT_BYTES // per_set_bytes))

    w = fill.normal(H * 2, 1.0, 0.02)
    # A plain device-to-device copy of 256 MiB by the HIP runtime's own copy
    # kernel: the counters' calibration and the copy rate of this GPU.
    if COPY_CASE in only:  # the counters' calibration: only when named
        n = COPY_BYTES
        srcs = [gpu.alloc(n) for _ in range(3)]
        dsts = [gpu.alloc(n) for _ in range(3)]
        stream = gpu.stream()
        cases.append((COPY_CASE, "device-to-device copy of 256 MiB (HIP runtime copy kernel)",
                      [lambda i=i: hip.copy_d2d(dsts[i].ptr, srcs[i].ptr, n, stream) for i in range(3)], 2 * n, 0))

    # RMSNorm 8 x 1024 (latency-bound decode shape).
    if want("rms_8x1024"):
        n = 64
        xs = [fill.normal(8 * H * 2) for _ in range(n)]
        outs = [gpu.alloc(8 * H * 2) for _ in range(n)]
        cases.append(("rms_8x1024", "RMSNorm x[8,1024]",
                      [lambda i=i: gpu.rms_norm(xs[i], w, outs[i], 8, H, EPS) for i in range(n)], bytes_rms(8, H), 8))

    # add-RMSNorm 8192 x 1024.
    T = 8192
    if want("add_rms_8192x1024"):
        s = sets_for(3 * T * H * 2)
        ax = [fill.normal(T * H * 2) for _ in range(s)]
        ar = [fill.normal(T * H * 2) for _ in range(s)]
        ao = [gpu.alloc(T * H * 2) for _ in range(s)]
        cases.append(("add_rms_8192x1024", "residual add + RMSNorm [8192,1024]",
                      [lambda i=i, T=T: gpu.add_rms_norm(ax[i], ar[i], w, ao[i], T, H, EPS) for i in range(s)],
                      bytes_add_rms(T, H), T))

    # SiLU 8192 x 6144 -> 8192 x 3072.
    if want("silu_8192x6144"):
        s = sets_for(3 * T * I * 2)
        gus = [fill.normal(T * 2 * I * 2, 0.0, 2.0) for _ in range(s)]
        acts = [gpu.alloc(T * I * 2) for _ in range(s)]
        cases.append(("silu_8192x6144", "SiLU(gate)*up [8192,6144] -> [8192,3072]",
                      [lambda i=i, T=T: gpu.silu_mul(gus[i], acts[i], T, I) for i in range(s)], bytes_silu(T, I), T))

    # q/k norm + RoPE + KV write at 2048, 4096 and 8192 tokens, uniform random
    # positions; slots from a random permutation of the cache blocks. At 8192
    # tokens the same buffers are also written through identity slots and five
    # more block permutations (cases "qkv_rope_8192@<layout>").
    for T in (2048, 4096, 8192):
        if not want(f"qkv_rope_{T}"):
            continue
        rng = np.random.default_rng(T)
        pos = rng.integers(0, MAX_POS, T).astype(np.int32)
        blocks = T // BS
        perm = rng.permutation(blocks)
        slots = (perm[np.arange(T) // BS] * BS + np.arange(T) % BS).astype(np.int32)
        pb = fill.ints(pos)
        per = T * HEADS * D * 2 * 2
        s = sets_for(per)
        qkvs = [fill.normal(T * HEADS * D * 2) for _ in range(s)]
        qos = [gpu.alloc(T * QH * D * 2) for _ in range(s)]
        kcs = [gpu.alloc(blocks * BS * KVH * D * 2) for _ in range(s)]
        vcs = [gpu.alloc(blocks * BS * KVH * D * 2) for _ in range(s)]
        qn, kn = fill.normal(D * 2, 1.0, 0.02), fill.normal(D * 2, 1.0, 0.02)
        nbytes = bytes_qkv_rope(T, len(np.unique(pos)))
        layouts = [("", slots)] + (slot_layouts(T, blocks) if T == 8192 and sweep_layouts else [])
        for tag, sl in layouts:
            sb = fill.ints(sl)
            cases.append((f"qkv_rope_{T}{tag}", f"q/k RMSNorm + NeoX RoPE + KV write, {T} tokens",
                          [lambda i=i, T=T, pb=pb, sb=sb, blocks=blocks, qkvs=qkvs, qos=qos, kcs=kcs, vcs=vcs, qn=qn,
                           kn=kn: gpu.qkv_rope_cached(qkvs[i], qn, kn, pb, sb, qos[i], kcs[i], vcs[i], T, QH, KVH, D,
                                                      BS, blocks, EPS, chain.rope, MAX_POS) for i in range(s)],
                          nbytes, T))

    # Embedding gather, 16384 tokens from a [151936, 1024] table (three tables).
    T = 16384
    if want("embedding_16384"):
        tables = [chain.table] + [fill.normal(V * H * 2, 0.0, 0.02) for _ in range(2)]
        toks = [fill.ints(np.random.default_rng(100 + j).integers(0, V, T)) for j in range(6)]
        eouts = [gpu.alloc(T * H * 2) for _ in range(6)]
        cases.append(("embedding_16384", "embedding gather, 16384 tokens, table [151936,1024]",
                      [lambda j=j, T=T: gpu.embedding(toks[j], tables[j % 3], eouts[j], T, H, V) for j in range(6)],
                      bytes_embedding(T, H), T))

    # Copy ceilings: plain 1:1 copies of 64 MiB and 128 MiB in all (half read,
    # half written), each through the library's faster copy kernel at that
    # size. 64 MiB: the row gather (nv_embedding) over identity ids, 16384
    # rows of 2 KiB (the KV write's 16 rows per wave would fill half the CUs).
    # 128 MiB: nv_kv_write of k, v [16384, 8, 128] through identity slots
    # (every load of a wave in flight before its stores; 0.63 of peak for the
    # gather at this size against 0.78). The streaming kernels'
    # "copy_ceiling" compares them with the copy of about their own traffic.
    if want("copy_64mb"):
        rows = 16384
        s = sets_for(2 * rows * H * 2)
        srcs = [fill.normal(rows * H * 2) for _ in range(s)]
        dsts = [gpu.alloc(rows * H * 2) for _ in range(s)]
        ident = fill.ints(np.arange(rows, dtype=np.int32))
        cases.append(("copy_64mb", f"copy: row gather of {rows} rows of 2 KiB over identity ids",
                      [lambda i=i, rows=rows, ident=ident, srcs=srcs, dsts=dsts:
                       gpu.embedding(ident, srcs[i], dsts[i], rows, H, rows) for i in range(s)],
                      bytes_embedding(rows, H), rows))
    if want("copy_128mb"):
        rows = 16384
        half = rows * KVH * D * 2
        s = sets_for(4 * half)
        cks = [fill.normal(half) for _ in range(s)]
        cvs = [fill.normal(half) for _ in range(s)]
        ckc = [gpu.alloc(half) for _ in range(s)]
        cvc = [gpu.alloc(half) for _ in range(s)]
        cid = fill.ints(np.arange(rows, dtype=np.int32))
        cases.append(("copy_128mb", f"copy: KV write of k, v [{rows},8,128] through identity slots",
                      [lambda i=i, rows=rows, cid=cid, cks=cks, cvs=cvs, ckc=ckc, cvc=cvc:
                       gpu.kv_write(cks[i], cvs[i], cid, ckc[i], cvc[i], rows, KVH, D, BS, rows // BS)
                       for i in range(s)],
                      bytes_kv_write(rows), rows))

    # Paged KV write, k/v [16384, 8, 128] into the per-layer caches of a
    # 28-layer layout ([128, 256, 8, 128] per layer and per K/V, 3.5 GiB in
    # all); launch l writes layer l from source set l mod 5. Slots come from a
    # random permutation of the 128 blocks (the first 64 are written); the
    # same launches also run with identity slots and five more permutations
    # (cases "kv_write_16384@<layout>").
    if want("kv_write_16384"):
        cache_blocks = 128
        nsrc = 5
        ks = [fill.normal(T * KVH * D * 2) for _ in range(nsrc)]
        vs = [fill.normal(T * KVH * D * 2) for _ in range(nsrc)]
        kcs = [gpu.alloc(cache_blocks * BS * KVH * D * 2) for _ in range(LAYERS)]
        vcs = [gpu.alloc(cache_blocks * BS * KVH * D * 2) for _ in range(LAYERS)]
        perm = np.random.default_rng(7).permutation(cache_blocks)
        layouts = [("", (perm[np.arange(T) // BS] * BS + np.arange(T) % BS).astype(np.int32))]
        if sweep_layouts:
            layouts += slot_layouts(T, cache_blocks)
        for tag, slots in layouts:
            sl = fill.ints(slots)
            cases.append((f"kv_write_16384{tag}", "paged KV write k,v [16384,8,128] into a 28-layer cache "
                          "[128,256,8,128] per layer",
                          [lambda l=l, sl=sl: gpu.kv_write(ks[l % nsrc], vs[l % nsrc], sl, kcs[l], vcs[l], T, KVH, D,
                                                           BS, cache_blocks) for l in range(LAYERS)],
                          bytes_kv_write(T), T))

    # Paged attention, decode: 64 sequences at context 4096 (one query row each).
    if want("attention_decode_64x4096"):
        ab, actx = 64, MAX_POS
        astride = actx // BS
        ablocks = ab * astride
        akc = fill.normal(ablocks * BS * KVH * D * 2)
        avc = fill.normal(ablocks * BS * KVH * D * 2)
        atab = fill.ints(np.random.default_rng(11).permutation(ablocks).astype(np.int32))
        apos = fill.ints(np.full(ab, actx - 1, np.int32))
        aseq = fill.ints(np.arange(ab, dtype=np.int32))
        aq = [fill.normal(ab * QH * D * 2) for _ in range(4)]
        aout = [gpu.alloc(ab * QH * D * 2) for _ in range(4)]
        cases.append(("attention_decode_64x4096", "paged GQA attention, 64 decode rows x 4096 context, 16/8 heads, "
                      "dim 128, 256-token blocks (K+V 1.07 GB per launch)",
                      [lambda i=i: gpu.paged_attention(aq[i], akc, avc, apos, aseq, atab, aout[i], ab, QH, KVH, D, BS,
                                                       ablocks, astride, ab, actx) for i in range(4)],
                      bytes_attention(ab, actx, astride), ab))

    # Paged attention, small decode batch: 8 sequences at context 1024 (one
    # query row each), the serving shape where each block walks its context
    # alone on a CU. The caches (8 x 4 blocks of 256 tokens) rotate over sets
    # that together exceed the MALL.
    if want("attention_decode_8x1024"):
        db, dctx = 8, 1024
        dstride = MAX_POS // BS
        dper = dctx // BS
        dsets = sets_for(2 * db * dper * BS * KVH * D * 2)
        dkc = [fill.normal(db * dper * BS * KVH * D * 2) for _ in range(dsets)]
        dvc = [fill.normal(db * dper * BS * KVH * D * 2) for _ in range(dsets)]
        dtab = np.full((db, dstride), -1, np.int32)
        dtab[:, :dper] = np.random.default_rng(12).permutation(db * dper).reshape(db, dper)
        dtab = fill.ints(dtab.reshape(-1))
        dpos = fill.ints(np.full(db, dctx - 1, np.int32))
        dseq = fill.ints(np.arange(db, dtype=np.int32))
        dq = fill.normal(db * QH * D * 2)
        dout = gpu.alloc(db * QH * D * 2)
        cases.append(("attention_decode_8x1024", "paged GQA attention, 8 decode rows x 1024 context, 16/8 heads, "
                      "dim 128, 256-token blocks",
                      [lambda i=i: gpu.paged_attention(dq, dkc[i], dvc[i], dpos, dseq, dtab, dout, db, QH, KVH, D, BS,
                                                       db * dper, dstride, db, MAX_POS) for i in range(dsets)],
                      bytes_attention(db, dctx, dstride), db))

    # The decode form with q/k norm + RoPE + KV write fused into attention, at
    # the same 8 x 1024 shape: it reads the packed qkv rows instead of q and
    # writes each row's K and V slot (token 1023 of its sequence).
    if want("attention_qkv_rope_decode_8x1024"):
        fb, fctx = 8, 1024
        fstride, fper = MAX_POS // BS, fctx // BS
        fsets = sets_for(2 * fb * fper * BS * KVH * D * 2)
        fkc = [fill.normal(fb * fper * BS * KVH * D * 2) for _ in range(fsets)]
        fvc = [fill.normal(fb * fper * BS * KVH * D * 2) for _ in range(fsets)]
        ftab = np.full((fb, fstride), -1, np.int32)
        ftab[:, :fper] = np.random.default_rng(13).permutation(fb * fper).reshape(fb, fper)
        fslots = fill.ints((ftab[:, (fctx - 1) // BS] * BS + (fctx - 1) % BS).astype(np.int32))
        ftab = fill.ints(ftab.reshape(-1))
        fpos = fill.ints(np.full(fb, fctx - 1, np.int32))
        fseq = fill.ints(np.arange(fb, dtype=np.int32))
        fqkv = fill.normal(fb * HEADS * D * 2)
        fqn, fkn = fill.normal(D * 2, 1.0, 0.02), fill.normal(D * 2, 1.0, 0.02)
        fout = gpu.alloc(fb * QH * D * 2)
        # Attention's bytes with the qkv rows read in place of q, plus the
        # K/V slot writes and one cos/sin row per sequence.
        fbytes = bytes_attention(fb, fctx, fstride) + fb * ((HEADS - QH) * D * 2 + 2 * KVH * D * 2 + D * 4)
        cases.append(("attention_qkv_rope_decode_8x1024", "q/k norm + RoPE + KV write fused into paged GQA attention, "
                      "8 decode rows x 1024 context, 16/8 heads, dim 128, 256-token blocks",
                      [lambda i=i: gpu.attention_qkv_rope(fqkv, fqn, fkn, fpos, fslots, fkc[i], fvc[i], fseq, ftab, fout,
                                                          fb, QH, KVH, D, BS, fb * fper, fstride, fb, MAX_POS, EPS,
                                                          chain.rope, MAX_POS) for i in range(fsets)],
                      fbytes, fb))

    # Sampling 256 x 151936: logits ~N(0,3), 1% of the rows (3) with +20 added
    # at one random token; rows 0-127 greedy, 128-255 Gumbel at T=0.6.
    if not want("sampling_256x151936", "sampling_greedy", "sampling_gumbel"):
        return cases
    B = 256
    per = B * V * 2
    s = sets_for(per)
    logits = [fill.normal(B * V * 2, 0.0, 3.0) for _ in range(s)]
    for i, buf in enumerate(logits):
        add_spikes(buf, B, V, round(0.01 * B), 20.0, np.random.default_rng(500 + i))
    parts = -(-V // 2048)
    ps, pi = gpu.alloc(B * parts * 4), gpu.alloc(B * parts * 4)
    out = gpu.alloc(B * 4)
    seeds = gpu.upload_array(np.array([nvr.sampling_seed(0, r, r % 32) for r in range(B)], np.uint64))
    mixed = gpu.upload_array(np.where(np.arange(B) < 128, 0.0, 0.6).astype(np.float32))
    greedy = gpu.upload_array(np.zeros(B, np.float32))
    gumbel = gpu.upload_array(np.full(B, 0.6, np.float32))
    for name, temps, label in (("sampling_256x151936", mixed, "128 greedy + 128 Gumbel (T=0.6) rows"),
                               ("sampling_greedy", greedy, "256 greedy rows"),
                               ("sampling_gumbel", gumbel, "256 Gumbel rows (T=0.6)")):
        if not want(name):
            continue
        cases.append((name, f"sampling logits [256,151936], {label}",
                      [lambda i=i, temps=temps, B=B: gpu.sample_parallel(logits[i], temps, seeds, out, ps, pi, B, V)
                       for i in range(s)], bytes_sampling(B, V), B))
    return cases


TRAFFIC_SUMMARY = os.path.join("profiles", "pmc_traffic.txt")
VALU_SUMMARY = os.path.join("profiles", "sampling_valu.txt")
SCLK_GHZ = 2.4  # MI355X peak engine clock

COPY_CASE, COPY_BYTES = "copy_256mb", 256 << 20
# The kernel each profiled case launches, as a substring of rocprofv3's Kernel_Name.
CASE_KERNEL = {
    COPY_CASE: "__amd_rocclr_copyBuffer",
    "silu_8192x6144": "silu16",
    "add_rms_8192x1024": "rms_rows_fast<4, true, false>",
    "qkv_rope_8192": "qkv_rope_d128<true, 4>",
    "embedding_16384": "gather_rows16",
    "kv_write_16384": "kv_write16",
    "attention_decode_64x4096": "attention_ordered<128, 2, 2, false, false>",
    "sampling_256x151936": "sample_paired<",
    "sampling_greedy": "sample_paired<",
    "sampling_gumbel": "sample_paired<",
}
# The copy case of about each streaming kernel's traffic (64 or 128 MiB).
COPY_CEILING = {"add_rms_8192x1024": "copy_64mb", "embedding_16384": "copy_64mb", "qkv_rope_4096": "copy_64mb",
                "qkv_rope_8192": "copy_128mb", "kv_write_16384": "copy_128mb", "silu_8192x6144": "copy_128mb"}
TRAFFIC_CASES = [COPY_CASE, "silu_8192x6144", "add_rms_8192x1024", "qkv_rope_8192", "embedding_16384",
                 "kv_write_16384", "attention_decode_64x4096", "sampling_gumbel"]
READ_COUNTERS = ["TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum"]
WRITE_COUNTERS = ["TCC_EA0_WRREQ_sum", "TCC_EA0_WRREQ_64B_sum"]
VALU_COUNTERS = ["SQ_INSTS_VALU", "SQ_WAVES", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_INSTS_VMEM"]


def summary_rows(path, width):
    """{case: fields} from a committed summary table whose rows start with a case name."""
    rows = {}
    try:
        for line in open(os.path.join(ROOT, path)):
            tok = line.split()
            if len(tok) == width and tok[0] in CASE_KERNEL and tok[-1].replace(".", "", 1).isdigit():
                rows[tok[0]] = tok
    except OSError:
        pass
    return rows


def measured_traffic(case):
    """HBM bytes per launch of `case` in the committed traffic summary (TCC-to-memory
    read and write requests by size, counted by rocprofv3), or None."""
    row = summary_rows(TRAFFIC_SUMMARY, 7).get(case)
    return int(row[4]) if row else None


def measured_valu(case):
    """VALU wave-instructions per launch of a sampling case in the committed SQ
    counter summary, or None."""
    row = summary_rows(VALU_SUMMARY, 9).get(case)
    return int(row[1]) if row else None


def read_dispatches(directory):
    """[(kernel name, grid size, {counter: value})] per dispatch in dispatch
    order, from the rocprofv3 counter_collection.csv under `directory`."""
    import csv
    import glob

    out = {}
    for path in sorted(glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True)):
        with open(path, newline="") as f:
            for rec in csv.DictReader(f):
                key = (path, int(rec["Dispatch_Id"]))
                name, grid = rec["Kernel_Name"], int(rec["Grid_Size"])
                out.setdefault(key, (name, grid, {}))[2][rec["Counter_Name"]] = float(rec["Counter_Value"])
    return [out[k] for k in sorted(out)]


def case_dispatches(dispatches, case):
    """The dispatches of `case`'s kernel. The runtime's copy kernel also fills
    the buffers while the cases are set up, so the copy case runs last and its
    dispatches are the copies after the last dispatch of any other kernel."""
    if case != COPY_CASE:
        return [d for d in dispatches if CASE_KERNEL[case] in d[0]]
    tail = []
    for d in reversed(dispatches):
        if CASE_KERNEL[case] not in d[0]:
            break
        tail.append(d)
    return tail[::-1]


def pmc_summary(kind, dirs, cases_bytes):
    """Prints the table of a counter pass (see --pmc-summary)."""
    def mean(ds, f):
        return sum(f(c) for _, _, c in ds) / len(ds)

    if kind == "traffic":
        rd, wr = read_dispatches(dirs[0]), read_dispatches(dirs[1])

        def read_b(c):
            return 32 * c["TCC_EA0_RDREQ_32B_sum"] + 64 * c["TCC_EA0_RDREQ_64B_sum"] + 128 * c["TCC_EA0_RDREQ_128B_sum"]

        def write_b(c):
            return 32 * (c["TCC_EA0_WRREQ_sum"] - c["TCC_EA0_WRREQ_64B_sum"]) + 64 * c["TCC_EA0_WRREQ_64B_sum"]

        cr, cw = case_dispatches(rd, COPY_CASE), case_dispatches(wr, COPY_CASE)
        rf, wf = COPY_BYTES / mean(cr, read_b), COPY_BYTES / mean(cw, write_b)
        print(f"calibration: the {COPY_BYTES >> 20} MiB runtime copy ({len(cr)} + {len(cw)} dispatches) reads "
              f"{mean(cr, read_b):.0f} B and writes {mean(cw, write_b):.0f} B by these counters: read factor "
              f"{rf:.4f}, write factor {wf:.4f}")
        print()
        print(f"{'case':26s} {'kernel':38s} {'read B':>12s} {'write B':>12s} {'traffic B':>12s} "
              f"{'algorithmic B':>13s} {'ratio':>6s}")
        for case in TRAFFIC_CASES:
            r, w = case_dispatches(rd, case), case_dispatches(wr, case)
            if not r or not w:
                continue
            rb, wb = mean(r, read_b) * rf, mean(w, write_b) * wf
            alg = cases_bytes[case]
            print(f"{case:26s} {CASE_KERNEL[case].replace(' ', ''):38s} {rb:12.0f} {wb:12.0f} {rb + wb:12.0f} "
                  f"{alg:13d} {(rb + wb) / alg:6.3f}")
    else:
        sq = read_dispatches(dirs[0])
        print(f"{'case':26s} {'VALU':>9s} {'per wave':>9s} {'SALU':>9s} {'LDS':>9s} {'VMEM':>8s} {'waves':>7s} "
              f"{'floor us':>9s} {'dispatches':>10s}")
        # The three sampling cases share a kernel and run in this order, one
        # after another, with the same number of dispatches each.
        ds = case_dispatches(sq, "sampling_gumbel")
        names = ["sampling_256x151936", "sampling_greedy", "sampling_gumbel"]
        per = len(ds) // len(names)
        for k, case in enumerate(names):
            part = ds[k * per:(k + 1) * per]
            if not part:
                continue
            valu, waves = mean(part, lambda c: c["SQ_INSTS_VALU"]), mean(part, lambda c: c["SQ_WAVES"])
            floor = valu / (256 * SCLK_GHZ * 1e3)
            print(f"{case:26s} {valu:9.0f} {valu / waves:9.0f} {mean(part, lambda c: c['SQ_INSTS_SALU']):9.0f} "
                  f"{mean(part, lambda c: c['SQ_INSTS_LDS']):9.0f} {mean(part, lambda c: c['SQ_INSTS_VMEM']):8.0f} "
                  f"{waves:7.0f} {floor:9.2f} {len(part):10d}")


def traffic_case_bytes():
    """Algorithmic bytes per launch of the traffic cases (the same figures the
    kernel table uses; no device needed)."""
    T = 8192
    distinct = len(np.unique(np.random.default_rng(T).integers(0, MAX_POS, T)))
    return {COPY_CASE: 2 * COPY_BYTES, "silu_8192x6144": bytes_silu(T, I), "add_rms_8192x1024": bytes_add_rms(T, H),
            "qkv_rope_8192": bytes_qkv_rope(T, distinct), "embedding_16384": bytes_embedding(16384, H),
            "kv_write_16384": bytes_kv_write(16384), "attention_decode_64x4096": bytes_attention(64, MAX_POS, MAX_POS // BS),
            "sampling_gumbel": bytes_sampling(256, V)}


def run_kernel_case(gpu, hip, launches, rounds):
    """Average launch time (ms) over `rounds` passes through the rotating sets."""
    graph = gpu.capture(lambda: [f() for f in launches])
    per_pass_ms = time_graph(gpu, hip, graph, rounds, 2)
    return per_pass_ms / len(launches)


# -------------------------------------------------------------- CPU leg ----
def decode_steps(sequences: int) -> dict | None:
    """The serving step of the Qwen3 forward runner (nano-vllm-rs_amd/decode_bench,
    C++): 1024 prompt tokens in one prefill, then 127 decode steps of
    `sequences` rows replayed as one HIP graph each, eager launches timed too.
    Runs as a child process (its own HIP context); None when not built."""
    exe = os.path.join(ROOT, "nano-vllm-rs_amd", "decode_bench")
    if not os.path.exists(exe):
        return None
    done = subprocess.run([exe, str(sequences), "127"], capture_output=True, text=True, timeout=300)
    if done.returncode != 0:
        raise RuntimeError(f"decode_bench failed: {done.stderr.strip()}")
    return json.loads(done.stdout)


def cpu_threads() -> tuple[int, int, int]:
    """(threads used, hardware concurrency, CPUs in this process's affinity mask).
    The leg uses every CPU of the affinity mask, capped at the job's CPU share
    when the environment states one (OMP_NUM_THREADS: the GPU hosts allot 16
    host CPUs to a one-GPU job whatever the mask shows)."""
    hw = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = hw
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return (min(affinity, share) if share > 0 else affinity), hw, affinity


def cpu_baseline(tokens: int, layers: int, runs: int = 5) -> dict:
    """The oracle's multithreaded C restatement of the same step: all layers at
    the step's token count, every layer with its own inputs (distinct buffers,
    so no layer reads bytes another layer left in a cache), one contiguous row
    range per thread. Median of `runs` timed steps after one warm-up layer."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as ora

    threads, hw, affinity = cpu_threads()
    T = tokens
    tok = np.random.default_rng(0).integers(0, V, T).astype(np.int32)
    table = ora.normal_bf16((V, H), 1, 0.0, 0.02)
    pools = dict(attn=ora.normal_bf16((T, H), 2), mlp=ora.normal_bf16((T, H), 3),
                 qkv=ora.normal_bf16((T, HEADS, D), 4), gu=ora.normal_bf16((T, 2, I), 5, 0.0, 2.0))
    # Layer l's inputs: the pools rotated by l rows, each layer its own copy.
    per_layer = [{k: np.ascontiguousarray(np.roll(v, l * 97, axis=0)) for k, v in pools.items()}
                 for l in range(layers)]
    wn = ora.normal_bf16(H, 6, 1.0, 0.02)
    qn, kn = ora.normal_bf16(D, 7, 1.0, 0.02), ora.normal_bf16(D, 8, 1.0, 0.02)
    pos = (np.arange(T) % MAX_POS).astype(np.int32)
    blocks = -(-T // BS)
    slots = np.arange(T, dtype=np.int32)
    rope = ora.rope_cache(MAX_POS, D, THETA, threads)
    caches = [(np.zeros((blocks, BS, KVH, D), np.uint16), np.zeros((blocks, BS, KVH, D), np.uint16))
              for _ in range(layers)]
    lib = ora.lib()
    res = np.empty((T, H), np.uint16)
    normed = np.empty((T, H), np.uint16)
    query = np.empty((T, QH, D), np.uint16)
    act = np.empty((T, I), np.uint16)
    p = lambda a: a.ctypes.data  # noqa: E731

    def step(nlayers):
        lib.ora_embedding(p(tok), p(table), p(res), T, H, V, threads)
        for i in range(nlayers):
            x, (kc, vc) = per_layer[i], caches[i]
            if i == 0:
                lib.ora_rms(p(res), p(wn), p(normed), T, H, EPS, threads)
            else:
                lib.ora_add_rms(p(per_layer[i - 1]["mlp"]), p(res), p(wn), p(normed), T, H, EPS, threads)
            lib.ora_qkv_rope(p(x["qkv"]), p(qn), p(kn), p(pos), p(slots), p(query), p(kc), p(vc), T, QH, KVH, D, BS,
                             blocks, EPS, 1.0, p(rope), MAX_POS, threads)
            lib.ora_add_rms(p(x["attn"]), p(res), p(wn), p(normed), T, H, EPS, threads)
            lib.ora_silu(p(x["gu"]), p(act), T, I, threads)
        lib.ora_add_rms(p(per_layer[nlayers - 1]["mlp"]), p(res), p(wn), p(normed), T, H, EPS, threads)

    step(1)  # warm-up
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        step(layers)
        times.append(time.perf_counter() - t0)
    sec = float(np.median(times))
    # Algorithmic bytes of the step, counted as for the GPU chain.
    nbytes = (bytes_embedding(T, H) + bytes_rms(T, H) + 2 * layers * bytes_add_rms(T, H)
              + layers * bytes_qkv_rope(T, len(np.unique(pos))) + layers * bytes_silu(T, I))
    return {"value": T / sec, "unit": "tokens/s", "GB/s": round(nbytes / sec / 1e9, 2), "cores": threads,
            "hardware_concurrency": hw, "affinity_cpus": affinity, "kind": "port",
            "sample": f"oracle C restatement, full step ({layers} layers, T={T}, distinct per-layer inputs), "
                      f"{threads} threads, median of {len(times)} runs = {sec * 1e3:.1f} ms/step"}


# ------------------------------------------------------------------ main ---
def warm_up(gpu, hip, seconds, graph=None):
    """Sustained load before anything is timed: the GPU's clocks settle over
    the first ~0.1-1 s of work, and launches timed earlier run up to ~8% slow.
    Replays `graph` (the step), or 512 MiB device copies when there is none
    (few dispatches, for runs under a kernel tracer)."""
    if seconds <= 0:
        return
    t0 = time.perf_counter()
    if graph is None:
        n = 512 << 20
        a, b = gpu.alloc(n), gpu.alloc(n)
        stream = gpu.stream()
        while time.perf_counter() - t0 < seconds:
            for _ in range(8):
                hip.copy_d2d(b.ptr, a.ptr, n, stream)
            gpu.sync()
        return
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            graph.replay()
        gpu.sync()


# ---------------------------------------------------- kernel-time child ----
TRACE_NOTE = "rocprofv3 --kernel-trace of a child run of this script over the same kernel cases (median duration)"


def trace_child(out_dir, rounds, only) -> int:
    """Child mode (under rocprofv3 --kernel-trace): the kernel cases only, in
    order, after a copy warm-up; writes the case list with its dispatch counts
    to out_dir/cases.json so the parent can assign the trace's dispatches."""
    hip = Hip()
    gpu = nvr.Gpu(0)
    fill = Filler(gpu, hip)
    chain = Chain(gpu, fill, 8192, 1)
    cases = kernel_cases(gpu, hip, fill, chain, only)
    gpu.sync()
    warm_up(gpu, hip, 1.0)
    order = []
    for name, _, launches, _, _ in cases:
        run_kernel_case(gpu, hip, launches, rounds)
        order.append({"case": name, "launches": len(launches), "warm": 2, "rounds": rounds})
    gpu.sync()
    with open(os.path.join(out_dir, "cases.json"), "w") as f:
        json.dump(order, f)
    return 0


def assign_dispatches(order, disp) -> tuple[dict, str]:
    """Splits the traced dispatches (start ns, duration us, kernel name), set-up
    kernels removed, over the cases in the order the child ran them: each case
    is (warm + rounds) x launches consecutive dispatches of one kernel, and its
    figure is the median of the timed ones."""
    import statistics

    disp = sorted(disp)
    result, i = {}, 0
    for c in order:
        n = (c["warm"] + c["rounds"]) * c["launches"]
        group = disp[i:i + n]
        i += n
        names = {g[2] for g in group}
        if len(group) != n or len(names) != 1:
            return {}, f"kernel trace does not line up with the cases at {c['case']}"
        timed = [g[1] for g in group[c["warm"] * c["launches"]:]]
        short = next(iter(names)).replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]
        result[c["case"]] = (short, statistics.median(timed), len(timed))
    if i != len(disp):
        return {}, f"kernel trace has {len(disp) - i} dispatches past the last case"
    return result, "ok"


def under_profiler(env=None) -> bool:
    """True when this process runs under rocprofv3 (its tool library is
    preloaded, or its ROCPROF_* settings are in the environment)."""
    env = os.environ if env is None else env
    return "rocprofiler" in env.get("LD_PRELOAD", "") or any(k.startswith("ROCPROF") for k in env)


def kernel_times(rounds, only, timeout_s=420) -> tuple[dict, str]:
    """{case: (kernel name, median kernel us, timed dispatches)} from a child
    run of this script under rocprofv3 --kernel-trace, and a status note.
    Runs before this process touches the GPU; empty when rocprofv3 is absent
    or the child fails (the line then carries event times only)."""
    import csv
    import glob
    import shutil
    import tempfile

    if under_profiler():
        # The tracer's launcher replaces itself with its target program; under
        # an outer profiler's preloaded library that process has already
        # initialised the GPU, and such an exec must not happen.
        return {}, "not run (this process runs under a profiler)"
    prof = shutil.which("rocprofv3") or ("/opt/rocm/bin/rocprofv3" if os.path.exists("/opt/rocm/bin/rocprofv3")
                                         else None)
    if prof is None:
        return {}, "rocprofv3 not found"
    out = tempfile.mkdtemp(prefix="nvr_trace_")
    try:
        cmd = [prof, "--kernel-trace", "-f", "csv", "-d", out, "-o", "kt", "--", sys.executable,
               os.path.abspath(__file__), "--trace-child", out, "--kernel-rounds", str(rounds)]
        if only:
            cmd += ["--only", ",".join(only)]
        done = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout_s, cwd=out,
                              env=dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp")))
        cases_path = os.path.join(out, "cases.json")
        if not os.path.exists(cases_path):
            return {}, f"kernel-trace child failed (status {done.returncode}): {done.stderr.strip()[-300:]}"
        order = json.load(open(cases_path))
        disp = []
        for path in glob.glob(os.path.join(out, "**", "*kernel_trace.csv"), recursive=True):
            with open(path, newline="") as f:
                for rec in csv.DictReader(f):
                    name = rec["Kernel_Name"]
                    if name.startswith("__amd_rocclr") or "rope_table" in name:
                        continue  # set-up copies and the RoPE table, before any case runs
                    start, end = int(rec["Start_Timestamp"]), int(rec["End_Timestamp"])
                    disp.append((start, (end - start) / 1e3, name))
        return assign_dispatches(order, disp)
    except subprocess.TimeoutExpired:
        return {}, f"kernel-trace child exceeded {timeout_s} s"
    finally:
        shutil.rmtree(out, ignore_errors=True)


def add_copy_ceilings(kernels):
    """Each streaming kernel's rate as a fraction of the copy case of about its
    own traffic (COPY_CEILING), by kernel time where both were traced, else by
    event time; cases without their copy case get no field."""
    for name, cname in COPY_CEILING.items():
        if name in kernels and cname in kernels:
            k, c = kernels[name], kernels[cname]
            key = "kernel_us" if "kernel_us" in k and "kernel_us" in c else "us"
            gbs, cgbs = k["bytes"] / k[key] / 1e3, c["bytes"] / c[key] / 1e3
            k["copy_ceiling"] = {"case": cname, "GB/s": round(cgbs, 1), "frac": round(gbs / cgbs, 4),
                                 "time": key}


def fold_layouts(kernels):
    """Moves the slot-layout cases ("<case>@<layout>") under their case and
    adds the min and median over all layouts (the case's own included)."""
    for name in [k for k in kernels if "@" in k]:
        base, tag = name.split("@", 1)
        entry = kernels.pop(name)
        if base in kernels:
            kernels[base].setdefault("layouts", {})[tag] = {k: entry[k] for k in ("us", "frac", "kernel_us", "kernel_frac")
                                                            if k in entry}
    for base, entry in kernels.items():
        if "layouts" not in entry:
            continue
        rows = [entry] + list(entry["layouts"].values())
        summary = {"layouts": len(rows), "default": entry.get("slot_layout", "")}
        for key in ("frac", "kernel_frac"):
            vals = [r[key] for r in rows if key in r]
            if len(vals) == len(rows):
                summary[f"{key}_min"] = round(min(vals), 4)
                summary[f"{key}_median"] = round(float(np.median(vals)), 4)
        entry["layout_sweep"] = summary


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--warm-seconds", type=float, default=1.5,
                    help="sustained replays of the step before anything is timed (clocks settle)")
    ap.add_argument("--tokens", type=int, default=8192)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-kernels", action="store_true", help="skip the per-kernel table")
    ap.add_argument("--no-decode", action="store_true", help="skip the forward runner's decode-step lines")
    ap.add_argument("--no-kernel-trace", action="store_true",
                    help="skip the child run under rocprofv3 that gives each case's kernel duration")
    ap.add_argument("--kernel-rounds", type=int, default=5)
    ap.add_argument("--only", default="", help="comma-separated kernel cases to run (implies --no-cpu, skips the step)")
    ap.add_argument("--trace-child", metavar="DIR", help=argparse.SUPPRESS)
    ap.add_argument("--pmc-summary", nargs="+", metavar=("KIND", "DIR"),
                    help="print the table of rocprofv3 counter runs instead of measuring: 'traffic READ_DIR WRITE_DIR' "
                         f"(passes of {' '.join(READ_COUNTERS)} and of {' '.join(WRITE_COUNTERS)}) or 'valu SQ_DIR' "
                         f"(a pass of {' '.join(VALU_COUNTERS)})")
    args = ap.parse_args()
    only = [k for k in args.only.split(",") if k]
    if args.trace_child:
        return trace_child(args.trace_child, args.kernel_rounds, only)
    if args.pmc_summary:
        kind, dirs = args.pmc_summary[0], args.pmc_summary[1:]
        if (kind, len(dirs)) not in (("traffic", 2), ("valu", 1)):
            ap.error("--pmc-summary takes 'traffic READ_DIR WRITE_DIR' or 'valu SQ_DIR'")
        pmc_summary(kind, dirs, traffic_case_bytes())
        return 0
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: --gpus {args.gpus} is not supported "
              "(the kernels are per-token; a data-parallel split needs no collectives).", file=sys.stderr)
        return 2

    # Child processes first, before this process touches the GPU: the
    # runner's decode steps, then the kernel cases under the kernel tracer.
    decode = None
    if not args.no_decode and not only:
        decode = {f"{n}_sequences": decode_steps(n) for n in (8, 32)}
    traced, trace_status = {}, "not run"
    if not args.no_kernels and not args.no_kernel_trace:
        traced, trace_status = kernel_times(args.kernel_rounds, only)

    hip = Hip()
    gpu = nvr.Gpu(0)
    fill = Filler(gpu, hip)
    chain = Chain(gpu, fill, args.tokens, 1 if only else LAYERS)
    gpu.sync()
    ms = float("nan")
    if not only:
        graph = gpu.capture(chain.step)
        warm_up(gpu, hip, args.warm_seconds, graph)
        ms = time_graph(gpu, hip, graph, args.steps, args.warmup)
    else:
        warm_up(gpu, hip, args.warm_seconds)
    tokens_per_s = args.tokens / (ms / 1e3)
    chain_gbs = chain.bytes() / (ms / 1e3) / 1e9

    kernels = {}
    if not args.no_kernels:
        cases = kernel_cases(gpu, hip, fill, chain, only)
        # The calibration copy runs last (its dispatches are told from the
        # set-up's copies by their place; see case_dispatches).
        cases.sort(key=lambda c: c[0] == COPY_CASE)
        for name, workload, launches, nbytes, rows in cases:
            t = run_kernel_case(gpu, hip, launches, args.kernel_rounds)
            gbs = nbytes / (t / 1e3) / 1e9
            kernels[name] = {"workload": workload, "us": round(t * 1e3, 3), "bytes": nbytes, "GB/s": round(gbs, 1),
                             "frac": round(gbs / HBM_PEAK_GBS, 4), "rows_per_s": round(rows / (t / 1e3), 1),
                             "launches": len(launches)}
            if name in traced:
                kname, kus, n = traced[name]
                kernels[name].update({"kernel": kname, "kernel_us": round(kus, 3),
                                      "kernel_frac": round(nbytes / (kus * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                      "kernel_dispatches": n})
            traffic = measured_traffic(name)
            if traffic is not None:
                kernels[name]["traffic"] = {"bytes": traffic, "ratio": round(traffic / nbytes, 3),
                                            "source": TRAFFIC_SUMMARY}
            valu = measured_valu(name)
            if valu is not None:
                # VALU roofline: one wave64 VALU instruction per CU per cycle.
                floor_us = valu / (gpu.sm_count() * SCLK_GHZ * 1e3)
                kernels[name]["valu"] = {"insts": valu, "floor_us": round(floor_us, 2),
                                         "frac": round(floor_us / (t * 1e3), 4), "source": VALU_SUMMARY}
        for name, tag in (("qkv_rope_8192", "perm of 32 blocks, seed 8192"), ("kv_write_16384", "perm of 128 blocks, seed 7")):
            if name in kernels:
                kernels[name]["slot_layout"] = tag
        add_copy_ceilings(kernels)
        fold_layouts(kernels)

    # Dominant kernel of the step: the largest share of the step's HBM bytes
    # (launches x algorithmic bytes at the step's shape). By time, SiLU and
    # qkv_rope tie within run-to-run noise; by bytes SiLU leads (4.23 GB of
    # 11.9 GB per step), so the choice is stable.
    roofline = None
    shape_of = {"add_rms": "add_rms_8192x1024", "qkv_rope_cached": "qkv_rope_8192", "silu": "silu_8192x6144"}
    share = {k: chain.launches()[k] * kernels[v]["bytes"] for k, v in shape_of.items() if v in kernels}
    if share:
        dom = max(share, key=share.get)
        kd = kernels[shape_of[dom]]
        roofline = {"kernel": shape_of[dom], "bound": "hbm", "achieved": kd["GB/s"], "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": kd["frac"], "traffic": measured_traffic(shape_of[dom]),
                    "traffic_source": TRAFFIC_SUMMARY}
        if "kernel_us" in kd:
            roofline.update({"kernel_us": kd["kernel_us"], "kernel_frac": kd["kernel_frac"]})

    cpu = None
    if not args.no_cpu and not only:
        cpu = cpu_baseline(args.tokens, LAYERS)

    line = {
        "metric": METRIC, "value": round(tokens_per_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "Qwen3-0.6B fused per-layer kernel chain: embedding + 28 x [add-RMSNorm, q/k-norm + "
                               "RoPE + paged KV write, add-RMSNorm, SiLU-mul] + final add-RMSNorm, one HIP graph",
                   "tokens": args.tokens, "layers": LAYERS, "hidden": H, "intermediate": I, "q_heads": QH,
                   "kv_heads": KVH, "head_dim": D, "block_size": BS, "parallelism": "none (1 GPU)"},
        "warm_seconds": args.warm_seconds,
        # Algorithmic bytes over step time. The residual stream and the
        # per-layer activations the chain rewrites stay in the 256 MB Infinity
        # Cache between kernels, so this is an effective rate, not HBM traffic.
        "step_effective_GB/s": round(chain_gbs, 1), "step_effective_frac": round(chain_gbs / HBM_PEAK_GBS, 4),
        "roofline": roofline, "kernel_time_source": TRACE_NOTE if traced else trace_status,
        "cpu_baseline": cpu, "kernels": kernels, "decode": decode,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
