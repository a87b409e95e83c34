"""The reference's own GPU tests (src/gpu.rs:1148-1472), restated over this
library through the Python host API (nvr.Gpu has the reference host's object
and method names), plus graph capture/replay of the fused kernels.

"""
import math

import numpy as np
import pytest

import nvr
import oracle as ora
from helpers import bf16_of, f32_of

pytestmark = pytest.mark.gpu


def values(buf, count):
    return f32_of(buf.download(np.uint16, count)).tolist()


def test_gpu_views_keep_allocations_and_reject_overlap():
    """src/gpu.rs:1169-1192."""
    gpu = nvr.Gpu(0)
    packed = gpu.alloc(32)
    packed.upload(np.array([1, 3, 0, 0, 5, 6, 7, 8], np.int32))
    tokens = packed.slice(0, 8)
    adjacent = packed.slice(8, 8)
    assert not tokens.overlaps(adjacent) and tokens.overlaps(packed.slice(4, 8))
    with pytest.raises(nvr.ArgumentError):
        tokens.slice(4, 8)
    weights = gpu.alloc(8)
    weights.upload(bf16_of([1.0, 2.0, 3.0, 4.0]))
    out = gpu.alloc(4)
    with pytest.raises(nvr.ArgumentError, match="alignment"):  # a misaligned i32 view
        gpu.embedding(packed.slice(1, 8), weights, out, 2, 1, 4)
    with pytest.raises(nvr.ArgumentError, match="overlap"):  # the output is part of an input
        gpu.embedding(tokens, weights, weights.slice(0, 4), 2, 1, 4)
    graph = gpu.capture(lambda: gpu.embedding(tokens, weights, out, 2, 1, 4))
    del tokens, adjacent, packed
    graph.replay()
    assert values(out, 2) == [2.0, 4.0]


def test_gpu_parallel_sampler_matches_serial_for_tail_ties_and_temperature():
    """src/gpu.rs:1194-1244."""
    gpu = nvr.Gpu(0)
    batch, vocab = 3, 151936
    idx = np.arange(batch * vocab)
    scores = ((idx * 31 % 101) - 50.0) * 0.125
    scores[[2047, 2048, 4096]] = 100.0
    logits = gpu.upload_array(bf16_of(scores))
    temps = gpu.upload_array(np.array([0.0, 0.6, 1.0], np.float32))
    seeds = gpu.upload_array(np.array([42, 43, 44], np.uint64))
    serial, parallel = gpu.alloc(batch * 4), gpu.alloc(batch * 4)
    parts = -(-vocab // 2048)
    ps, pi = gpu.alloc(batch * parts * 4), gpu.alloc(batch * parts * 4)
    gpu.sample(logits, temps, seeds, serial, batch, vocab)
    gpu.sample_parallel(logits, temps, seeds, parallel, ps, pi, batch, vocab)
    expected = serial.download(np.int32, batch)
    assert expected[0] == 2047
    assert parallel.download(np.int32, batch).tolist() == expected.tolist()
    # The oracle agrees, including the Gumbel rows.
    want = ora.sample(bf16_of(scores).reshape(batch, vocab), np.array([0.0, 0.6, 1.0], np.float32),
                      np.array([42, 43, 44], np.uint64), batch, vocab)
    assert expected.tolist() == want.tolist()
    parallel.upload(np.zeros(batch, np.int32))
    graph = gpu.capture(lambda: gpu.sample_parallel(logits, temps, seeds, parallel, ps, pi, batch, vocab))
    for _ in range(3):
        graph.replay()
        assert parallel.download(np.int32, batch).tolist() == expected.tolist()
        parallel.upload(np.zeros(batch, np.int32))


def test_gpu_cached_rope_matches_direct_at_context_boundary():
    """src/gpu.rs:1246-1289: cached and direct RoPE agree byte for byte."""
    gpu = nvr.Gpu(0)
    rows, qh, kvh, dim = 4, 4, 2, 128
    idx = np.arange(rows * (qh + kvh * 2) * dim)
    packed = gpu.upload_array(bf16_of(((idx * 17 % 37) - 18.0) / 8.0))
    norm = gpu.upload_array(bf16_of(np.ones(dim)))
    positions = gpu.upload_array(np.array([0, 1, 350, 4095], np.int32))
    slots = gpu.upload_array(np.array([0, 1, 2, 3], np.int32))
    direct = [gpu.alloc(n) for n in (rows * qh * dim * 2, 4 * kvh * dim * 2, 4 * kvh * dim * 2)]
    cached = [gpu.alloc(n) for n in (rows * qh * dim * 2, 4 * kvh * dim * 2, 4 * kvh * dim * 2)]
    cache = gpu.alloc(4096 * dim * 4)
    gpu.rope_cache(cache, 4096, dim, 1e6)
    gpu.qkv_rope(packed, norm, norm, positions, slots, *direct, rows, qh, kvh, dim, 4, 1, 1e-6, 1e6)
    gpu.qkv_rope_cached(packed, norm, norm, positions, slots, *cached, rows, qh, kvh, dim, 4, 1, 1e-6, cache, 4096)
    for d, c in zip(direct, cached):
        assert d.download_bytes() == c.download_bytes()


def test_gpu_gemm_rms_sampling_graph():
    """src/gpu.rs:1290-1329."""
    gpu = nvr.Gpu(0)
    x = gpu.alloc(12)
    x.upload(bf16_of([1, 2, 3, 4, 5, 6]))
    w = gpu.alloc(12)
    w.upload(bf16_of([1, 0, 1, 0, 1, 0]))
    y = gpu.alloc(8)
    gpu.gemm(x, w, y, 2, 2, 3)
    assert values(y, 4) == [4.0, 2.0, 10.0, 5.0]
    with pytest.raises(ValueError):
        gpu.gemm(x, w, y, 3, 2, 3)
    with pytest.raises(ValueError):
        gpu.gemm(x, w, x, 2, 2, 3)
    normw = gpu.alloc(4)
    normw.upload(bf16_of([1.0, 1.0]))
    normalized = gpu.alloc(8)
    gpu.rms_norm(y, normw, normalized, 2, 2, 1e-6)
    assert abs(values(normalized, 4)[0] - 1.264911) < 0.008
    temps = gpu.alloc(8)
    temps.upload(np.array([0.0, 0.0], np.float32))
    seeds = gpu.alloc(16)
    seeds.upload(np.array([42, 43], np.uint64))
    output = gpu.alloc(8)
    gpu.sample(y, temps, seeds, output, 2, 2)
    assert output.download(np.int32, 2).tolist() == [0, 0]
    gpu.sync()
    graph = gpu.capture(lambda: gpu.gemm(x, w, y, 2, 2, 3))
    x.upload(bf16_of([2, 4, 6, 8, 10, 12]))
    graph.replay()
    assert values(y, 4) == [8.0, 4.0, 20.0, 10.0]
    del x, w
    graph.replay()
    gpu.sync()
    with pytest.raises(nvr.BackendError, match="allocation"):
        gpu.capture(lambda: gpu.alloc(4))
    gpu.sync()


def test_gpu_rope_known_answers_and_v_slot_write():
    """Second half of src/gpu.rs:1330-1380 (the RoPE and V-cache part)."""
    gpu = nvr.Gpu(0)
    rows, dim, qh, kvh = 3, 32, 2, 1
    q = gpu.alloc(rows * qh * dim * 2)
    k = gpu.alloc(2 * 2 * kvh * dim * 2)
    v = gpu.alloc(2 * 2 * kvh * dim * 2)
    positions = gpu.upload_array(np.array([0, 1, 2], np.int32))
    packed = gpu.upload_array(bf16_of(np.ones(rows * (qh + 2 * kvh) * dim)))
    weight = gpu.upload_array(bf16_of(np.ones(dim)))
    slots = gpu.upload_array(np.array([2, 3, 0], np.int32))
    gpu.qkv_rope(packed, weight, weight, positions, slots, q, k, v, rows, qh, kvh, dim, 2, 2, 1e-6, 1000000.0)
    actualq = values(q, rows * qh * dim)
    assert all(abs(t - 1.0) < 0.01 for t in actualq[: qh * dim])
    assert abs(actualq[qh * dim] - (math.cos(1.0) - math.sin(1.0))) < 0.008
    assert values(v, 4 * dim)[0] == 1.0


def test_gpu_causal_paged_attention_known_answer():
    """First half of src/gpu.rs:1330-1380: zero queries over reversed physical
    blocks holding V rows 1, 2, 3 give the running means 1, 1.5, 2."""
    gpu = nvr.Gpu(0)
    rows, dim, qh, kvh = 3, 32, 2, 1
    q = gpu.alloc(rows * qh * dim * 2)
    k = gpu.alloc(2 * 2 * kvh * dim * 2)
    cache = np.zeros(4 * dim, np.float32)
    cache[2 * dim:3 * dim] = 1.0
    cache[3 * dim:4 * dim] = 2.0
    cache[:dim] = 3.0
    v = gpu.upload_array(bf16_of(cache))
    positions = gpu.upload_array(np.array([0, 1, 2], np.int32))
    seqs = gpu.upload_array(np.array([0, 0, 0], np.int32))
    tables = gpu.upload_array(np.array([1, 0], np.int32))
    out = gpu.alloc(rows * qh * dim * 2)
    gpu.paged_attention(q, k, v, positions, seqs, tables, out, rows, qh, kvh, dim, 2, 2, 2, 1, 4)
    actual = values(out, rows * qh * dim)
    for r in range(rows):
        assert actual[r * qh * dim:(r + 1) * qh * dim] == [1.0 + 0.5 * r] * (qh * dim)


@pytest.mark.parametrize("dim,block_size,pos,seq,table", [
    (32, 2, [0, 2, 1, 0], [0, 0, 1, 2], [3, 1, 0, 2, 2, -1]),
    (128, 256, [0, 255, 256, 510], [0, 0, 1, 1], [3, 1, 0, 2]),
])
def test_gpu_ragged_gqa_matches_cpu(dim, block_size, pos, seq, table):
    """src/gpu.rs:1382-1470: ragged GQA rows against the reference test's own
    f32 formula (tolerance 0.004), and bit for bit against the oracle."""
    gpu = nvr.Gpu(0)
    rows, qheads, kvheads, blocks = 4, 4, 2, 4
    query = ((np.arange(rows * qheads * dim) * 7 % 19) - 9.0) * 0.125
    key = ((np.arange(blocks * block_size * kvheads * dim) * 11 % 23) - 11.0) * 0.125
    value = ((np.arange(key.size) * 3 % 13) - 6.0) * 0.125
    qb, kb, vb = bf16_of(query), bf16_of(key), bf16_of(value)
    pos_a, seq_a, table_a = (np.array(x, np.int32) for x in (pos, seq, table))
    out = gpu.alloc(qb.nbytes)
    gpu.paged_attention(gpu.upload_array(qb), gpu.upload_array(kb), gpu.upload_array(vb), gpu.upload_array(pos_a),
                        gpu.upload_array(seq_a), gpu.upload_array(table_a), out, rows, qheads, kvheads, dim,
                        block_size, blocks, 2, len(table) // 2, max(pos) + 1)
    got = out.download(np.uint16, qb.size)
    actual = f32_of(got)
    q32, k32, v32 = query.astype(np.float32), key.astype(np.float32), value.astype(np.float32)
    for row in range(rows):
        context = pos[row] + 1
        for head in range(qheads):
            kvhead = head // (qheads // kvheads)
            qbase = (row * qheads + head) * dim

            def base(t):
                return ((table[seq[row] * 2 + t // block_size] * block_size + t % block_size) * kvheads
                        + kvhead) * dim

            scores = np.array([np.sum(q32[qbase:qbase + dim] * k32[base(t):base(t) + dim], dtype=np.float32)
                               / np.float32(math.sqrt(dim)) for t in range(context)], np.float32)
            probs = np.exp(scores - scores.max()).astype(np.float32)
            total = probs.sum(dtype=np.float32)
            for d in range(dim):
                expected = sum(float(probs[t]) * float(v32[base(t) + d]) for t in range(context)) / float(total)
                assert abs(actual[qbase + d] - expected) < 0.004, (row, head, d)
    want = ora.attention(qb, kb, vb, pos_a, seq_a, table_a, rows, qheads, kvheads, dim, block_size, blocks, 2,
                         len(table) // 2, max(pos) + 1)
    assert np.array_equal(got, want.reshape(-1))


def test_gpu_attention_rejects_unsupported_arguments():
    gpu = nvr.Gpu(0)
    lib, h = gpu.lib, gpu.handle
    assert lib.nv_attention(h, *([None] * 7), 1, 2, 1, 32, 2, 2, 2, 1, 4097) == -2
    assert b"max_context" in lib.nv_last_error()
    assert lib.nv_attention(h, *([None] * 7), 1, 3, 2, 32, 2, 2, 2, 1, 4) == -2
    assert lib.nv_attention(h, *([None] * 7), 1, 2, 1, 33, 2, 2, 2, 1, 4) == -2
    assert lib.nv_attention(h, *([None] * 7), 0, 2, 1, 32, 2, 2, 2, 1, 4) == -2
    with pytest.raises(ValueError):
        gpu.paged_attention(*([gpu.alloc(64)] * 7), 1, 2, 1, 32, 2, 2, 2, 1, 4097)


def test_gpu_alloc_is_zero_filled_and_errors_carry_messages():
    gpu = nvr.Gpu(0)
    buf = gpu.alloc(1 << 20)
    assert not buf.download(np.uint8, 1 << 20).any()
    free, total = gpu.mem_info()
    assert 0 < free <= total
    assert gpu.sm_count() > 0
    with pytest.raises(nvr.BackendError, match="status -2"):
        nvr.check_status(gpu.lib.nv_silu(gpu.handle, None, None, 0, 8))


def test_gpu_forward_chain_graph_replays_match_eager():
    """One layer's fused kernels captured as a graph; every replay, with eager
    work and host syncs in between, reproduces the eager result."""
    gpu = nvr.Gpu(0)
    T, H, I, qh, kvh, D, bs = 512, 1024, 3072, 16, 8, 128, 256
    blocks = T // bs
    heads = qh + 2 * kvh
    hidden = ora.normal_bf16((T, H), 200)
    res0 = ora.normal_bf16((T, H), 201)
    wn = ora.normal_bf16(H, 202, 1.0, 0.02)
    qkv = ora.normal_bf16((T, heads, D), 203)
    qw = ora.normal_bf16(D, 204, 1.0, 0.02)
    kw = ora.normal_bf16(D, 205, 1.0, 0.02)
    gu = ora.normal_bf16((T, 2, I), 206, 0.0, 2.0)
    pos = np.arange(T, dtype=np.int32)
    slots = np.arange(T, dtype=np.int32)
    b = {name: gpu.upload_array(a) for name, a in dict(hidden=hidden, wn=wn, qkv=qkv, qw=qw, kw=kw, gu=gu, pos=pos,
                                                        slots=slots).items()}
    res = gpu.upload_array(res0)
    normed = gpu.alloc(T * H * 2)
    qout = gpu.alloc(T * qh * D * 2)
    kc, vc = gpu.alloc(blocks * bs * kvh * D * 2), gpu.alloc(blocks * bs * kvh * D * 2)
    act = gpu.alloc(T * I * 2)
    table = gpu.alloc(4096 * D * 4)
    gpu.rope_cache(table, 4096, D, 1e6)

    def layer():
        gpu.add_rms_norm(b["hidden"], res, b["wn"], normed, T, H, 1e-6)
        gpu.qkv_rope_cached(b["qkv"], b["qw"], b["kw"], b["pos"], b["slots"], qout, kc, vc, T, qh, kvh, D, bs, blocks,
                            1e-6, table, 4096)
        gpu.silu_mul(b["gu"], act, T, I)

    def snapshot():
        return [x.download_bytes() for x in (res, normed, qout, kc, vc, act)]

    def reset():
        res.upload(res0)
        for x in (normed, qout, kc, vc, act):
            x.upload(np.zeros(x.bytes, np.uint8))

    layer()
    eager = snapshot()
    reset()
    graph = gpu.capture(layer)
    for _ in range(3):
        graph.replay()
        gpu.sync()
        assert snapshot() == eager
        reset()
        gpu.silu_mul(b["gu"], act, T, I)  # unrelated eager work between replays
        gpu.sync()
        reset()
