"""HIP kernels vs the CPU oracle, through the nv_* C ABI.

Seeded synthetic inputs at the workload shapes (Qwen3-0.6B: hidden 1024,
intermediate 3072, 16 q heads, 8 kv heads, head dim 128, vocab 151936) plus
ragged/misaligned/out-of-range edge cases. Bars:
  - copies, indices, residuals, q/k norm + RoPE, RMSNorm: bit-exact
    (the kernels keep the oracle's summation order and fp32 rounding points);
  - SiLU: within 1 bf16 ulp (hardware exp/reciprocal vs the C library).
"""
import numpy as np
import pytest

import nvr
import oracle as ora
from helpers import assert_bits_equal, bf16_of, bf16_ulp_diff, f32_of, unique_slots

pytestmark = pytest.mark.gpu

EPS = 1e-6
THETA = 1e6


def up(gpu, arr):
    return gpu.upload_array(np.ascontiguousarray(arr))


def down(buf, dtype, shape):
    return buf.download(dtype, int(np.prod(shape))).reshape(shape)


def misaligned(gpu, arr):
    """Upload `arr` at a 2-byte offset so only the generic kernels apply."""
    arr = np.ascontiguousarray(arr)
    raw = gpu.alloc(arr.nbytes + 16)
    view = raw.slice(2, arr.nbytes)
    view.upload(arr)
    return view


# ------------------------------------------------------------------ norms ----
def test_rms_small_rows(gpu):
    """8 tokens x 1024 (RMSNorm-only workload)."""
    x = ora.normal_bf16((8, 1024), 0)
    w = ora.normal_bf16(1024, 1, 1.0, 0.02)
    out = gpu.alloc(8 * 1024 * 2)
    gpu.rms_norm(up(gpu, x), up(gpu, w), out, 8, 1024, EPS)
    got = down(out, np.uint16, (8, 1024))
    assert_bits_equal(got, ora.rms(x, w, 8, 1024, EPS))


def test_add_rms_8192x1024(gpu):
    rows, hidden = 8192, 1024
    x = ora.normal_bf16((rows, hidden), 2)
    res = ora.normal_bf16((rows, hidden), 3)
    w = ora.normal_bf16(hidden, 4, 1.0, 0.02)
    rb = up(gpu, res)
    out = gpu.alloc(rows * hidden * 2)
    gpu.add_rms_norm(up(gpu, x), rb, up(gpu, w), out, rows, hidden, EPS)
    want_res, want_out = ora.add_rms(x, res, w, rows, hidden, EPS, threads=8)
    assert_bits_equal(down(rb, np.uint16, (rows, hidden)), want_res)
    assert_bits_equal(down(out, np.uint16, (rows, hidden)), want_out)


@pytest.mark.parametrize("rows,hidden", [(7, 256), (33, 2048), (5, 4096), (3, 5120), (9, 1536)])
def test_rms_other_hidden_sizes(gpu, rows, hidden):
    x = ora.normal_bf16((rows, hidden), 5 + hidden)
    res = ora.normal_bf16((rows, hidden), 6 + hidden)
    w = ora.normal_bf16(hidden, 7, 1.0, 0.02)
    out = gpu.alloc(rows * hidden * 2)
    gpu.rms_norm(up(gpu, x), up(gpu, w), out, rows, hidden, EPS)
    assert_bits_equal(down(out, np.uint16, (rows, hidden)), ora.rms(x, w, rows, hidden, EPS))
    rb = up(gpu, res)
    gpu.add_rms_norm(up(gpu, x), rb, up(gpu, w), out, rows, hidden, EPS)
    want_res, want_out = ora.add_rms(x, res, w, rows, hidden, EPS)
    assert_bits_equal(down(rb, np.uint16, (rows, hidden)), want_res)
    assert_bits_equal(down(out, np.uint16, (rows, hidden)), want_out)


@pytest.mark.parametrize("hidden", [1000, 1024, 1, 3])
def test_rms_generic_path_misaligned(gpu, hidden):
    rows = 5
    x = ora.normal_bf16((rows, hidden), 8)
    res = ora.normal_bf16((rows, hidden), 9)
    w = ora.normal_bf16(hidden, 10, 1.0, 0.02)
    out = misaligned(gpu, np.zeros((rows, hidden), np.uint16))
    gpu.rms_norm(misaligned(gpu, x), misaligned(gpu, w), out, rows, hidden, EPS)
    assert_bits_equal(down(out, np.uint16, (rows, hidden)), ora.rms(x, w, rows, hidden, EPS))
    rb = misaligned(gpu, res)
    gpu.add_rms_norm(misaligned(gpu, x), rb, misaligned(gpu, w), out, rows, hidden, EPS)
    want_res, want_out = ora.add_rms(x, res, w, rows, hidden, EPS)
    assert_bits_equal(down(rb, np.uint16, (rows, hidden)), want_res)
    assert_bits_equal(down(out, np.uint16, (rows, hidden)), want_out)


@pytest.mark.parametrize("input_rows,hidden,align,picks", [
    (1024, 1024, True, "last"),     # a prefill's last tokens of 8 sequences of 128
    (8, 1024, True, "all"),         # a decode step: every row sampled
    (40, 2048, True, "ragged"),     # duplicates and indices outside the input
    (9, 1000, False, "ragged"),     # the generic path
])
def test_add_rms_gather_equals_add_rms_then_gather(gpu, input_rows, hidden, align, picks):
    """nv_add_rms_gather against the oracle's add-RMSNorm over every row followed by
    the gather; the residual is read, not written."""
    rng = np.random.default_rng(input_rows + hidden)
    if picks == "last":
        idx = np.arange(127, input_rows, 128, dtype=np.int32)
    elif picks == "all":
        idx = np.arange(input_rows, dtype=np.int32)
    else:
        idx = rng.integers(-2, input_rows + 2, 13).astype(np.int32)
        idx[[0, 5]] = idx[3]  # one row gathered three times
    rows = len(idx)
    x = ora.normal_bf16((input_rows, hidden), 11 + hidden)
    res = ora.normal_bf16((input_rows, hidden), 12 + hidden)
    w = ora.normal_bf16(hidden, 13, 1.0, 0.02)
    put = up if align else misaligned
    rb = put(gpu, res)
    out = put(gpu, np.full((rows, hidden), 0x7FC1, np.uint16))
    gpu.add_rms_norm_gather(put(gpu, x), rb, put(gpu, w), up(gpu, idx), out, rows, hidden, input_rows, EPS)
    _, full_out = ora.add_rms(x, res, w, input_rows, hidden, EPS, threads=8)
    assert_bits_equal(down(out, np.uint16, (rows, hidden)), ora.gather(full_out, idx, rows, hidden, input_rows))
    assert_bits_equal(down(rb, np.uint16, (input_rows, hidden)), res.reshape(input_rows, hidden))


# ------------------------------------------------------------------- RoPE ----
def test_rope_table_bit_exact(gpu):
    table = gpu.alloc(4096 * 128 * 4)
    gpu.rope_cache(table, 4096, 128, THETA)
    assert_bits_equal(down(table, np.float32, (4096, 128)), ora.rope_cache(4096, 128, THETA, threads=8))


def _rope_case(gpu, rows, qh, kvh, dim, bs, blocks, seed, positions, slots, cached=True, align=True):
    heads = qh + 2 * kvh
    qkv = ora.normal_bf16((rows, heads, dim), seed)
    qw = ora.normal_bf16(dim, seed + 1, 1.0, 0.02)
    kw = ora.normal_bf16(dim, seed + 2, 1.0, 0.02)
    cache0 = ora.normal_bf16((blocks, bs, kvh, dim), seed + 3)  # stale contents must survive skipped slots
    put = up if align else misaligned
    kcb, vcb = put(gpu, cache0), put(gpu, cache0)
    qout = put(gpu, np.zeros((rows, qh, dim), np.uint16))
    args = (put(gpu, qkv), put(gpu, qw), put(gpu, kw), up(gpu, positions), up(gpu, slots), qout, kcb, vcb, rows, qh,
            kvh, dim, bs, blocks, EPS)
    if cached:
        tb = gpu.alloc(4096 * dim * 4)
        gpu.rope_cache(tb, 4096, dim, THETA)
        table = down(tb, np.float32, (4096, dim))
        gpu.qkv_rope_cached(*args, tb, 4096)
        want = ora.qkv_rope(qkv, qw, kw, positions, slots, cache0, cache0, rows, qh, kvh, dim, bs, blocks, EPS,
                            table=table, max_positions=4096, threads=8)
    else:
        gpu.qkv_rope(*args, THETA)
        want = ora.qkv_rope(qkv, qw, kw, positions, slots, cache0, cache0, rows, qh, kvh, dim, bs, blocks, EPS,
                            theta=THETA, threads=8)
    got = (down(qout, np.uint16, (rows, qh, dim)), down(kcb, np.uint16, cache0.shape),
           down(vcb, np.uint16, cache0.shape))
    for name, g, w in zip(("q", "k cache", "v cache"), got, want):
        assert_bits_equal(g, w, name)


def test_qkv_rope_cached_2048_tokens(gpu):
    rows, bs = 2048, 256
    blocks = rows // bs
    pos = np.random.default_rng(11).integers(0, 4096, rows).astype(np.int32)
    _rope_case(gpu, rows, 16, 8, 128, bs, blocks, 40, pos, unique_slots(rows, bs, blocks, 12))


def test_qkv_rope_cached_8192_tokens(gpu):
    rows, bs = 8192, 256
    blocks = rows // bs
    pos = np.random.default_rng(13).integers(0, 4096, rows).astype(np.int32)
    _rope_case(gpu, rows, 16, 8, 128, bs, blocks, 50, pos, unique_slots(rows, bs, blocks, 14))


@pytest.mark.parametrize("qh,kvh,cached", [(16, 8, False), (32, 8, True), (8, 8, True), (12, 2, True)])
def test_qkv_rope_four_waves_per_row(gpu, qh, kvh, cached):
    """From 4096 rows the d128 kernel spreads a row over four waves: head
    counts that are not 32 (extra passes, partial quads), the uncached angle
    path, and out-of-range positions and slots."""
    rows, bs = 4096, 256
    blocks = rows // bs
    rng = np.random.default_rng(qh * 10 + kvh)
    pos = rng.integers(0, 4096, rows).astype(np.int32)
    pos[::97] = -5
    pos[1::89] = 4200
    slots = unique_slots(rows, bs, blocks, qh + kvh)
    slots[::53] = -1
    slots[2::71] = bs * blocks + 3
    _rope_case(gpu, rows, qh, kvh, 128, bs, blocks, 300 + qh, pos, slots, cached=cached)


def test_qkv_rope_guards(gpu):
    """Positions outside the table rotate by 0; slots outside the cache are skipped."""
    rows, bs, blocks = 12, 4, 4
    pos = np.array([0, 1, -1, 4096, 5000, 4095, 2**31 - 1, -2**31, 7, 8, 9, 10], np.int32)
    slots = np.array([0, 15, -1, 16, 3, 100, 5, 6, -7, 2**31 - 1, 9, 10], np.int32)
    _rope_case(gpu, rows, 16, 8, 128, bs, blocks, 60, pos, slots)


@pytest.mark.parametrize("dim,qh,kvh,align", [(64, 4, 2, True), (96, 6, 3, True), (128, 16, 8, False),
                                              (256, 2, 1, True), (2, 2, 2, True)])
def test_qkv_rope_generic_shapes(gpu, dim, qh, kvh, align):
    rows, bs, blocks = 17, 4, 5
    pos = np.random.default_rng(dim).integers(0, 4096, rows).astype(np.int32)
    _rope_case(gpu, rows, qh, kvh, dim, bs, blocks, 70 + dim, pos, unique_slots(rows, bs, blocks, dim), align=align)


def test_qkv_rope_direct_matches_oracle(gpu):
    rows, bs, blocks = 64, 16, 4
    pos = np.random.default_rng(15).integers(0, 4096, rows).astype(np.int32)
    _rope_case(gpu, rows, 16, 8, 128, bs, blocks, 80, pos, unique_slots(rows, bs, blocks, 16), cached=False)


# ------------------------------------------------------------------- SiLU ----
def test_silu_8192x3072(gpu):
    rows, inter = 8192, 3072
    gu = ora.normal_bf16((rows, 2, inter), 90, 0.0, 2.0)
    out = gpu.alloc(rows * inter * 2)
    gpu.silu_mul(up(gpu, gu), out, rows, inter)
    got = down(out, np.uint16, (rows, inter))
    want = ora.silu(gu, rows, inter, threads=8)
    d = bf16_ulp_diff(got, want)
    assert d.max() <= 1, f"max {d.max()} ulp"
    assert np.mean(d == 0) > 0.999


@pytest.mark.parametrize("rows,inter", [(7, 296), (3, 2056), (1, 8), (513, 24)])
def test_silu_blocks_straddling_rows(gpu, rows, inter):
    """The flat grid puts chunks of consecutive rows in one block; chunk counts
    per row of 37, 257, 1 and 3 cross every block boundary case."""
    gu = ora.normal_bf16((rows, 2, inter), 92 + rows, 0.0, 2.0)
    out = gpu.alloc(rows * inter * 2)
    gpu.silu_mul(up(gpu, gu), out, rows, inter)
    assert bf16_ulp_diff(down(out, np.uint16, (rows, inter)), ora.silu(gu, rows, inter)).max() <= 1


def test_silu_edges_and_generic(gpu):
    g = np.array([-1e4, -100.0, -88.5, -87.0, -20.0, -0.0, 0.0, 1e-30, 3.0, 88.0, 1e4, np.inf, -np.inf, np.nan, 1.0,
                  -1.0], np.float32)
    u = np.array([1.0, 2.0, -3.0, 0.5, 1.0, 1.0, -1.0, 1.0, np.inf, 2.0, -1.0, 1.0, 1.0, 1.0, np.nan, 0.0],
                 np.float32)
    gu = np.stack([bf16_of(g), bf16_of(u)])[None]  # [1, 2, 16]
    out = gpu.alloc(32)
    gpu.silu_mul(up(gpu, gu), out, 1, 16)
    got = down(out, np.uint16, (1, 16))
    assert bf16_ulp_diff(got, ora.silu(gu, 1, 16)).max() <= 1
    rows, inter = 7, 1001
    gu2 = ora.normal_bf16((rows, 2, inter), 91, 0.0, 2.0)
    out2 = misaligned(gpu, np.zeros((rows, inter), np.uint16))
    gpu.silu_mul(misaligned(gpu, gu2), out2, rows, inter)
    assert bf16_ulp_diff(down(out2, np.uint16, (rows, inter)), ora.silu(gu2, rows, inter)).max() <= 1


# ------------------------------------------------------------------ copies ---
def test_embedding_16384_tokens(gpu):
    vocab, hidden, rows = 151936, 1024, 16384
    table = ora.normal_bf16((vocab, hidden), 100, 0.0, 0.02)
    tokens = np.random.default_rng(101).integers(0, vocab, rows).astype(np.int32)
    tokens[[5, 77, 9000]] = [-1, vocab, 2**31 - 1]  # out of range -> +0 rows
    out = gpu.alloc(rows * hidden * 2)
    gpu.embedding(up(gpu, tokens), up(gpu, table), out, rows, hidden, vocab)
    assert_bits_equal(down(out, np.uint16, (rows, hidden)), ora.embedding(tokens, table, rows, hidden, vocab))


@pytest.mark.parametrize("hidden,align", [(1, True), (12, True), (1000, False), (2048, True)])
def test_gather_shapes(gpu, hidden, align):
    input_rows, rows = 50, 23
    x = ora.normal_bf16((input_rows, hidden), 110 + hidden)
    idx = np.random.default_rng(hidden).integers(-3, input_rows + 3, rows).astype(np.int32)
    put = up if align else misaligned
    out = put(gpu, np.zeros((rows, hidden), np.uint16))
    gpu.gather(put(gpu, x), up(gpu, idx), out, rows, hidden, input_rows)
    assert_bits_equal(down(out, np.uint16, (rows, hidden)), ora.gather(x, idx, rows, hidden, input_rows))


def test_kv_write_16384_tokens(gpu):
    rows, kvh, dim, bs, blocks = 16384, 8, 128, 256, 64
    k = ora.normal_bf16((rows, kvh, dim), 120)
    v = ora.normal_bf16((rows, kvh, dim), 121)
    slots = unique_slots(rows, bs, blocks, 122)
    slots[[3, 4000]] = [-1, bs * blocks]  # skipped rows
    cache0 = np.zeros((blocks, bs, kvh, dim), np.uint16)
    kc, vc = up(gpu, cache0), up(gpu, cache0)
    gpu.kv_write(up(gpu, k), up(gpu, v), up(gpu, slots), kc, vc, rows, kvh, dim, bs, blocks)
    want_k, want_v = ora.kv_write(k, v, slots, cache0, cache0, rows, kvh, dim, bs, blocks)
    assert_bits_equal(down(kc, np.uint16, cache0.shape), want_k)
    assert_bits_equal(down(vc, np.uint16, cache0.shape), want_v)


def test_kv_write_generic(gpu):
    rows, kvh, dim, bs, blocks = 9, 3, 6, 2, 8
    k = ora.normal_bf16((rows, kvh, dim), 123)
    v = ora.normal_bf16((rows, kvh, dim), 124)
    slots = unique_slots(rows, bs, blocks, 125)
    cache0 = np.zeros((blocks, bs, kvh, dim), np.uint16)
    kc, vc = misaligned(gpu, cache0), misaligned(gpu, cache0)
    gpu.kv_write(misaligned(gpu, k), misaligned(gpu, v), up(gpu, slots), kc, vc, rows, kvh, dim, bs, blocks)
    want_k, want_v = ora.kv_write(k, v, slots, cache0, cache0, rows, kvh, dim, bs, blocks)
    assert_bits_equal(down(kc, np.uint16, cache0.shape), want_k)
    assert_bits_equal(down(vc, np.uint16, cache0.shape), want_v)


# ---------------------------------------------------------------- sampling ---
def sampling_batch(batch=256, vocab=151936, seed=130):
    """Logits ~N(0,3); round(0.01*batch) rows get +20 at a random index; first half
    greedy, second half T=0.6; seeds from src/runtime.rs:780-790."""
    logits = ora.normal_bf16((batch, vocab), seed, 0.0, 3.0)
    rng = np.random.default_rng(seed + 1)
    spiked = rng.choice(batch, size=max(1, round(0.01 * batch)), replace=False)
    for r in spiked:
        i = int(rng.integers(0, vocab))
        logits[r, i] = bf16_of(f32_of(logits[r, i]) + np.float32(20.0))
    temps = np.where(np.arange(batch) < batch // 2, 0.0, 0.6).astype(np.float32)
    seeds = np.array([ora.sampling_seed(0, r, r % 32) for r in range(batch)], np.uint64)
    return logits, temps, seeds


def _run_sampler(gpu, logits, temps, seeds, batch, vocab, parallel=True, align=True):
    put = up if align else misaligned
    lb, tb, sb = put(gpu, logits), up(gpu, temps), up(gpu, seeds)
    out = gpu.alloc(batch * 4)
    if parallel:
        parts = -(-vocab // 2048)
        ps, pi = gpu.alloc(batch * parts * 4), gpu.alloc(batch * parts * 4)
        gpu.sample_parallel(lb, tb, sb, out, ps, pi, batch, vocab)
    else:
        gpu.sample(lb, tb, sb, out, batch, vocab)
    return out.download(np.int32, batch)


def test_sampling_256x151936(gpu):
    batch, vocab = 256, 151936
    logits, temps, seeds = sampling_batch(batch, vocab)
    want = ora.sample(logits, temps, seeds, batch, vocab, threads=8)
    assert_bits_equal(_run_sampler(gpu, logits, temps, seeds, batch, vocab), want)
    assert_bits_equal(_run_sampler(gpu, logits, temps, seeds, batch, vocab, parallel=False), want)


@pytest.mark.parametrize("batch", [1, 3, 8, 64])
def test_sampling_small_batches(gpu, batch):
    vocab = 151936
    logits, temps, seeds = sampling_batch(batch, vocab, seed=140 + batch)
    temps[:] = np.where(np.arange(batch) % 2 == 0, 0.0, 1.3)
    want = ora.sample(logits, temps, seeds, batch, vocab, threads=8)
    assert_bits_equal(_run_sampler(gpu, logits, temps, seeds, batch, vocab), want)


@pytest.mark.parametrize("vocab,align", [(5, True), (2048, True), (2049, True), (10001, False), (151936, False)])
def test_sampling_ragged_vocab(gpu, vocab, align):
    batch = 4
    logits = ora.normal_bf16((batch, vocab), 150 + vocab, 0.0, 3.0)
    temps = np.array([0.0, 0.6, 1.0, -1.0], np.float32)
    seeds = np.array([42, 43, 44, 45], np.uint64)
    want = ora.sample(logits, temps, seeds, batch, vocab)
    assert_bits_equal(_run_sampler(gpu, logits, temps, seeds, batch, vocab, align=align), want)
    assert_bits_equal(_run_sampler(gpu, logits, temps, seeds, batch, vocab, parallel=False, align=align), want)


def test_sampling_special_values(gpu):
    vocab = 4096
    rows = np.stack([
        bf16_of(np.full(vocab, np.nan)),
        bf16_of(np.full(vocab, -np.inf)),
        bf16_of(np.where(np.arange(vocab) == 3000, np.inf, np.nan)),
        bf16_of(np.r_[np.full(vocab - 1, -1.0), 5.0]),
        bf16_of(np.where(np.arange(vocab) % 2048 == 2047, 9.0, 0.0)),
    ])
    for t in (0.0, 0.8):
        temps = np.full(5, t, np.float32)
        seeds = np.arange(5, dtype=np.uint64)
        want = ora.sample(rows, temps, seeds, 5, vocab)
        assert_bits_equal(_run_sampler(gpu, rows, temps, seeds, 5, vocab), want)
        assert_bits_equal(_run_sampler(gpu, rows, temps, seeds, 5, vocab, parallel=False), want)


def _noise(temperature, seed, vocab):
    """Gumbel term of every token: the score of a zero logit."""
    return np.array([ora.gumbel_score(0.0, temperature, seed, t) for t in range(vocab)], np.float32)


def test_sampling_pruning_edges(gpu):
    """Rows where the Gumbel sampler's pruning bound is tight or useless:
    scores flattened to within bf16 rounding (every token a candidate, full
    per-wave queues), extreme temperatures, equal logits, and a planted near
    tie between the largest logit and the token with the largest noise."""
    vocab = 3 * 4096 + 8
    batch = 7
    rng = np.random.default_rng(170)
    seeds = np.array([ora.sampling_seed(5, r, 3) for r in range(batch)], np.uint64)
    temps = np.array([0.6, 1.7, 1e-4, 1e4, 0.6, 0.6, 0.6], np.float32)
    logits = ora.normal_bf16((batch, vocab), 171, 0.0, 3.0)
    for r, base in ((0, 6.0), (1, -2.0)):  # logit = base - T * noise: every score ~ base / T
        logits[r] = bf16_of(np.float32(base) - temps[r] * _noise(float(temps[r]), int(seeds[r]), vocab))
    logits[4] = bf16_of(np.ones(vocab, np.float32))
    for r in (5, 6):
        noise = _noise(float(temps[r]), int(seeds[r]), vocab)
        m = int(np.argmax(f32_of(logits[r])))
        j = int(np.argmax(np.where(np.arange(vocab) == m, -np.inf, noise)))
        lm = f32_of(logits[r, m])
        target = np.float32(lm - temps[r] * (noise[j] - noise[m]))
        step = np.float32(0.0) if r == 5 else np.float32(abs(target) * 2**-7)
        logits[r, j] = bf16_of(target + step)
    want = ora.sample(logits, temps, seeds, batch, vocab)
    assert_bits_equal(_run_sampler(gpu, logits, temps, seeds, batch, vocab), want)
    assert_bits_equal(_run_sampler(gpu, logits, temps, seeds, batch, vocab, parallel=False), want)


def _edge_rows(batch, vocab, seed):
    """Rows that stress exact pruning and the total order (see the comments),
    then ordinary rows with mixed temperatures."""
    seeds = np.array([ora.sampling_seed(seed, r, 7) for r in range(batch)], np.uint64)
    temps = np.array([(0.0, 0.6, 1.3)[r % 3] for r in range(batch)], np.float32)
    logits = ora.normal_bf16((batch, vocab), seed + 1, 0.0, 3.0)
    idx = np.arange(vocab)
    temps[:7] = (0.6, 1.7, 1e-4, 1e4, 0.6, 0.6, 0.6)
    for r, base in ((0, 6.0), (1, -2.0)):  # every score ~ base / T: all tokens candidates
        logits[r] = bf16_of(np.float32(base) - temps[r] * _noise(float(temps[r]), int(seeds[r]), vocab))
    logits[4] = bf16_of(np.ones(vocab, np.float32))  # equal logits
    for r in (5, 6):  # the largest logit against the largest noise, tied (5) or one step apart (6)
        noise = _noise(float(temps[r]), int(seeds[r]), vocab)
        m = int(np.argmax(f32_of(logits[r])))
        j = int(np.argmax(np.where(idx == m, -np.inf, noise)))
        target = np.float32(f32_of(logits[r, m]) - temps[r] * (noise[j] - noise[m]))
        logits[r, j] = bf16_of(target + (np.float32(0.0) if r == 5 else np.float32(abs(target) * 2**-7)))
    special = {
        7: np.full(vocab, np.nan),
        8: np.full(vocab, -np.inf),
        9: np.where(idx == vocab // 3, np.inf, np.nan),
        10: np.r_[np.full(vocab - 1, -1.0), 5.0],
        11: np.where(idx % 2048 == 2047, 9.0, 0.0),
        16: np.where(idx % 1000 == 999, np.inf, 1.0),  # s0 = +inf: no pruning
        17: np.where(idx % 777 == 5, 3e38, -3e38),  # logit / T overflows
        18: np.where(idx < vocab // 2, -np.inf, np.nan),
    }
    for r, row in special.items():
        logits[r] = bf16_of(row)
        temps[r] = 0.8
    temps[12], temps[13], temps[14], temps[15], temps[17] = 1e-40, np.inf, np.nan, -1.0, 1e-3
    if batch > 19:  # the candidate floor's estimate bound * T is past 2^100: its full search decides
        temps[19] = 1e30
    return logits, temps, seeds


@pytest.mark.parametrize("start,batch,vocab", [(0, 16, 40000), (3, 16, 40000), (0, 19, 12296), (0, 40, 40000),
                                                (0, 100, 151936)])
def test_sampling_partition_paths_on_edge_rows(gpu, start, batch, vocab):
    """Below one row per CU: up to 16 rows every token is scored in one
    partition pass; from 17 rows the partitions prune against the row's best
    partial in a second pass. Both on the rows that stress pruning, special
    values and temperatures (rows start .. start + batch of the edge rows),
    against the oracle and the serial scan."""
    logits, temps, seeds = _edge_rows(max(19, start + batch), vocab, 190 + batch)
    logits, temps, seeds = (a[start:start + batch].copy() for a in (logits, temps, seeds))
    want = ora.sample(logits, temps, seeds, batch, vocab, threads=8)
    assert_bits_equal(_run_sampler(gpu, logits, temps, seeds, batch, vocab), want)
    assert_bits_equal(_run_sampler(gpu, logits, temps, seeds, batch, vocab, parallel=False), want)


@pytest.mark.parametrize("vocab", [3 * 4096 + 8, 40000, 90000, 131072, 163840, 163848])
def test_sampling_large_batches(gpu, vocab):
    """From one row per CU, rows of up to 163840 tokens are sampled by one
    block per row holding the row in registers; parity with the serial scan
    and the oracle on rows that stress pruning, special values and
    temperatures, for every register-tile width (4 to 20 chunks a lane) and
    just past the limit."""
    batch = max(256, gpu.sm_count())
    logits, temps, seeds = _edge_rows(batch, vocab, 180 + vocab % 97)
    want = ora.sample(logits, temps, seeds, batch, vocab, threads=8)
    assert_bits_equal(_run_sampler(gpu, logits, temps, seeds, batch, vocab), want)
    assert_bits_equal(_run_sampler(gpu, logits, temps, seeds, batch, vocab, parallel=False), want)


@pytest.mark.parametrize("greedy_rows", [1, 64, 128, 200, 255])
def test_sampling_mixed_batches_one_row_per_cu(gpu, greedy_rows):
    """One row per CU (the row-resident path), greedy rows spread over the
    batch among Gumbel rows that include the pruning edge rows (flat rows,
    extreme and subnormal temperatures, NaN and infinite logits), three calls
    in a row on the same buffers, each against the oracle."""
    batch, vocab = gpu.sm_count(), 151936
    logits, temps, seeds = _edge_rows(batch, vocab, 400 + greedy_rows)
    rng = np.random.default_rng(401 + greedy_rows)
    temps = np.where(temps > 0, temps, np.float32(0.6)).astype(np.float32)  # NaN / <= 0 -> Gumbel
    temps[rng.choice(batch, size=min(greedy_rows, batch - 1), replace=False)] = 0.0
    want = ora.sample(logits, temps, seeds, batch, vocab, threads=8)
    lb, tb, sb = up(gpu, logits), up(gpu, temps), up(gpu, seeds)
    parts = -(-vocab // 2048)
    ps, pi = gpu.alloc(batch * parts * 4), gpu.alloc(batch * parts * 4)
    for _ in range(3):
        out = gpu.alloc(batch * 4)
        gpu.sample_parallel(lb, tb, sb, out, ps, pi, batch, vocab)
        assert_bits_equal(out.download(np.int32, batch), want)


def test_sampling_one_row_per_cu_queue_windows(gpu):
    """One row per CU at temperatures whose candidates overflow a wave's LDS
    queue (2240 entries) without reaching twice that. A numpy model of these
    N(0, 3) rows puts 76-83% of the waves at T = 0.8-0.9 in that range. Those
    waves compact and score in windows; the compaction's clamped positions
    then feed the scored queue. Greedy rows, T = 0.6 rows (queues that fit) and
    T = 1.0 rows (scored in place) are mixed in, so every path of the
    paired kernel runs in one launch, against the oracle."""
    batch, vocab = gpu.sm_count(), 151936
    logits = ora.normal_bf16((batch, vocab), 460, 0.0, 3.0)
    temps = np.array([(0.0, 0.8, 0.85, 0.9, 0.6, 1.0, 0.75)[r % 7] for r in range(batch)], np.float32)
    seeds = np.array([ora.sampling_seed(461, r, 3) for r in range(batch)], np.uint64)
    want = ora.sample(logits, temps, seeds, batch, vocab, threads=8)
    assert_bits_equal(_run_sampler(gpu, logits, temps, seeds, batch, vocab), want)


@pytest.mark.parametrize("extra", [1, 37, 300])
def test_sampling_more_rows_than_cus(gpu, extra):
    """More rows than CUs: blocks of a greedy/Gumbel pair need not be resident
    together, so a Gumbel half may prune against its own best lane score
    after a bounded wait for its partner's; every row still matches the
    oracle. Greedy and Gumbel rows interleave, with edge rows among them."""
    batch, vocab = gpu.sm_count() + extra, 40000
    logits, temps, seeds = _edge_rows(batch, vocab, 420 + extra)
    temps[19:] = np.where(np.arange(19, batch) % 3 == 0, 0.0, np.float32(0.6))
    want = ora.sample(logits, temps, seeds, batch, vocab, threads=8)
    assert_bits_equal(_run_sampler(gpu, logits, temps, seeds, batch, vocab), want)


def test_sampling_beyond_paired_rows(gpu):
    """Past the context's 16384 rows of exchange words the whole-row
    resident kernel samples every row (one block per row, no partner):
    16424 rows of 8200 tokens, edge rows first, greedy and Gumbel rows
    interleaved, against the oracle."""
    batch, vocab = 16384 + 40, 8200
    logits, temps, seeds = _edge_rows(batch, vocab, 440)
    temps[19:] = np.where(np.arange(19, batch) % 3 == 0, 0.0, np.float32(0.6))
    want = ora.sample(logits, temps, seeds, batch, vocab, threads=8)
    assert_bits_equal(_run_sampler(gpu, logits, temps, seeds, batch, vocab), want)


def test_sampling_paired_graph_replays(gpu):
    """The one-row-per-CU sampler in a HIP graph: three replays with eager
    calls on other inputs between them, each against the oracle (the rows'
    exchange words must be left zero by every launch)."""
    batch, vocab = gpu.sm_count(), 151936
    logits, temps, seeds = sampling_batch(batch, vocab, seed=430)
    other, otemps, oseeds = sampling_batch(batch, vocab, seed=431)
    otemps = otemps[::-1].copy()  # Gumbel rows first
    want = ora.sample(logits, temps, seeds, batch, vocab, threads=8)
    owant = ora.sample(other, otemps, oseeds, batch, vocab, threads=8)
    lb, tb, sb = up(gpu, logits), up(gpu, temps), up(gpu, seeds)
    olb, otb, osb = up(gpu, other), up(gpu, otemps), up(gpu, oseeds)
    parts = -(-vocab // 2048)
    ps, pi = gpu.alloc(batch * parts * 4), gpu.alloc(batch * parts * 4)
    out, oout = gpu.alloc(batch * 4), gpu.alloc(batch * 4)
    graph = gpu.capture(lambda: gpu.sample_parallel(lb, tb, sb, out, ps, pi, batch, vocab))
    for _ in range(3):
        gpu.sample_parallel(olb, otb, osb, oout, ps, pi, batch, vocab)
        assert_bits_equal(oout.download(np.int32, batch), owant)
        graph.replay()
        gpu.sync()
        assert_bits_equal(out.download(np.int32, batch), want)


def test_sampling_reference_golden_vectors(gpu):
    """All 20 last-position logit rows of the reference's validation run and
    the tokens its GPU greedy sampler picked (row 4: an exact tie, lower index
    wins), through the serial kernel, the partition path (20 rows), and the
    row-resident path (the rows tiled to at least one per CU)."""
    import os

    data = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_logits.npz"))
    logits, expected = data["logits_bf16"], data["expected_greedy"]
    b, v = logits.shape
    assert b == 20
    temps, seeds = np.zeros(b, np.float32), np.zeros(b, np.uint64)
    assert _run_sampler(gpu, logits, temps, seeds, b, v).tolist() == expected.tolist()
    assert _run_sampler(gpu, logits, temps, seeds, b, v, parallel=False).tolist() == expected.tolist()
    reps = -(-max(256, gpu.sm_count()) // b)
    tiled = np.tile(logits, (reps, 1))
    n = tiled.shape[0]
    got = _run_sampler(gpu, tiled, np.zeros(n, np.float32), np.zeros(n, np.uint64), n, v)
    assert got.tolist() == np.tile(expected, reps).tolist()


# -------------------------------------------------------- paged attention ---
def _attention(gpu, q, kc, vc, pos, seqs, tables, rows, qh, kvh, dim, bs, blocks, stride, batch, max_context,
               align=True):
    put = up if align else misaligned
    out = gpu.alloc(rows * qh * dim * 2)
    gpu.paged_attention(put(gpu, q), up(gpu, kc), up(gpu, vc), up(gpu, pos), up(gpu, seqs), up(gpu, tables), out,
                        rows, qh, kvh, dim, bs, blocks, stride, batch, max_context)
    return down(out, np.uint16, (rows, qh, dim))


def _attention_case(gpu, seed, pos, seqs, qh, kvh, dim, bs, batch, stride, max_context, q_std=1.0, holes=(),
                    align=True):
    rows = len(pos)
    blocks = batch * stride
    rng = np.random.default_rng(seed)
    tables = rng.permutation(blocks).astype(np.int32)
    for i, b in holes:
        tables[i] = b
    pos, seqs = np.asarray(pos, np.int32), np.asarray(seqs, np.int32)
    q = ora.normal_bf16((rows, qh, dim), seed + 1, 0.0, q_std)
    kc = ora.normal_bf16((blocks, bs, kvh, dim), seed + 2, 0.0, 1.0)
    vc = ora.normal_bf16((blocks, bs, kvh, dim), seed + 3, 0.0, 1.0)
    want = ora.attention(q, kc, vc, pos, seqs, tables, rows, qh, kvh, dim, bs, blocks, stride, batch, max_context,
                         threads=8)
    got = _attention(gpu, q, kc, vc, pos, seqs, tables, rows, qh, kvh, dim, bs, blocks, stride, batch, max_context,
                     align)
    assert_bits_equal(got, want)
    return want


@pytest.mark.parametrize("q_std", [1.0, 6.0])
def test_attention_decode_qwen3_shapes(gpu, q_std):
    """16 decode rows of Qwen3-0.6B attention (16 q heads, 8 kv heads, dim 128,
    256-token blocks) with contexts up to 4096; q_std 6 spreads the scores so
    many probabilities are subnormal or zero."""
    rng = np.random.default_rng(200)
    batch, stride = 16, 16
    pos = np.r_[4095, 0, 255, 256, rng.integers(0, 4096, size=12)]
    _attention_case(gpu, 201, pos, np.arange(batch), 16, 8, 128, 256, batch, stride, 4096, q_std=q_std)


def test_attention_ragged_prefill_rows(gpu):
    """Flattened prefill of three sequences (300, 1 and 700 tokens) with
    16-token blocks, one row per token."""
    lens = [300, 1, 700]
    pos = np.concatenate([np.arange(n) for n in lens])
    seqs = np.concatenate([np.full(n, i) for i, n in enumerate(lens)])
    _attention_case(gpu, 210, pos, seqs, 16, 8, 128, 16, 3, 44, 1024)


def test_attention_many_rows_odd_block_size(gpu):
    """600 prefill rows (two 300-token prompts) with 7-token blocks: more than
    two head-pair blocks per CU, so the occupancy layout runs, with the
    block-size division path."""
    lens = [300, 300]
    pos = np.concatenate([np.arange(n) for n in lens])
    seqs = np.concatenate([np.full(n, i) for i, n in enumerate(lens)])
    _attention_case(gpu, 215, pos, seqs, 16, 8, 128, 7, 2, 44, 300)


@pytest.mark.parametrize("dim,qh,kvh,bs", [(32, 4, 2, 8), (64, 8, 2, 256), (256, 4, 4, 16), (128, 6, 2, 7),
                                           (128, 4, 4, 32), (80, 4, 2, 16), (96, 2, 1, 5), (2, 2, 2, 4),
                                           (32, 4, 2, 256), (128, 8, 8, 64), (64, 2, 2, 128)])
def test_attention_head_dims_groups_and_block_sizes(gpu, dim, qh, kvh, bs):
    rng = np.random.default_rng(dim * 7 + bs)
    batch, max_context = 4, 520
    stride = -(-max_context // bs)
    pos = rng.integers(0, max_context, size=9)
    pos[0] = max_context - 1
    seqs = rng.integers(0, batch, size=9)
    _attention_case(gpu, 220 + dim, pos, seqs, qh, kvh, dim, bs, batch, stride, max_context)


@pytest.mark.parametrize("dim,qh,kvh,bs", [(256, 4, 4, 64), (256, 4, 4, 256), (64, 8, 2, 256), (32, 4, 2, 64)])
@pytest.mark.parametrize("above_cus", [False, True])
def test_attention_aligned_tile_paths_other_head_dims(gpu, dim, qh, kvh, bs, above_cus):
    """Head dims other than 128 with blocks that hold whole K steps and V
    tiles: at most one block per CU (V tiles streamed into LDS slots; at head
    dim 256 a tile is 32 tokens, two rows per 1 KB wave load) and more blocks
    than CUs (V tiles through registers); contexts ending on and inside
    tiles."""
    cus = gpu.sm_count()
    rows = cus // qh + 1 if above_cus else min(9, cus // qh)
    batch, max_context = 4, 520
    stride = -(-max_context // bs)
    rng = np.random.default_rng(dim * 11 + bs + above_cus)
    pos = rng.integers(0, max_context, size=rows)
    pos[:5] = [max_context - 1, 31, 32, 63, 0]
    seqs = rng.integers(0, batch, size=rows)
    _attention_case(gpu, 270 + dim + bs + above_cus, pos, seqs, qh, kvh, dim, bs, batch, stride, max_context)


def test_attention_invalid_rows_and_blocks(gpu):
    """Rows with a bad sequence index or a context beyond max_context or the
    table give zeros; table entries outside [0, blocks) drop their tokens."""
    batch, stride, bs = 3, 4, 64
    pos = [100, 0, 255, 300, 200, 63, 64, 10]
    seqs = [0, -1, 1, 0, 3, 2, 2, 1]
    holes = [(1, -1), (stride + 0, 3 * stride + 9), (2 * stride + 1, -7)]
    want = _attention_case(gpu, 230, pos, seqs, 4, 2, 128, bs, batch, stride, 256, holes=holes)
    assert not want[1].any() and not want[3].any() and not want[4].any()


def test_attention_aligned_blocks_with_holes_mid_context(gpu):
    """256-token blocks (whole K steps and V tiles per block: the block table is
    read once per step from a register) with invalid entries in the middle and
    at the end of long contexts, and contexts ending inside a step or a tile."""
    batch, stride, bs = 4, 16, 256
    pos = [999, 4095, 700, 63, 64, 1023, 2047, 300]
    seqs = [0, 1, 2, 3, 0, 1, 2, 3]
    holes = [(1, -1), (stride + 7, batch * stride + 5), (2 * stride + 2, -3), (3 * stride + 1, batch * stride)]
    _attention_case(gpu, 235, pos, seqs, 16, 8, 128, bs, batch, stride, 4096, holes=holes)


@pytest.mark.parametrize("rows", [8, 32])
def test_attention_streamed_tiles_signed_zero_and_tiny_values(gpu, rows):
    """The streamed-tile value chain (one block per CU, head dim 128, 256-token
    blocks; one q head per block at 8 rows, a GQA pair at 32): scores spread
    so that many probabilities are subnormal or zero (q_std 6), V dimensions
    of the smallest subnormals, whose products and outputs round to -0 or +0
    (the sign must survive the chain), and of tiny values with subnormal
    outputs; contexts ending on, just past and inside 64-token tiles."""
    qh, kvh, dim, bs, stride, max_context = 16, 8, 128, 256, 16, 4096
    rng = np.random.default_rng(260 + rows)
    blocks = rows * stride
    tables = rng.permutation(blocks).astype(np.int32)
    pos = rng.integers(0, 2048, size=rows).astype(np.int32)
    pos[:8] = [1023, 63, 64, 127, 150, 4095, 0, 700]
    seqs = np.arange(rows, dtype=np.int32)
    q = ora.normal_bf16((rows, qh, dim), 261, 0.0, 6.0)
    kc = ora.normal_bf16((blocks, bs, kvh, dim), 262, 0.0, 1.0)
    vc = ora.normal_bf16((blocks, bs, kvh, dim), 263, 0.0, 1.0)
    vc[..., 16:20] = 0x8001  # the smallest bf16 subnormals, negative and positive:
    vc[..., 20:24] = 0x0001  # products and outputs round to signed zeros
    vc[..., 24:32] = ora.normal_bf16((blocks, bs, kvh, 8), 264, 0.0, 1e-38)  # subnormal outputs
    want = ora.attention(q, kc, vc, pos, seqs, tables, rows, qh, kvh, dim, bs, blocks, stride, rows, max_context,
                         threads=8)
    got = _attention(gpu, q, kc, vc, pos, seqs, tables, rows, qh, kvh, dim, bs, blocks, stride, rows, max_context)
    assert_bits_equal(got, want)
    assert (want == 0x8000).any() and (want == 0).any()  # both signed zeros occur


@pytest.mark.parametrize("extra_rows", [0, 1])
def test_attention_aligned_streamed_and_register_tiles(gpu, extra_rows):
    """256-token blocks with a GQA pair per block at exactly one block per CU
    (the V tiles stream from memory into LDS slots) and with one row more
    (the V tiles pass through registers): contexts that end on, just past and
    inside 64-token tiles, one-tile contexts, and invalid table entries in the
    middle and at the end of contexts."""
    qh, kvh, dim, bs, stride, max_context = 16, 8, 128, 256, 16, 4096
    rows = gpu.sm_count() // (qh // 2) + extra_rows
    rng = np.random.default_rng(240 + extra_rows)
    pos = rng.integers(0, 2048, size=rows)
    edges = [0, 62, 63, 64, 127, 128, 191, 192, 255, 256, 4095, 1000]
    pos[:len(edges)] = edges
    holes = [(1 * stride + 0, -1), (11 * stride + 2, rows * stride), (12 * stride + 3, -5), (13 * stride, -1)]
    _attention_case(gpu, 245 + extra_rows, pos, np.arange(rows), qh, kvh, dim, bs, rows, stride, max_context,
                    holes=holes)


@pytest.mark.parametrize("rows,bs,seed", [(8, 256, 300), (32, 256, 310), (8, 16, 320), (5, 7, 330), (32, 16, 340),
                                         (32, 7, 350)])
def test_attention_qkv_rope_matches_separate_launches(gpu, rows, bs, seed):
    """The fused decode form (q/k norm + RoPE + KV write inside the attention
    launch) against qkv_rope_cached + paged_attention and the oracle: out and
    both caches bit for bit. One row per sequence with the slot its table
    gives; 8 rows take one q head per block, 32 a GQA pair; 256-, 16- and
    7-token blocks cover the three table lookups (register table, shift and
    divide), each with a GQA pair per block at 32 rows. The last row of the 5-row
    case has an invalid sequence and slot -1 (zero output, no KV write)."""
    qh, kvh, dim, max_context = 16, 8, 128, 4096
    rng = np.random.default_rng(seed)
    batch, stride = rows, -(-max_context // bs)
    blocks = batch * stride
    tables = rng.permutation(blocks).astype(np.int32)
    pos = rng.integers(0, max_context, size=rows).astype(np.int32)
    pos[:4] = [max_context - 1, 0, bs - 1, bs][:min(4, rows)]
    seqs = np.arange(rows, dtype=np.int32)
    slots = (tables[seqs * stride + pos // bs] * bs + pos % bs).astype(np.int32)
    if rows == 5:
        seqs[-1], slots[-1] = -1, -1
    heads = qh + 2 * kvh
    qkv = ora.normal_bf16((rows, heads, dim), seed + 1)
    qw = ora.normal_bf16(dim, seed + 2, 1.0, 0.02)
    kw = ora.normal_bf16(dim, seed + 3, 1.0, 0.02)
    kc0 = ora.normal_bf16((blocks, bs, kvh, dim), seed + 4)
    vc0 = ora.normal_bf16((blocks, bs, kvh, dim), seed + 5)
    tb = gpu.alloc(max_context * dim * 4)
    gpu.rope_cache(tb, max_context, dim, THETA)
    dq, dqw, dkw, dpos, dslots, dseqs, dtab = (up(gpu, a) for a in (qkv, qw, kw, pos, slots, seqs, tables))

    kc1, vc1 = up(gpu, kc0), up(gpu, vc0)
    qout, out1 = gpu.alloc(rows * qh * dim * 2), gpu.alloc(rows * qh * dim * 2)
    gpu.qkv_rope_cached(dq, dqw, dkw, dpos, dslots, qout, kc1, vc1, rows, qh, kvh, dim, bs, blocks, EPS, tb,
                        max_context)
    gpu.paged_attention(qout, kc1, vc1, dpos, dseqs, dtab, out1, rows, qh, kvh, dim, bs, blocks, stride, batch,
                        max_context)
    kc2, vc2 = up(gpu, kc0), up(gpu, vc0)
    out2 = gpu.alloc(rows * qh * dim * 2)
    gpu.attention_qkv_rope(dq, dqw, dkw, dpos, dslots, kc2, vc2, dseqs, dtab, out2, rows, qh, kvh, dim, bs, blocks,
                           stride, batch, max_context, EPS, tb, max_context)
    shape = (blocks, bs, kvh, dim)
    for name, a, b, sh in (("out", out1, out2, (rows, qh, dim)), ("k cache", kc1, kc2, shape),
                           ("v cache", vc1, vc2, shape)):
        assert_bits_equal(down(b, np.uint16, sh), down(a, np.uint16, sh), name)

    table = down(tb, np.float32, (max_context, dim))
    q_r, kc_r, vc_r = ora.qkv_rope(qkv, qw, kw, pos, slots, kc0, vc0, rows, qh, kvh, dim, bs, blocks, EPS,
                                   table=table, max_positions=max_context, threads=8)
    want = ora.attention(q_r, kc_r, vc_r, pos, seqs, tables, rows, qh, kvh, dim, bs, blocks, stride, batch,
                         max_context, threads=8)
    assert_bits_equal(down(out2, np.uint16, (rows, qh, dim)), want, "out vs oracle")
    assert_bits_equal(down(kc2, np.uint16, shape), kc_r, "k cache vs oracle")


def test_attention_qkv_rope_rejects_other_head_dims(gpu):
    b = gpu.alloc(1 << 16)
    with pytest.raises(Exception):
        gpu.attention_qkv_rope(b, b, b, b, b, b, b, b, b, b, 1, 2, 1, 64, 16, 1, 1, 1, 16, EPS, b, 16)


def test_attention_generic_path_for_unaligned_queries(gpu):
    _attention_case(gpu, 240, [0, 77, 399], [0, 1, 1], 4, 2, 128, 16, 2, 25, 400, align=False)


def test_attention_special_values(gpu):
    """An infinite score (maximum not finite) zeroes the row; NaN keys give NaN
    scores that the maximum ignores."""
    dim, bs, blocks = 32, 4, 2
    q = bf16_of(np.r_[np.full(dim, 3e38), np.ones(dim), np.ones(dim)].astype(np.float32))
    kc = bf16_of(np.ones((blocks, bs, 1, dim), np.float32))
    kc2 = kc.copy()
    kc2[0, 1, 0, 5] = bf16_of(np.float32(np.nan))
    tables = np.array([0, 1], np.int32)
    vc = ora.normal_bf16((blocks, bs, 1, dim), 250, 0.0, 1.0)
    pos, seqs = np.array([5, 5, 2], np.int32), np.zeros(3, np.int32)
    for keys in (kc, kc2):
        want = ora.attention(q, keys, vc, pos, seqs, tables, 3, 1, 1, dim, bs, blocks, 2, 1, 8)
        got = _attention(gpu, q, keys, vc, pos, seqs, tables, 3, 1, 1, dim, bs, blocks, 2, 1, 8)
        assert_bits_equal(got, want)
        assert not want[0].any()


# ------------------------------------------------------------------- GEMM ----
def test_gemm_known_answer_and_random(gpu):
    # src/gpu.rs:1290-1298: X = [[1,2,3],[4,5,6]], W = [[1,0,1],[0,1,0]] -> [[4,2],[10,5]].
    x = up(gpu, bf16_of([1, 2, 3, 4, 5, 6]))
    w = up(gpu, bf16_of([1, 0, 1, 0, 1, 0]))
    y = gpu.alloc(8)
    gpu.gemm(x, w, y, 2, 2, 3)
    assert f32_of(y.download(np.uint16, 4)).tolist() == [4.0, 2.0, 10.0, 5.0]
    m, n, k = 64, 96, 256
    xa = ora.normal_bf16((m, k), 160)
    wa = ora.normal_bf16((n, k), 161)
    yb = gpu.alloc(m * n * 2)
    gpu.gemm(up(gpu, xa), up(gpu, wa), yb, m, n, k)
    got = f32_of(down(yb, np.uint16, (m, n))).astype(np.float64)
    want = f32_of(xa).astype(np.float64) @ f32_of(wa).astype(np.float64).T
    assert np.max(np.abs(got - want) / (np.abs(want) + 1.0)) < 1e-2


def _gemm_bound(xa, wa):
    """float64 product and an error bound for fp32 accumulation + one bf16
    rounding: 2^-8 |y| + 2^-20 k sum|x w| (a dropped or doubled 8-element
    chunk is far outside it)."""
    xf, wf = f32_of(xa).astype(np.float64), f32_of(wa).astype(np.float64)
    return xf @ wf.T, 2.0 ** -8 * np.abs(xf @ wf.T) + 2.0 ** -20 * xa.shape[1] * (np.abs(xf) @ np.abs(wf).T)


@pytest.mark.parametrize("m,n,k", [(8, 4096, 1024), (8, 1024, 2048), (8, 6144, 1024), (8, 1024, 3072),
                                   (1, 1000, 512), (5, 77, 1536), (32, 4096, 1024), (16, 1024, 2048),
                                   (3, 2050, 4096), (32, 300, 2048), (33, 64, 512)])
def test_gemm_few_rows(gpu, m, n, k):
    """Decode-sized GEMMs (the Qwen3-0.6B layer shapes at 8, 16 and 32 rows,
    ragged n and odd row counts) against the float64 product."""
    seed = m * 131 + n * 7 + k
    xa = ora.normal_bf16((m, k), seed)
    wa = ora.normal_bf16((n, k), seed + 1)
    yb = gpu.alloc(m * n * 2)
    gpu.gemm(up(gpu, xa), up(gpu, wa), yb, m, n, k)
    got = f32_of(down(yb, np.uint16, (m, n))).astype(np.float64)
    want, bound = _gemm_bound(xa, wa)
    assert np.all(np.abs(got - want) <= bound), np.max(np.abs(got - want) - bound)


def test_gemm_few_rows_graph_replays(gpu):
    """A decode-sized GEMM captured in a graph: every replay (new X uploaded
    between them) equals an eager launch bit for bit."""
    m, n, k = 8, 1024, 1024
    wa = ora.normal_bf16((n, k), 170)
    w, x, y = up(gpu, wa), gpu.alloc(m * k * 2), gpu.alloc(m * n * 2)
    x.upload(ora.normal_bf16((m, k), 171))
    gpu.sync()
    graph = gpu.capture(lambda: gpu.gemm(x, w, y, m, n, k))
    for seed in (172, 173, 174):
        xa = ora.normal_bf16((m, k), seed)
        x.upload(xa)
        graph.replay()
        replayed = down(y, np.uint16, (m, n)).copy()
        gpu.gemm(x, w, y, m, n, k)
        assert_bits_equal(replayed, down(y, np.uint16, (m, n)))
        want, bound = _gemm_bound(xa, wa)
        assert np.all(np.abs(f32_of(replayed).astype(np.float64) - want) <= bound)


# ------------------------------------------------------- norm fused into GEMM --
@pytest.mark.parametrize("m,n,k,add", [
    (8, 4096, 1024, True),    # decode: post-attention norm + ... the qkv shape
    (8, 6144, 1024, True),    # gate_up
    (1, 4096, 1024, False),   # layer 0's plain RMSNorm, one row
    (32, 4096, 1024, True),   # two row tiles
    (17, 512, 2048, True),    # ragged second tile, k 2048
    (5, 16, 512, False),      # one column tile, k 512
    (16, 4096, 1024, True),   # 8-wave blocks: all 16 rows in one norm pass
    (12, 6144, 2048, True),   # 4-wave blocks: two norm passes, the second ragged
])
def test_rms_gemm_norm_bits_and_gemm_bound(gpu, m, n, k, add):
    """nv_rms_gemm: the normalised rows and the updated residual equal the oracle's
    (add-)RMSNorm bit for bit; y lies within the float64 GEMM bound of those rows
    times W; a second launch gives the same bits."""
    seed = m * 7 + n + k
    xa = ora.normal_bf16((m, k), seed)
    ra = ora.normal_bf16((m, k), seed + 1)
    nw = ora.normal_bf16(k, seed + 2, 1.0, 0.02)
    wa = ora.normal_bf16((n, k), seed + 3, 0.0, 0.05)
    x, r, w = up(gpu, xa), up(gpu, ra), up(gpu, wa)
    y, normed = gpu.alloc(m * n * 2), gpu.alloc(m * k * 2)
    r_out = gpu.alloc(m * k * 2) if add else None
    gpu.rms_gemm(x, r if add else None, r_out, up(gpu, nw), w, y, normed, m, n, k, EPS)
    if add:
        want_res, want_norm = ora.add_rms(xa, ra, nw, m, k, EPS)
        assert_bits_equal(down(r_out, np.uint16, (m, k)), want_res, "residual_out")
        assert_bits_equal(down(r, np.uint16, (m, k)), ra.reshape(m, k), "residual (read only)")
    else:
        want_norm = ora.rms(xa, nw, m, k, EPS)
    assert_bits_equal(down(normed, np.uint16, (m, k)), want_norm, "normed")
    first = down(y, np.uint16, (m, n)).copy()
    want, bound = _gemm_bound(want_norm.reshape(m, k), wa)
    got = f32_of(first).astype(np.float64)
    assert np.all(np.abs(got - want) <= bound), np.max(np.abs(got - want) - bound)
    gpu.rms_gemm(x, r if add else None, None, up(gpu, nw), w, y, None, m, n, k, EPS)
    assert_bits_equal(down(y, np.uint16, (m, n)), first, "second launch")


def test_rms_gemm_rejects_unsupported_shapes(gpu):
    x, w, y = gpu.alloc(40 * 1024 * 2), gpu.alloc(4096 * 1024 * 2), gpu.alloc(40 * 4096 * 2)
    nw = gpu.alloc(1024 * 2)
    for m, n, k in ((33, 4096, 1024), (8, 4008, 1024), (8, 4096, 768)):
        with pytest.raises(nvr.ArgumentError):
            gpu.rms_gemm(x, None, None, nw, w, y, None, m, n, k, EPS)
    lib, h = gpu.lib, gpu.handle
    assert lib.nv_rms_gemm(h, x.ptr, None, None, nw.ptr, w.ptr, y.ptr, None, 33, 4096, 1024, EPS) == -2
    assert lib.nv_rms_gemm(h, x.ptr, None, y.ptr, nw.ptr, w.ptr, y.ptr, None, 8, 4096, 1024, EPS) == -2
    assert b"residual_out" in lib.nv_last_error()


@pytest.mark.parametrize("m,inter,k,add", [(8, 3072, 1024, True), (1, 3072, 1024, False), (20, 512, 2048, True),
                                           (5, 64, 512, False), (16, 3072, 1024, True), (16, 2048, 1024, True)])
def test_rms_gemm_silu_epilogue(gpu, m, inter, k, add):
    """nv_rms_gemm_silu: the norm outputs are the oracle's bits; gate_up (written in
    [gate | up] order from the tile-ordered weight) equals nv_rms_gemm's output with
    the plain weight bit for bit and lies within the float64 GEMM bound; act equals
    the oracle's SiLU·up of those gate_up values within 1 bf16 ulp."""
    seed = m + inter + k
    xa = ora.normal_bf16((m, k), seed)
    ra = ora.normal_bf16((m, k), seed + 1)
    nw = ora.normal_bf16(k, seed + 2, 1.0, 0.02)
    wa = ora.normal_bf16((2 * inter, k), seed + 3, 0.0, 0.05)
    x, r, nwb = up(gpu, xa), up(gpu, ra), up(gpu, nw)
    tiled = up(gpu, nvr.tile_gate_up_rows(wa, inter))
    gu, act, normed = gpu.alloc(m * 2 * inter * 2), gpu.alloc(m * inter * 2), gpu.alloc(m * k * 2)
    r_out = gpu.alloc(m * k * 2) if add else None
    gpu.rms_gemm_silu(x, r if add else None, r_out, nwb, tiled, gu, act, normed, m, inter, k, EPS)
    if add:
        want_res, want_norm = ora.add_rms(xa, ra, nw, m, k, EPS)
        assert_bits_equal(down(r_out, np.uint16, (m, k)), want_res, "residual_out")
    else:
        want_norm = ora.rms(xa, nw, m, k, EPS)
    assert_bits_equal(down(normed, np.uint16, (m, k)), want_norm, "normed")
    got_gu = down(gu, np.uint16, (m, 2 * inter))
    plain = gpu.alloc(m * 2 * inter * 2)
    gpu.rms_gemm(x, r if add else None, None, nwb, up(gpu, wa), plain, None, m, 2 * inter, k, EPS)
    assert_bits_equal(got_gu, down(plain, np.uint16, (m, 2 * inter)), "gate_up vs nv_rms_gemm")
    want, bound = _gemm_bound(want_norm.reshape(m, k), wa)
    assert np.all(np.abs(f32_of(got_gu).astype(np.float64) - want) <= bound)
    want_act = ora.silu(got_gu.reshape(m, 2, inter), m, inter).reshape(m, inter)
    assert bf16_ulp_diff(down(act, np.uint16, (m, inter)), want_act).max() <= 1



@pytest.mark.parametrize("m,n,k", [(8, 1024, 2048), (8, 1024, 3072), (8, 151936, 1024), (1, 4096, 1024),
                                   (16, 1024, 2048), (32, 1024, 3072), (17, 2048, 4096), (3, 16, 1024),
                                   (1, 1024, 1024), (12, 1024, 4096), (9, 2032, 3072), (5, 4096, 4096)])
def test_gemm_rows_within_bound_and_deterministic(gpu, m, n, k):
    """nv_gemm_rows against the float64 product (the bound of nv_gemm's test); a
    second launch and a graph replay give the same bits."""
    seed = m * 3 + n + k
    xa = ora.normal_bf16((m, k), seed)
    wa = ora.normal_bf16((n, k), seed + 1, 0.0, 0.05)
    x, w, y = up(gpu, xa), up(gpu, wa), gpu.alloc(m * n * 2)
    gpu.gemm_rows(x, w, y, m, n, k)
    first = down(y, np.uint16, (m, n)).copy()
    if n * k <= 4096 * 4096:
        want, bound = _gemm_bound(xa, wa)
        assert np.all(np.abs(f32_of(first).astype(np.float64) - want) <= bound)
    else:  # the vocabulary-wide shape: 4096 columns spread over the output
        cols = np.random.default_rng(seed).choice(n, 4096, replace=False)
        want, bound = _gemm_bound(xa, wa[cols])
        assert np.all(np.abs(f32_of(first[:, cols]).astype(np.float64) - want) <= bound)
    gpu.sync()
    graph = gpu.capture(lambda: gpu.gemm_rows(x, w, y, m, n, k))
    graph.replay()
    assert_bits_equal(down(y, np.uint16, (m, n)), first, "graph replay")
