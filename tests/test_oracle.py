"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Each test checks the oracle against something it does not share code with:
the reference's own known answers (src/gpu.rs tests), golden vectors from the
reference's data files (tests/golden/), the published SplitMix64 algorithm,
closed forms in float64, or brute force on small inputs. No GPU needed.
"""
import json
import math
import os
import re

import numpy as np
import pytest

import oracle as ora
from helpers import bf16_of, bf16_ulp_diff, f32_of

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
M64 = 2**64 - 1


# ------------------------------------------------------------- bf16 -------
def test_bf16_rounding_matches_round_to_nearest_even():
    # Halfway cases: 1 + 2^-8 lies between bf16 1.0 and 1.0078125 -> even (1.0);
    # 1 + 3*2^-8 lies between 1.0078125 and 1.015625 -> even (1.015625).
    assert ora.lib().ora_bf16_from_f32(1.0 + 2**-8) == 0x3F80
    assert ora.lib().ora_bf16_from_f32(1.0 + 3 * 2**-8) == 0x3F82
    assert ora.lib().ora_bf16_from_f32(1.0 + 2**-8 + 2**-20) == 0x3F81
    assert ora.lib().ora_bf16_from_f32(-0.0) == 0x8000
    assert ora.lib().ora_bf16_from_f32(float("inf")) == 0x7F80
    assert ora.lib().ora_bf16_from_f32(3.4028234663852886e38) == 0x7F80  # rounds up to inf
    assert (ora.lib().ora_bf16_from_f32(float("nan")) & 0x7FFF) > 0x7F80
    # Against numpy-float64 nearest selection on random values.
    rng = np.random.default_rng(0)
    x = rng.standard_normal(20000).astype(np.float32) * np.float32(37.0)
    bits = np.array([ora.lib().ora_bf16_from_f32(float(v)) for v in x[:2000]], np.uint16)
    lo = (x[:2000].view(np.uint32) >> 16).astype(np.uint16)
    hi = lo + 1
    d_lo = np.abs(f32_of(lo).astype(np.float64) - x[:2000])
    d_hi = np.abs(f32_of(hi).astype(np.float64) - x[:2000])
    want = np.where(d_lo < d_hi, lo, np.where(d_hi < d_lo, hi, np.where(lo % 2 == 0, lo, hi)))
    assert np.array_equal(bits, want)


# -------------------------------------------------------- SplitMix64 -------
def _splitmix64_py(v: int) -> int:
    v = (v + 0x9E3779B97F4A7C15) & M64
    v = ((v ^ (v >> 30)) * 0xBF58476D1CE4E5B9) & M64
    v = ((v ^ (v >> 27)) * 0x94D049BB133111EB) & M64
    return v ^ (v >> 31)


def test_splitmix64_known_answers():
    assert ora.splitmix64(0) == 0xE220A8397B1DCDAF
    assert ora.splitmix64(1) == 0x910A2DEC89025CC1
    for v in [2, 42, 2**63, M64, 0x123456789ABCDEF0]:
        assert ora.splitmix64(v) == _splitmix64_py(v)


def test_sampling_seed_matches_runtime_rs_definition():
    # src/runtime.rs:780-790: mix(mix(base) ^ mix(request_id) ^ mix(generated)).
    for base, rid, gen in [(0, 0, 0), (0, 5, 3), (1234, 17, 100), (M64, 1, 2)]:
        want = _splitmix64_py(_splitmix64_py(base) ^ _splitmix64_py(rid) ^ _splitmix64_py(gen))
        assert ora.sampling_seed(base, rid, gen) == want


# --------------------------------------------------------------- log -------
def _ulp_error(got: np.ndarray, want: np.ndarray) -> np.ndarray:
    spacing = np.spacing(np.abs(want.astype(np.float32))).astype(np.float64)
    return np.abs(got.astype(np.float64) - want) / spacing


def test_logf_is_faithful_on_the_whole_gumbel_domain():
    """Exhaustive over every uniform the sampler can draw and every -ln(u)."""
    k = np.arange(1 << 23, dtype=np.float32)
    u = (k + np.float32(0.5)) * np.float32(1.0 / 8388608.0)
    l1 = ora.logf_array(u)
    assert _ulp_error(l1, np.log(u.astype(np.float64))).max() < 1.0
    l2 = ora.logf_array(-l1)
    assert _ulp_error(l2, np.log((-l1).astype(np.float64))).max() < 1.0
    # Bounds of the Gumbel noise -ln(-ln u) the sampler can produce.
    assert float(l2.min()) == pytest.approx(-16.6355324, abs=1e-6)
    assert float(l2.max()) == pytest.approx(2.81154084, abs=1e-6)
    # The GPU sampler prunes tokens with this maximum as the noise bound
    # (kNoiseMax in csrc/sample.hip); it must not be below the true maximum.
    src = open(os.path.join(os.path.dirname(__file__), "..", "nano-vllm-rs_amd", "csrc", "sample.hip")).read()
    bound = float.fromhex(re.search(r"kNoiseMax = (0x[0-9a-fA-Fp.+-]+)f;", src).group(1))
    assert np.float32(bound) == np.float32(-l2.min())


def test_gumbel_noise_floors_are_lower_bounds():
    """The row-resident sampler rejects a candidate when its hash value m is
    below floor_k, the bound it computes for noise level D_k = -4 + k/16. That
    is exact only if every m whose noise -ln(-ln u) reaches D_k is >= floor_k:
    checked here for every k against the noise of all 2^23 hash values, with
    floor_k computed by the same operations (nvr_expf = ora_expf)."""
    src = open(os.path.join(os.path.dirname(__file__), "..", "nano-vllm-rs_amd", "csrc", "sample.hip")).read()
    steps = int(re.search(r"kFloorSteps = (\d+);", src).group(1))
    assert "float(k) * 0.0625f - 4.0f" in src and "(d - 0x1.0p-12f)" in src and "* 8388608.0f) - 64.0f" in src
    k = np.arange(1 << 23, dtype=np.float32)
    u = (k + np.float32(0.5)) * np.float32(1.0 / 8388608.0)
    noise = -ora.logf_array(-ora.logf_array(u))
    reach = np.maximum.accumulate(noise.astype(np.float64))  # first m reaching D = searchsorted
    d = np.arange(steps, dtype=np.float32) * np.float32(0.0625) - np.float32(4.0)
    e1 = ora.expf_array(-(d - np.float32(2.0**-12)))
    uu = ora.expf_array(-e1)
    floors = np.maximum(np.floor(uu * np.float32(8388608.0)) - np.float32(64.0), 0).astype(np.int64)
    noise_max = float(noise.max())
    floors = np.where(d.astype(np.float64) > noise_max, 1 << 23, floors)
    first = np.searchsorted(reach, d.astype(np.float64), side="left")  # 2^23 when no m reaches D_k
    assert (floors <= first).all()
    # Tight enough to matter: within 1024 of the exact first m (of 2^23).
    assert ((first - floors) <= 1024).all()
    assert d[-1] > noise_max


def test_logf_is_faithful_on_random_positive_normals():
    rng = np.random.default_rng(1)
    bits = rng.integers(0x00800000, 0x7F800000, size=2_000_000, dtype=np.uint32)
    x = bits.view(np.float32)
    assert _ulp_error(ora.logf_array(x), np.log(x.astype(np.float64))).max() < 1.0
    assert ora.logf(1.0) == 0.0
    assert ora.logf(2.0) == np.float32(math.log(2.0))


# ----------------------------------------------------------- Gumbel -------
def test_gumbel_max_reproduces_softmax_frequencies():
    """Gumbel-max with temperature T draws token i with probability softmax(l/T)_i.
    A sign error or a wrong uniform mapping shifts these frequencies."""
    logits = np.array([1.0, 2.0, 0.5, 2.0, -1.0, 0.0, 1.5, 3.0], np.float32)
    T = 0.6
    draws = 20000
    bits = np.tile(bf16_of(logits), (draws, 1))
    temps = np.full(draws, T, np.float32)
    seeds = np.array([ora.sampling_seed(7, r, 0) for r in range(draws)], np.uint64)
    picks = ora.sample(bits, temps, seeds, draws, logits.size, threads=8)
    p = np.exp(f32_of(bits[0]).astype(np.float64) / T)
    p /= p.sum()
    freq = np.bincount(picks, minlength=logits.size) / draws
    sigma = np.sqrt(p * (1 - p) / draws)
    assert np.all(np.abs(freq - p) < 5 * sigma + 1e-4), (freq, p)


def test_gumbel_score_definition():
    seed, token, logit, T = 0xDEADBEEF, 1234, 3.25, 0.6
    r = _splitmix64_py(seed ^ ((token * 0xD2B74407B1CE6E93) & M64))
    u = np.float32((np.float32(r >> 41) + np.float32(0.5)) * np.float32(2.0**-23))
    want = np.float32(np.float32(logit) / np.float32(T)) - np.float32(math.log(-math.log(float(u))))
    assert ora.gumbel_score(logit, T, seed, token) == pytest.approx(float(want), abs=2e-6)


# -------------------------------------------------------- reductions -------
def test_block_sum_sq_is_exact_on_exact_inputs_and_close_otherwise():
    v = np.arange(1, 129, dtype=np.float32)  # sum of squares 1..128 is exact in fp32
    assert ora.block_sum_sq(v) == float(np.sum(np.arange(1, 129, dtype=np.int64) ** 2))
    rng = np.random.default_rng(2)
    for n in (1, 7, 128, 255, 256, 257, 1024, 3000):
        x = rng.standard_normal(n).astype(np.float32)
        got = ora.block_sum_sq(x)
        assert got == pytest.approx(math.fsum(float(t) ** 2 for t in x), rel=2e-6)


def test_block_sum_sq_follows_the_256_thread_tree_order():
    """Brute-force model of kernels/kernels.cu:109-125 with one value per thread:
    a 3-level tree where ordering is visible (large + small cancellation)."""
    x = np.zeros(256, np.float32)
    x[0], x[16], x[64] = 2.0**12, 1.0, 2.0**12
    # warp 0: lanes 0 and 16 meet at offset 16: (2^24 + 1) rounds to 2^24.
    # warp 2: 2^24. Block: warp0 + warp2 = 2^25 exactly.
    assert ora.block_sum_sq(x) == 2.0**25
    y = np.zeros(256, np.float32)
    y[0], y[1], y[2] = 2.0**12, 1.0, 1.0
    # lanes 0,1,2 of warp 0: offset 2 folds lane 2 into lane 0 first:
    # (2^24 + 1) -> 2^24, then offset 1 adds lane 1: (2^24 + 1) -> 2^24.
    assert ora.block_sum_sq(y) == 2.0**24
    # A sequential left-to-right sum would instead give the same here, so also
    # check a case where pairing with a later lane keeps the small terms:
    z = np.zeros(256, np.float32)
    z[1], z[3], z[0] = 1.0, 1.0, 2.0**12
    # offset 2: lane1 + lane3 = 2 (exact); offset 1: lane0 (2^24) + lane1 (2) = 2^24 + 2
    assert ora.block_sum_sq(z) == 2.0**24 + 2.0


# ------------------------------------------------------------ RMSNorm -------
def test_rms_known_answer_from_reference_test():
    # src/gpu.rs:1299-1308: rows [[4,2],[10,5]], weight 1 -> 4/sqrt(10) +- 0.008.
    x = bf16_of([4.0, 2.0, 10.0, 5.0])
    out = f32_of(ora.rms(x, bf16_of([1.0, 1.0]), 2, 2, 1e-6))
    assert abs(out[0, 0] - 1.264911) < 0.008
    assert abs(out[1, 0] - 10 / math.sqrt(62.5)) < 0.008


@pytest.mark.parametrize("hidden", [1024, 1000, 64])
def test_rms_and_add_rms_match_float64_closed_form(hidden):
    rows = 16
    x = ora.normal_bf16((rows, hidden), 11)
    res = ora.normal_bf16((rows, hidden), 12)
    w = ora.normal_bf16(hidden, 13, 1.0, 0.02)
    out = ora.rms(x, w, rows, hidden, 1e-6)
    xf = f32_of(x).astype(np.float64)
    want = xf / np.sqrt((xf**2).mean(axis=1, keepdims=True) + 1e-6) * f32_of(w)
    assert bf16_ulp_diff(out, bf16_of(want)).max() <= 1
    new_res, out2 = ora.add_rms(x, res, w, rows, hidden, 1e-6)
    v = (f32_of(x) + f32_of(res)).astype(np.float32)  # one fp32 add
    assert np.array_equal(new_res, bf16_of(v))  # residual is exact
    vf = v.astype(np.float64)
    want2 = vf / np.sqrt((vf**2).mean(axis=1, keepdims=True) + 1e-6) * f32_of(w)
    assert bf16_ulp_diff(out2, bf16_of(want2)).max() <= 1


# --------------------------------------------------------------- RoPE -------
def test_rope_table_matches_float64_trig_of_the_fp32_angle():
    dim, theta = 128, 1e6
    table = ora.rope_cache(4096, dim, theta, threads=8)
    half = dim // 2
    pair = np.arange(half)
    expo = (-(2 * pair).astype(np.float32) / np.float32(dim)).astype(np.float32)
    inv_freq = np.power(np.float64(theta), expo.astype(np.float64)).astype(np.float32)
    pos = np.arange(4096, dtype=np.float32)[:, None]
    angle = (pos * inv_freq[None, :]).astype(np.float32).astype(np.float64)
    # cos/sin are correctly rounded from float64 except for rare near-ties.
    c_err = np.abs(table[:, :half].astype(np.float64) - np.cos(angle)) / np.spacing(np.float32(1.0))
    s_err = np.abs(table[:, half:].astype(np.float64) - np.sin(angle)) / np.spacing(np.float32(1.0))
    assert c_err.max() <= 1.0 and s_err.max() <= 1.0
    assert table[0, :half].tolist() == [1.0] * half and table[0, half:].tolist() == [0.0] * half


def test_rope_known_answers_and_cached_equals_direct():
    """src/gpu.rs:1246-1289 (cached == direct bytewise at positions 0, 1, 350,
    4095) and src/gpu.rs:1371-1377 (pos 0 -> 1 +- 0.01, pos 1 d0 -> cos1 - sin1)."""
    rows, qh, kvh, dim = 4, 4, 2, 128
    idx = np.arange(rows * (qh + 2 * kvh) * dim)
    qkv = bf16_of(((idx * 17 % 37) - 18.0) / 8.0)
    ones = bf16_of(np.ones(dim))
    pos = np.array([0, 1, 350, 4095], np.int32)
    slots = np.array([0, 1, 2, 3], np.int32)
    kc = np.zeros((1, 4, kvh, dim), np.uint16)
    table = ora.rope_cache(4096, dim, 1e6)
    direct = ora.qkv_rope(qkv, ones, ones, pos, slots, kc, kc, rows, qh, kvh, dim, 4, 1, 1e-6, theta=1e6)
    cached = ora.qkv_rope(qkv, ones, ones, pos, slots, kc, kc, rows, qh, kvh, dim, 4, 1, 1e-6, table=table,
                          max_positions=4096)
    for a, b in zip(direct, cached):
        assert np.array_equal(a, b)
    # Known answers with an all-ones input (src/gpu.rs:1360-1377).
    rows2, qh2, kvh2, d2 = 3, 2, 1, 32
    packed = bf16_of(np.ones(rows2 * (qh2 + 2 * kvh2) * d2))
    w = bf16_of(np.ones(d2))
    pos2 = np.array([0, 1, 2], np.int32)
    sl2 = np.array([2, 3, 0], np.int32)
    cache = np.zeros((2, 2, kvh2, d2), np.uint16)
    q, _, v = ora.qkv_rope(packed, w, w, pos2, sl2, cache, cache, rows2, qh2, kvh2, d2, 2, 2, 1e-6, theta=1e6)
    qf = f32_of(q).reshape(rows2, -1)
    assert np.all(np.abs(qf[0] - 1.0) < 0.01)
    assert abs(qf[1, 0] - (math.cos(1.0) - math.sin(1.0))) < 0.008
    assert f32_of(v).reshape(-1)[0] == 1.0


def test_qkv_rope_matches_float64_formula():
    rows, qh, kvh, dim, bs, blocks = 32, 16, 8, 128, 16, 4
    heads = qh + 2 * kvh
    qkv = ora.normal_bf16((rows, heads, dim), 21)
    qw = ora.normal_bf16(dim, 22, 1.0, 0.02)
    kw = ora.normal_bf16(dim, 23, 1.0, 0.02)
    pos = np.random.default_rng(3).integers(0, 4096, rows).astype(np.int32)
    slots = np.arange(rows, dtype=np.int32)[::-1].copy()
    table = ora.rope_cache(4096, dim, 1e6)
    cache = np.zeros((blocks, bs, kvh, dim), np.uint16)
    q, k, v = ora.qkv_rope(qkv, qw, kw, pos, slots, cache, cache, rows, qh, kvh, dim, bs, blocks, 1e-6, table=table,
                           max_positions=4096)
    x = f32_of(qkv).astype(np.float64)

    def ref(head_block, w):
        inv = 1.0 / np.sqrt((head_block**2).mean(axis=-1, keepdims=True) + 1e-6)
        n = f32_of(bf16_of(head_block * inv * f32_of(w)[None, None, :])).astype(np.float64)
        c = table[pos][:, None, :64].astype(np.float64)
        s = table[pos][:, None, 64:].astype(np.float64)
        lo = n[..., :64] * c - n[..., 64:] * s
        hi = n[..., 64:] * c + n[..., :64] * s
        return np.concatenate([lo, hi], axis=-1)

    q_want = bf16_of(ref(x[:, :qh], qw))
    k_want = bf16_of(ref(x[:, qh:qh + kvh], kw))
    # Rounding the normalised value to bf16 may flip with the last fp32 bit of
    # the norm; allow 1 ulp on the bf16 intermediate (-> a few ulps after a
    # cancelling rotation) but require almost everything to agree exactly.
    dq = bf16_ulp_diff(q, q_want)
    assert np.mean(dq == 0) > 0.995 and dq.max() <= 8
    flat_k = k.reshape(blocks * bs, kvh, dim)[slots]
    dk = bf16_ulp_diff(flat_k, k_want)
    assert np.mean(dk == 0) > 0.995 and dk.max() <= 8
    flat_v = v.reshape(blocks * bs, kvh, dim)[slots]
    assert np.array_equal(flat_v, qkv[:, qh + kvh:])


# --------------------------------------------------------------- SiLU -------
def test_silu_matches_float64_closed_form():
    rows, inter = 64, 3072
    gu = ora.normal_bf16((rows, 2, inter), 31, 0.0, 2.0)
    out = ora.silu(gu, rows, inter, threads=4)
    g = f32_of(gu[:, 0]).astype(np.float64)
    u = f32_of(gu[:, 1]).astype(np.float64)
    want = bf16_of(g / (1.0 + np.exp(-g)) * u)
    assert bf16_ulp_diff(out, want).max() <= 1
    edge = bf16_of(np.array([[[-100.0, 100.0, 0.0, -0.0, -88.0, 88.0, 1e-30, -1e-30],
                              [1.0, 2.0, 3.0, 4.0, 1.0, 1.0, 1.0, 1.0]]]))
    e_out = f32_of(ora.silu(edge, 1, 8)).reshape(-1)
    assert e_out[0] == 0.0 and math.copysign(1.0, e_out[0]) < 0  # -100/(1+e^100) = -0
    assert e_out[1] == f32_of(bf16_of(200.0))
    assert e_out[2] == 0.0 and e_out[3] == 0.0


# ------------------------------------------------------------- copies -------
def test_embedding_gather_and_kv_write_known_answers():
    # src/gpu.rs:1169-1192: tokens [1,3], W = [1,2,3,4] (hidden 1) -> [2,4].
    w = bf16_of([1.0, 2.0, 3.0, 4.0])
    out = ora.embedding(np.array([1, 3], np.int32), w, 2, 1, 4)
    assert f32_of(out).reshape(-1).tolist() == [2.0, 4.0]
    # Out-of-range ids give +0 rows.
    out = ora.embedding(np.array([-1, 4, 0], np.int32), w, 3, 1, 4)
    assert out.reshape(-1).tolist() == [0, 0, w[0]]
    x = np.arange(12, dtype=np.uint16).reshape(4, 3)
    g = ora.gather(x, np.array([3, 0, 7], np.int32), 3, 3, 4)
    assert g.tolist() == [[9, 10, 11], [0, 1, 2], [0, 0, 0]]
    k = np.arange(2 * 2 * 4, dtype=np.uint16).reshape(2, 2, 4)
    v = k + 100
    cache = np.zeros((2, 2, 2, 4), np.uint16)
    kc, vc = ora.kv_write(k, v, np.array([3, 9], np.int32), cache, cache, 2, 2, 4, 2, 2)
    assert np.array_equal(kc.reshape(4, 2, 4)[3], k[0]) and np.array_equal(vc.reshape(4, 2, 4)[3], v[0])
    assert kc.reshape(4, 2, 4)[:3].max() == 0  # slot 9 >= capacity 4 is skipped


# ----------------------------------------------------------- sampling -------
def test_greedy_golden_vectors_from_reference_runs():
    data = np.load(os.path.join(GOLDEN, "reference_logits.npz"))
    logits, expected = data["logits_bf16"], data["expected_greedy"]
    b, v = logits.shape
    temps = np.zeros(b, np.float32)
    seeds = np.zeros(b, np.uint64)
    assert ora.sample(logits, temps, seeds, b, v).tolist() == expected.tolist()
    out, _, _ = ora.sample_partitioned(logits, temps, seeds, b, v, 2048)
    assert out.tolist() == expected.tolist()
    # Row 4 is an exact tie for the maximum; the lower index wins.
    assert expected[4] == 9625
    summary = json.load(open(os.path.join(GOLDEN, "reference_greedy.json")))
    assert len(summary["cases"]) == b == 20
    for case in summary["cases"]:
        assert case["expected_token"] == min(case["argmax_indices"])
        assert expected[case["case"]] == case["expected_token"]


def test_planted_tie_and_partitioned_equals_serial():
    """src/gpu.rs:1194-1244: ties at 2047/2048/4096 straddle partition edges."""
    batch, vocab = 3, 151936
    idx = np.arange(batch * vocab)
    scores = ((idx * 31 % 101) - 50.0) * 0.125
    scores[[2047, 2048, 4096]] = 100.0
    logits = bf16_of(scores).reshape(batch, vocab)
    temps = np.array([0.0, 0.6, 1.0], np.float32)
    seeds = np.array([42, 43, 44], np.uint64)
    serial = ora.sample(logits, temps, seeds, batch, vocab)
    assert serial[0] == 2047
    for width in (2048, 8192, 16384):
        out, _, _ = ora.sample_partitioned(logits, temps, seeds, batch, vocab, width)
        assert out.tolist() == serial.tolist()


def test_sampling_edge_rows():
    vocab = 4096
    nan = float("nan")
    rows = np.stack([
        bf16_of(np.full(vocab, nan)),                       # nothing wins -> 0
        bf16_of(np.full(vocab, -np.inf)),                   # -inf ties -> index 0
        bf16_of(np.where(np.arange(vocab) == 77, np.inf, nan)),
        bf16_of(np.r_[np.full(vocab - 1, -1.0), 5.0]),      # last index
    ])
    temps = np.array([0.0, 0.0, 0.0, 0.0], np.float32)
    seeds = np.zeros(4, np.uint64)
    assert ora.sample(rows, temps, seeds, 4, vocab).tolist() == [0, 0, 77, vocab - 1]
    temps[:] = 0.7
    out = ora.sample(rows, temps, seeds, 4, vocab)
    assert out[0] == 0 and out[2] == 77


# ---------------------------------------------------------- exponential -----
def test_expf_is_faithful_on_the_attention_domain():
    """exp(x) for x <= 0 (scores minus their maximum), subnormal results
    included, within one ulp of binary64 exp; special values."""
    rng = np.random.default_rng(3)
    bits = rng.integers(0x80000000, 0xC2DC0000, size=3_000_000, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([bits.view(np.float32), -np.linspace(0, 110, 1_000_001, dtype=np.float32),
                        np.linspace(0, 88.7, 100_001, dtype=np.float32)])
    got = ora.expf_array(x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    spacing = np.maximum(np.spacing(np.abs(want.astype(np.float32))).astype(np.float64), 2.0**-149)
    assert (np.abs(got - want) / spacing).max() < 1.0
    assert ora.expf(0.0) == 1.0
    assert ora.expf(float("-inf")) == 0.0
    assert math.isnan(ora.expf(float("nan")))
    assert ora.expf(-120.0) == 0.0 and ora.expf(100.0) == float("inf")


# ----------------------------------------------------- paged attention -----
def attention_f64(q, kc, vc, pos, seqs, tables, qh, kvh, dim, bs, blocks, stride, batch, max_context):
    """Softmax attention in binary64 from the contract of
    kernels/kernels.cu:226-270 (no fp32 rounding order)."""
    rows = len(pos)
    qf, kf, vf = (f32_of(a).astype(np.float64) for a in (q, kc, vc))
    qf = qf.reshape(rows, qh, dim)
    kf = kf.reshape(blocks, bs, kvh, dim)
    vf = vf.reshape(blocks, bs, kvh, dim)
    out = np.zeros((rows, qh, dim))
    for r in range(rows):
        ctx = int(pos[r]) + 1
        if not (0 <= seqs[r] < batch) or ctx < 1 or ctx > max_context or ctx > stride * bs:
            continue
        ks, vs = [], []
        for t in range(ctx):
            b = int(tables[seqs[r] * stride + t // bs])
            if 0 <= b < blocks:
                ks.append(kf[b, t % bs])
                vs.append(vf[b, t % bs])
        if not ks:
            continue
        K, V = np.stack(ks), np.stack(vs)
        for h in range(qh):
            s = K[:, h // (qh // kvh)] @ qf[r, h] / math.sqrt(dim)
            p = np.exp(s - s.max())
            out[r, h] = p @ V[:, h // (qh // kvh)] / p.sum()
    return out


def test_attention_known_answers():
    # src/gpu.rs:1330-1362: zero queries, reversed blocks holding V rows 1, 2, 3.
    dim = 32
    v = np.zeros(4 * dim, np.float32)
    v[2 * dim:3 * dim], v[3 * dim:], v[:dim] = 1.0, 2.0, 3.0
    out = ora.attention(np.zeros(3 * 2 * dim, np.uint16), np.zeros(4 * dim, np.uint16), bf16_of(v),
                        np.array([0, 1, 2], np.int32), np.zeros(3, np.int32), np.array([1, 0], np.int32),
                        3, 2, 1, dim, 2, 2, 2, 1, 4)
    for r in range(3):
        assert np.all(f32_of(out[r]) == 1.0 + 0.5 * r)
    # One key: p = 1, den = 1, the output is that key's V row exactly.
    rng = np.random.default_rng(4)
    vrow = bf16_of(rng.normal(size=(1, 1, 1, 64)).astype(np.float32))
    q = bf16_of(rng.normal(size=(1, 1, 64)).astype(np.float32))
    k = bf16_of(rng.normal(size=(1, 1, 1, 64)).astype(np.float32))
    out = ora.attention(q, k, vrow, np.array([0], np.int32), np.array([0], np.int32), np.array([0], np.int32),
                        1, 1, 1, 64, 1, 1, 1, 1, 1)
    assert np.array_equal(out.reshape(-1), vrow.reshape(-1))
    # Equal scores over a constant V column: the mean is the constant exactly.
    vconst = bf16_of(np.tile(np.linspace(-2, 2, 32, dtype=np.float32), 8 * 4))
    out = ora.attention(np.zeros(32, np.uint16), np.zeros(8 * 4 * 32, np.uint16), vconst,
                        np.array([29], np.int32), np.array([0], np.int32), np.arange(4, dtype=np.int32),
                        1, 1, 1, 32, 8, 4, 4, 1, 30)
    assert np.array_equal(out.reshape(-1), vconst[:32])


@pytest.mark.parametrize("dim,bs,qh,kvh", [(128, 256, 16, 8), (64, 16, 4, 1), (80, 3, 6, 2), (32, 2, 3, 3)])
def test_attention_matches_float64_softmax(dim, bs, qh, kvh):
    """Random ragged rows, invalid rows and invalid table entries against the
    binary64 formula; GQA head mapping included."""
    rng = np.random.default_rng(dim + bs)
    batch, stride = 3, -(-600 // bs)
    blocks = batch * stride
    tables = rng.permutation(blocks).astype(np.int32)
    tables[stride + 1] = -1          # a hole in sequence 1
    tables[2 * stride] = blocks + 5  # an out-of-range block in sequence 2
    pos = np.array([0, 5, 599, 300, 17, 4096, 42, 599], np.int32)
    seqs = np.array([0, 1, 2, 1, 0, 0, 7, -1], np.int32)
    rows, max_context = len(pos), 600
    q = ora.normal_bf16((rows, qh, dim), 11 + dim, 0.0, 1.0)
    kc = ora.normal_bf16((blocks, bs, kvh, dim), 12 + dim, 0.0, 1.0)
    vc = ora.normal_bf16((blocks, bs, kvh, dim), 13 + dim, 0.0, 1.0)
    got = f32_of(ora.attention(q, kc, vc, pos, seqs, tables, rows, qh, kvh, dim, bs, blocks, stride, batch,
                               max_context, threads=4)).astype(np.float64)
    want = attention_f64(q, kc, vc, pos, seqs, tables, qh, kvh, dim, bs, blocks, stride, batch, max_context)
    assert np.all(np.abs(got - want) <= 2.0**-8 * np.abs(want) + 2.0**-16)
    assert np.all(got[5:] == 0.0)  # context above max_context, seq out of range, negative seq
