"""nv_sample_parallel_static (no allocation: the partials live in the
library's static device array) against nv_sample_parallel with caller scratch,
through the C ABI: two calls in a row, the second with a smaller batch, so the
second call runs over partials the first one left behind; and the size limit
is refused with an error before any launch."""
import numpy as np
import pytest

import nvr
import oracle as ora

pytestmark = pytest.mark.gpu


def _batch(batch, vocab, seed):
    logits = ora.normal_bf16((batch, vocab), seed, 0.0, 3.0)
    temps = np.array([(0.0, 0.6, 1.3)[r % 3] for r in range(batch)], np.float32)
    seeds = np.array([ora.sampling_seed(seed, r, r % 7) for r in range(batch)], np.uint64)
    return logits, temps, seeds


def _both(gpu, logits, temps, seeds, batch, vocab):
    lb, tb, sb = (gpu.upload_array(np.ascontiguousarray(a)) for a in (logits, temps, seeds))
    parts = -(-vocab // 2048)
    ps, pi = gpu.alloc(batch * parts * 4), gpu.alloc(batch * parts * 4)
    out_scratch, out_static = gpu.alloc(batch * 4), gpu.alloc(batch * 4)
    gpu.sample_parallel(lb, tb, sb, out_scratch, ps, pi, batch, vocab)
    gpu.sample_parallel_static(lb, tb, sb, out_static, batch, vocab)
    return out_scratch.download(np.int32, batch), out_static.download(np.int32, batch)


@pytest.mark.parametrize("first,second", [((300, 151936), (40, 151936)), ((64, 151936), (3, 10001))])
def test_static_partials_match_caller_scratch(first, second):
    gpu = nvr.Gpu(0)
    for i, (batch, vocab) in enumerate((first, second)):
        print(f"static sampler call {i}: batch {batch}, vocab {vocab}", flush=True)
        logits, temps, seeds = _batch(batch, vocab, 900 + i + batch)
        want = ora.sample(logits, temps, seeds, batch, vocab, threads=8)
        got_scratch, got_static = _both(gpu, logits, temps, seeds, batch, vocab)
        assert got_static.tolist() == got_scratch.tolist()
        assert got_static.tolist() == want.tolist()


def test_static_partials_limit_is_refused():
    gpu = nvr.Gpu(0)
    vocab = 151936
    batch = nvr.Gpu.STATIC_PARTIALS // 75 + 1  # one row past 131072 partials
    lb = gpu.alloc(batch * vocab * 2)
    tb, sb, ob = gpu.alloc(batch * 4), gpu.alloc(batch * 8), gpu.alloc(batch * 4)
    with pytest.raises(nvr.BackendError, match="static scratch"):
        gpu.sample_parallel_static(lb, tb, sb, ob, batch, vocab)
    # The largest batch that fits runs.
    ok = nvr.Gpu.STATIC_PARTIALS // 75
    gpu.sample_parallel_static(lb, tb, sb, ob, ok, vocab)
    gpu.sync()


def test_static_partials_filled_to_the_limit():
    """A batch that fills the static array exactly (16 rows of 8192 partitions
    of 2048 tokens: 131072 partials, written by the one-pass partition path),
    each row's winner planted in its last partition so the top entries of
    both halves of the array decide the result; then a smaller call."""
    gpu = nvr.Gpu(0)
    batch, vocab = 16, 8191 * 2048 + 8
    assert batch * -(-vocab // 2048) == nvr.Gpu.STATIC_PARTIALS
    print(f"static sampler at the limit: batch {batch}, vocab {vocab}", flush=True)
    logits = np.random.default_rng(950).integers(0x3C00, 0x4000, size=(batch, vocab), dtype=np.uint16)
    planted = vocab - 1 - 37 * np.arange(batch)
    logits[np.arange(batch), planted] = 0x4300  # 128.0: wins greedy and Gumbel (T = 0.6) rows alike
    temps = np.array([0.0, 0.6] * (batch // 2), np.float32)
    seeds = np.array([ora.sampling_seed(950, r, r) for r in range(batch)], np.uint64)
    got_scratch, got_static = _both(gpu, logits, temps, seeds, batch, vocab)
    del logits
    assert got_static.tolist() == got_scratch.tolist() == planted.tolist()
    small, temps2, seeds2 = _batch(3, 151936, 951)
    got_scratch, got_static = _both(gpu, small, temps2, seeds2, 3, 151936)
    assert got_static.tolist() == got_scratch.tolist() == ora.sample(small, temps2, seeds2, 3, 151936).tolist()
