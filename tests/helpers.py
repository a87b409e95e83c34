"""Shared helpers for the parity tests."""
import numpy as np


def ordered(bits) -> np.ndarray:
    """bf16 bit patterns -> integers monotone in value (+0 and -0 both map to 0)."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.int64)
    mag = b & 0x7FFF
    return np.where(b & 0x8000, -mag, mag)


def bf16_ulp_diff(a, b) -> np.ndarray:
    """Distance in bf16 ulps between two arrays of bf16 bit patterns (NaN vs NaN = 0)."""
    a = np.asarray(a, dtype=np.uint16)
    b = np.asarray(b, dtype=np.uint16)
    nan_a = (a & 0x7FFF) > 0x7F80
    nan_b = (b & 0x7FFF) > 0x7F80
    d = np.abs(ordered(a) - ordered(b))
    d = np.where(nan_a & nan_b, 0, d)
    return np.where(nan_a ^ nan_b, 1 << 20, d)


def bf16_of(x) -> np.ndarray:
    """float64/float32 values -> bf16 bits, rounding once from float32."""
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    return np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r).astype(np.uint16)


def f32_of(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def unique_slots(rows: int, bs: int, blocks: int, seed: int) -> np.ndarray:
    """slot = perm[t // bs] * bs + t % bs over a random permutation of blocks
    (src/runtime.rs:747-755 with one sequence per block)."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(blocks)
    t = np.arange(rows)
    return (perm[t // bs] * bs + t % bs).astype(np.int32)


def assert_bits_equal(got, want, name: str = "") -> None:
    """Bit-exact comparison that reports how many elements differ and by how much."""
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, f"{name}: shape {got.shape} != {want.shape}"
    bad = got != want
    if not bad.any():
        return
    n = int(bad.sum())
    first = np.argwhere(bad)[0].tolist()
    detail = ""
    if got.dtype == np.uint16:
        d = bf16_ulp_diff(got, want)
        detail = f", max {int(d.max())} bf16 ulp, {int((d > 1).sum())} beyond 1 ulp"
    raise AssertionError(f"{name}: {n} of {got.size} differ{detail}; first at {first}: "
                         f"got {got[tuple(first)]!r} want {want[tuple(first)]!r}")
