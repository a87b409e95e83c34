"""The benchmark's composed step (bench.Chain) against the oracle, end to end.

The step is the fused-kernel chain of a Qwen3-0.6B forward in the order of
src/model.rs:649-789: embedding into the residual stream; layer 0's RMSNorm,
later layers' residual-add + RMSNorm of the previous MLP output; q/k norm +
RoPE + paged KV write into that layer's own caches; the post-attention
add-RMSNorm; SiLU·up; and the final add-RMSNorm. The GEMM and attention outputs
that feed it are seeded synthetic tensors, exactly as in the benchmark.

The step is captured as one HIP graph (as bench.py times it) and replayed
several times, with eager work and host synchronisations between replays.
After every replay each observable output is compared with the oracle run
through the same chain on the CPU, on the inputs downloaded from the device:
the residual stream and the final norm's output, the last layer's rotated q,
every layer's K and V cache bit for bit, and SiLU's output within 1 bf16 ulp.
"""
import os
import sys

import numpy as np
import pytest

import oracle as ora
from helpers import assert_bits_equal, bf16_ulp_diff

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402

pytestmark = pytest.mark.gpu


def _down(buf, dtype, shape):
    return buf.download(dtype, int(np.prod(shape))).reshape(shape)


def _oracle_step(chain, threads=8):
    """The chain's inputs, downloaded, through the oracle in the step's order.
    Returns (residual, normed, query, act, [(kcache, vcache) per layer])."""
    T, H, I, QH, KVH, D, V = chain.T, bench.H, bench.I, bench.QH, bench.KVH, bench.D, bench.V
    heads, bs, blocks = bench.HEADS, bench.BS, chain.blocks
    tok = _down(chain.tok, np.int32, (T,))
    table = _down(chain.table, np.uint16, (V, H))
    pos = _down(chain.pos, np.int32, (T,))
    slots = _down(chain.slots, np.int32, (T,))
    rope = _down(chain.rope, np.float32, (bench.MAX_POS, D))
    assert np.array_equal(rope, ora.rope_cache(bench.MAX_POS, D, bench.THETA, threads)), "rope table"
    eps = bench.EPS
    res = ora.embedding(tok, table, T, H, V, threads)
    del table
    caches = []
    query = act = normed = None
    mlp_prev = None
    zero = np.zeros((blocks, bs, KVH, D), np.uint16)
    for i, l in enumerate(chain.layers):
        in_norm = _down(l["in_norm"], np.uint16, (H,))
        if i == 0:
            normed = ora.rms(res, in_norm, T, H, eps, threads)
        else:
            res, normed = ora.add_rms(mlp_prev, res, in_norm, T, H, eps, threads)
        qkv = _down(l["qkv"], np.uint16, (T, heads, D))
        qn, kn = _down(l["q_norm"], np.uint16, (D,)), _down(l["k_norm"], np.uint16, (D,))
        query, kc, vc = ora.qkv_rope(qkv, qn, kn, pos, slots, zero, zero, T, QH, KVH, D, bs, blocks, eps, table=rope,
                                     max_positions=bench.MAX_POS, threads=threads)
        caches.append((kc, vc))
        attn = _down(l["attn_out"], np.uint16, (T, H))
        res, normed = ora.add_rms(attn, res, _down(l["post_norm"], np.uint16, (H,)), T, H, eps, threads)
        act = ora.silu(_down(l["gate_up"], np.uint16, (T, 2, I)), T, I, threads)
        mlp_prev = _down(l["mlp_out"], np.uint16, (T, H))
    res, normed = ora.add_rms(mlp_prev, res, _down(chain.final_norm, np.uint16, (H,)), T, H, eps, threads)
    return res, normed, query, act, caches


def _check(chain, want, label):
    T, H, I, QH, KVH, D = chain.T, bench.H, bench.I, bench.QH, bench.KVH, bench.D
    res, normed, query, act, caches = want
    assert_bits_equal(_down(chain.residual, np.uint16, (T, H)), res, f"{label}: residual stream")
    assert_bits_equal(_down(chain.normed, np.uint16, (T, H)), normed, f"{label}: final norm output")
    assert_bits_equal(_down(chain.query, np.uint16, (T, QH, D)), query, f"{label}: last layer's rotated q")
    for i, (l, (kc, vc)) in enumerate(zip(chain.layers, caches)):
        assert_bits_equal(_down(l["kc"], np.uint16, kc.shape), kc, f"{label}: layer {i} K cache")
        assert_bits_equal(_down(l["vc"], np.uint16, vc.shape), vc, f"{label}: layer {i} V cache")
    d = bf16_ulp_diff(_down(chain.act, np.uint16, (T, I)), act)
    assert int(d.max()) <= 1, f"{label}: SiLU output {int(d.max())} bf16 ulp from the oracle"


def _clear(chain):
    """Zero every output the step writes, so a replay has to rewrite all of them."""
    for buf in [chain.residual, chain.normed, chain.query, chain.act] + [l[k] for l in chain.layers
                                                                        for k in ("kc", "vc")]:
        buf.upload(np.zeros(buf.bytes, np.uint8))


@pytest.mark.parametrize("tokens,layers", [(512, 3), (8192, 2)])
def test_composed_step_graph_matches_oracle_chain(gpu, tokens, layers):
    print(f"composed step: T={tokens}, {layers} layers", flush=True)
    hip = bench.Hip()
    fill = bench.Filler(gpu, hip)
    chain = bench.Chain(gpu, fill, tokens, layers, seed=tokens + layers)
    gpu.sync()
    want = _oracle_step(chain)
    graph = gpu.capture(chain.step)
    for replay in range(3):
        _clear(chain)
        graph.replay()
        gpu.sync()
        _check(chain, want, f"replay {replay}")
        # Unrelated eager work between replays (the step's own kernels on other buffers).
        scratch = gpu.alloc(tokens * bench.H * 2)
        gpu.rms_norm(chain.normed, chain.final_norm, scratch, tokens, bench.H, bench.EPS)
        gpu.sync()


def test_composed_step_eager_matches_oracle_chain(gpu):
    """The same chain launched eagerly (no graph), 2 layers at 1024 tokens."""
    hip = bench.Hip()
    chain = bench.Chain(gpu, bench.Filler(gpu, hip), 1024, 2, seed=77)
    gpu.sync()
    want = _oracle_step(chain)
    _clear(chain)
    chain.step()
    gpu.sync()
    _check(chain, want, "eager")
