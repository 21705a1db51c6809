"""Seeded random shapes and a sweep of sequence lengths, against the FP64 oracle
through the C ABI, every row compared (the comparator of
benchmarks/bench_flash_attention.cu:183-213 plus BASELINE's 2^-7 row gate).

The fixed cases elsewhere sit on tile multiples, the reference's boundary set
(N <= 256) and the grid (multiples of 512). Here the lengths fall anywhere up
to a few thousand keys, so the tail tile, the split of the key range between
wave groups, the paired causal layout's half blocks and the list layout's
crossing group all land at positions the fixed cases do not reach. Both sets
are drawn once from fixed seeds, so a failure names a reproducible case.
"""
import numpy as np
import pytest

from gpu_common import HOST_THREADS, kernels_for, run_bits, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fa(fa_lib):
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    return fa_lib


def random_shapes(count, seed):
    """(B, H, N, D, causal): B 1-3, H 1-5; N log-uniform in [1, 256) for a
    third of the shapes, uniform in [256, 2600] for the rest."""
    rng = np.random.default_rng(seed)
    shapes = []
    for i in range(count):
        n = int(np.exp(rng.uniform(0.0, np.log(256.0)))) if i % 3 == 0 else int(rng.integers(256, 2601))
        shapes.append((int(rng.integers(1, 4)), int(rng.integers(1, 6)), max(1, n), int(rng.choice([64, 128])),
                       bool(rng.integers(0, 2))))
    return shapes


RANDOM_SHAPES = random_shapes(30, seed=20261202)


def test_random_shapes(fa, oracle_mod):
    """Every kernel that supports the head dim (v0 and each fused
    configuration) on each shape; inputs uniform [-1, 1) from per-shape seeds."""
    for idx, (B, H, N, D, causal) in enumerate(RANDOM_SHAPES):
        q, k, v = oracle_mod.make_inputs(B, H, N, D, seeds={"q": 100 + idx, "k": 200 + idx, "v": 300 + idx})
        ref = oracle_mod.attention(q, k, v, causal, threads=HOST_THREADS)
        for kernel in kernels_for(D):
            say("random shape", idx, kernel, B, H, N, D, causal)
            acc = oracle_mod.compare(run_bits(fa, kernel, q, k, v, causal), ref)
            assert acc.passed, f"random shape {idx} {kernel} {(B, H, N, D, causal)}: {acc}"


# One slab pair at head_dim 64: every length gives a one-round grid, so the
# list layout pairs half blocks; the crossing group and its step move with N.
LIST_SWEEP_N = [33, 97, 160, 255, 300, 511, 700, 777, 1023, 1100, 1234, 1500, 1537, 1663, 1777, 1888, 1999,
                2047, 2111, 2300, 2500, 2600]


def test_list_layout_length_sweep(fa, oracle_mod):
    """The four-group list layout (pinned) and the v3 default, causal and
    dense, at 22 lengths between 33 and 2600."""
    for N in LIST_SWEEP_N:
        q, k, v = oracle_mod.make_inputs(1, 2, N, 64, seeds={"q": N, "k": N + 1, "v": N + 2})
        for causal in (True, False):
            ref = oracle_mod.attention(q, k, v, causal, threads=HOST_THREADS)
            for kernel in ("v3_128x4", "v3_mfma"):
                say("list sweep", kernel, N, causal)
                acc = oracle_mod.compare(run_bits(fa, kernel, q, k, v, causal), ref)
                assert acc.passed, f"list sweep {kernel} N={N} causal={causal}: {acc}"


def random_scales(count, seed):
    """(B, H, N, D, causal, a, b, c): Q, K and V scaled by 2^a, 2^b and 2^c.
    a + b <= 8 keeps the logits within a few hundred (beyond that, fp32 score
    rounding alone moves the softmax and no fp32 kernel matches the FP64
    oracle); c spans 2^-120 to 2^60, inside the fused kernels' documented
    range (P may grow to 2^48 between base moves)."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(count):
        a = int(rng.integers(-30, 9))
        b = int(rng.integers(-30, 9 - a)) if a < 8 else int(rng.integers(-30, 1))
        cases.append((1, int(rng.integers(1, 4)), int(rng.integers(1, 700)), int(rng.choice([64, 128])),
                      bool(rng.integers(0, 2)), a, b, int(rng.integers(-120, 61))))
    return cases


RANDOM_SCALES = random_scales(40, seed=20261203)


def test_random_scales(fa, oracle_mod):
    """Seeded random shapes with random power-of-two scales on Q, K and V:
    logits from vanishing to a few hundred, V over 180 binary orders of
    magnitude. Every kernel, every row against the oracle."""
    for idx, (B, H, N, D, causal, a, b, c) in enumerate(RANDOM_SCALES):
        q, k, v = oracle_mod.make_inputs(B, H, N, D, seeds={"q": 400 + idx, "k": 500 + idx, "v": 600 + idx})
        qf, kf, vf = (oracle_mod.bf16_to_f32(x).astype(np.float64) for x in (q, k, v))
        q, k, v = (oracle_mod.bf16_bits(x * 2.0 ** e) for x, e in ((qf, a), (kf, b), (vf, c)))
        ref = oracle_mod.attention(q, k, v, causal, threads=HOST_THREADS)
        for kernel in kernels_for(D):
            say("random scales", idx, kernel, B, H, N, D, causal, a, b, c)
            acc = oracle_mod.compare(run_bits(fa, kernel, q, k, v, causal), ref)
            assert acc.passed, f"random scales {idx} {kernel} {(B, H, N, D, causal, a, b, c)}: {acc}"


def rising_logits(count, seed):
    """(B, H, N, D, causal, a, r, c, ramp): Q scaled by 2^a, key j scaled by
    ramp(j) rising from 1 to r along the sequence (linear, quadratic, or a
    step over the last quarter of the keys), V by 2^c. A row's maximum then
    keeps growing as the walk proceeds, by up to a few hundred log2 units, so
    the fused kernels move their exponent base several times per row, at
    positions that depend on the shape. a + log2 r <= 8 keeps the logits
    well conditioned in fp32 (as for the random scales)."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(count):
        a = int(rng.integers(-4, 5))
        r = float(2.0 ** rng.uniform(0, 8 - max(a, 0)))
        cases.append((int(rng.integers(1, 3)), int(rng.integers(1, 3)), int(rng.integers(2, 1500)),
                      int(rng.choice([64, 128])), bool(rng.integers(0, 2)), a, r, int(rng.integers(-100, 41)),
                      str(rng.choice(["linear", "square", "late"]))))
    return cases


RISING_LOGITS = rising_logits(30, seed=20261204)


def test_rising_logits(fa, oracle_mod):
    """Seeded random shapes whose logits rise along the key sequence (the
    exponent-base moves and their tile recomputation at shape-dependent
    positions), with V scaled from 2^-100 to 2^40. Every kernel, every row
    against the oracle."""
    for idx, (B, H, N, D, causal, a, r, c, kind) in enumerate(RISING_LOGITS):
        q, k, v = oracle_mod.make_inputs(B, H, N, D, seeds={"q": 700 + idx, "k": 800 + idx, "v": 900 + idx})
        qf, kf, vf = (oracle_mod.bf16_to_f32(x).astype(np.float64) for x in (q, k, v))
        t = np.arange(N, dtype=np.float64) / max(N - 1, 1)
        ramp = {"linear": 1 + (r - 1) * t, "square": 1 + (r - 1) * t * t, "late": np.where(t > 0.75, r, 1.0)}[kind]
        q = oracle_mod.bf16_bits(qf * 2.0 ** a)
        k = oracle_mod.bf16_bits(kf * ramp[None, None, :, None])
        v = oracle_mod.bf16_bits(vf * 2.0 ** c)
        ref = oracle_mod.attention(q, k, v, causal, threads=HOST_THREADS)
        for kernel in kernels_for(D):
            say("rising logits", idx, kernel, B, H, N, D, causal, a, round(r, 2), c, kind)
            acc = oracle_mod.compare(run_bits(fa, kernel, q, k, v, causal), ref)
            assert acc.passed, f"rising logits {idx} {kernel} {(B, H, N, D, causal, a, r, c, kind)}: {acc}"
