"""Parity at BASELINE scale: the 60-workload study grid (config 4) and the
long-sequence stress (config 5), both against the FP64 oracle.

Grid: B in {1,2,4} x N in {512..8192} x D in {64,128} x {dense, causal}, H=8,
Q/K/V uniform[-1,1) reseeded per shape. The reference checks only finiteness
at grid scale (benchmarks/bench_flash_attention.cu:673-683); here every output
row of every case goes through the full tolerance gate against the FP64
oracle (benchmarks/bench_flash_attention.cu:167-218 compares every element),
and every element is checked finite after a NaN prefill.

Stress: (1,16,16384,128) causal with Q, K ~ N(0, 3^2) so logits exceed 50 and
the online-softmax rescale is exercised; V uniform. Every row is checked; the
test also asserts that the inputs do reach |s| > 50.
"""
import numpy as np
import pytest

from gpu_common import HOST_THREADS, from_dev, kernels_for, run, say, to_dev

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

GRID = [(b, 8, n, d, c) for b in (1, 2, 4) for n in (512, 1024, 2048, 4096, 8192) for d in (64, 128)
        for c in (False, True)]


@pytest.fixture(scope="module")
def fa(fa_lib):
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    return fa_lib


def grid_seeds(B, N, D):
    base = 1000 * B + 10 * (N // 512) + D
    return {"q": 11 + base, "k": 22 + base, "v": 33 + base}


@pytest.mark.parametrize("B", [1, 2, 4])
@pytest.mark.parametrize("D", [64, 128])
def test_grid_tolerance(fa, oracle_mod, B, D):
    fails = []
    for (b, H, N, d, causal) in GRID:
        if b != B or d != D:
            continue
        qb, kb, vb = oracle_mod.make_inputs(B, H, N, D, seeds=grid_seeds(B, N, D))
        ref = oracle_mod.attention(qb, kb, vb, causal, threads=HOST_THREADS).reshape(-1, D)
        q, k, v = to_dev(qb), to_dev(kb), to_dev(vb)
        for kernel in kernels_for(D):
            say("grid", kernel, B, H, N, D, causal)
            out = from_dev(run(fa, kernel, q, k, v, causal)).reshape(-1, D)
            # every element of the output must be finite (NaN prefill)
            n_bad = int(np.count_nonzero((out & 0x7F80) == 0x7F80))
            acc = oracle_mod.compare(out, ref)
            print(f"{kernel} {(B, H, N, D, causal)} rows checked {out.shape[0]}/{B * H * N} ulp={acc.ulp:.2f} "
                  f"gate={acc.abs_gate:.3f} nonfinite={n_bad}")
            if not acc.passed or n_bad:
                fails.append((kernel, N, causal, n_bad, acc))
        del q, k, v
    assert not fails, fails


def causal_row_max_logit(qf, kf, scale, chunk=2048):
    """max over visible keys of |scale * q.k| for every query row of one slab
    (float32 products of the bf16 inputs; an input property, not a result)."""
    n = qf.shape[0]
    out = np.empty(n, dtype=np.float32)
    cols = np.arange(n)[None, :]
    for r0 in range(0, n, chunk):
        s = np.abs(qf[r0:r0 + chunk] @ kf.T)
        s = np.where(cols <= np.arange(r0, r0 + chunk)[:, None], s, 0.0)
        out[r0:r0 + chunk] = s.max(axis=1) * scale
    return out


def test_long_sequence_stress(fa, oracle_mod):
    B, H, N, D = 1, 16, 16384, 128
    qb, kb, vb = oracle_mod.make_inputs(B, H, N, D, "stress")
    # Logits reach |s| > 50 (logit std ~9 at sigma 3, D 128): an input
    # property, checked on head 0.
    row_max = causal_row_max_logit(oracle_mod.bf16_to_f32(qb[0, 0]), oracle_mod.bf16_to_f32(kb[0, 0]),
                                   oracle_mod.default_scale(D))
    assert row_max.max() > 50, row_max.max()
    ref = oracle_mod.attention(qb, kb, vb, True, threads=HOST_THREADS).reshape(-1, D)
    q, k, v = to_dev(qb), to_dev(kb), to_dev(vb)
    for kernel in kernels_for(D):
        say("stress", kernel)
        out = from_dev(run(fa, kernel, q, k, v, True)).reshape(-1, D)
        assert int(np.count_nonzero((out & 0x7F80) == 0x7F80)) == 0
        acc = oracle_mod.compare(out, ref)
        print(f"stress {kernel} rows checked {out.shape[0]}/{B * H * N} ulp={acc.ulp:.2f} gate={acc.abs_gate:.3f} "
              f"max_abs={acc.max_abs:.3e}")
        assert acc.passed, (kernel, acc)
