"""GPU parity of the HIP path against the FP64 oracle, through the C ABI.

Gate (BASELINE + the reference's comparator, benchmarks/bench_flash_attention.cu:
159-163,183-213): every output finite, row-scale ULP <= 2, and
|O - O_ref| <= 2^-7 * max|O_ref row|. Both are checked by oracle.compare().
Cases: BASELINE config 1, the reference's own accuracy shapes and inputs,
the committed golden fixture, the boundary-N x input-family matrix of
kernels/ablation/experiments.cu:283-295 plus the lite N set
(benchmarks/bench_flash_attention_lite.cu:48), determinism, v3/v3b agreement,
the v0 profile API's bitwise equality (benchmarks/profile_attention_v0.cu:98-122),
the standalone softmax, and the error paths.
"""
import hashlib
import os

import numpy as np
import pytest

from gpu_common import (FUSED_KERNELS, HOST_THREADS, KERNELS, from_dev, kernels_for, nan_like, run, run_bits, say,
                        supports, to_dev)

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def fa(fa_lib):
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    return fa_lib


def check(oracle, got_bits, ref, what):
    acc = oracle.compare(got_bits, ref)
    assert acc.passed, f"{what}: {acc}"
    return acc


@pytest.mark.parametrize("kernel", KERNELS)
def test_config1_uniform_dense(fa, oracle_mod, kernel):
    say("config1", kernel)
    q, k, v = oracle_mod.make_inputs(1, 2, 128, 64)
    ref = oracle_mod.attention(q, k, v, False)
    got = run_bits(fa, kernel, q, k, v, False)
    check(oracle_mod, got, ref, f"c1 {kernel}")


@pytest.mark.parametrize("kernel", KERNELS)
def test_golden_fixture(fa, oracle_mod, kernel):
    g = np.load(os.path.join(HERE, "golden", "c1_uniform_dense.npz"))
    B, H, N, D = (int(x) for x in g["shape"])
    q, k, v = oracle_mod.make_inputs(B, H, N, D)
    for name, arr in (("q", q), ("k", k), ("v", v)):
        assert hashlib.sha256(arr.tobytes()).hexdigest() == str(g[f"sha_{name}"])
    say("golden", kernel)
    got = run_bits(fa, kernel, q, k, v, False)
    check(oracle_mod, got, g["o_ref"], f"golden {kernel}")


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_reference_accuracy_shapes(fa, oracle_mod, kernel, head_dim, causal):
    """The reference's accuracy suite: (1,2,256,D), its own mt19937 normal inputs."""
    if not supports(kernel, head_dim):
        pytest.skip(f"{kernel} has no head_dim {head_dim} configuration")
    q, k, v = oracle_mod.make_inputs(1, 2, 256, head_dim, "normal_mt19937")
    ref = oracle_mod.attention(q, k, v, causal)
    say("refacc", kernel, head_dim, causal)
    acc = check(oracle_mod, run_bits(fa, kernel, q, k, v, causal), ref, f"refacc {kernel}")
    print(f"{kernel} D={head_dim} causal={causal} vs_double={acc.vs_double:.4e} row_scaled={acc.row_scaled:.4e} "
          f"max_abs={acc.max_abs:.4e} ulp={acc.ulp:.2f}")


BOUNDARY_N = [1, 7, 8, 9, 31, 32, 33, 63, 64, 65, 127, 128, 129, 256]
# BASELINE-style families on uniform inputs, then the reference's own five
# (kernels/ablation/experiments.cu:283-289: normal(0,1) mt19937 base,
# Q=K=V=0, all ones, a ramp V over normal Q/K, normal Q/K x4).
FAMILIES = ["uniform", "zeros", "ones", "ramp", "scaled", "ref_normal", "ref_zeros", "ref_ramp", "ref_scaled"]


@pytest.mark.parametrize("family", FAMILIES)
@pytest.mark.parametrize("kernel", KERNELS)
def test_boundary_matrix(fa, oracle_mod, kernel, family):
    fails = []
    for n in BOUNDARY_N:
        for d in (64, 128):
            if not supports(kernel, d):
                continue
            q, k, v = oracle_mod.make_inputs(1, 2, n, d, family)
            for causal in (False, True):
                ref = oracle_mod.attention(q, k, v, causal, threads=HOST_THREADS)
                say("boundary", kernel, family, n, d, causal)
                acc = oracle_mod.compare(run_bits(fa, kernel, q, k, v, causal), ref)
                if not acc.passed:
                    fails.append((n, d, causal, acc))
    assert not fails, fails


def test_multi_slab_ragged(fa, oracle_mod):
    """Several (b,h) slabs with a partial last query block and partial KV tile."""
    for (B, H, N, D) in [(2, 3, 200, 64), (3, 1, 333, 128), (1, 5, 65, 128)]:
        q, k, v = oracle_mod.make_inputs(B, H, N, D, seeds={"q": 5, "k": 6, "v": 7})
        for causal in (False, True):
            ref = oracle_mod.attention(q, k, v, causal, threads=HOST_THREADS)
            for kernel in kernels_for(D):
                say("ragged", kernel, B, H, N, D, causal)
                check(oracle_mod, run_bits(fa, kernel, q, k, v, causal), ref, f"ragged {kernel} {(B, H, N, D, causal)}")


def test_causal_work_layouts(fa, oracle_mod):
    """Causal grids that fit one round on the device pair an early and a late
    half block per workgroup; larger grids keep whole blocks issued heaviest
    first. Both layouts, with even and odd half-block counts (an odd count
    leaves the middle half block without a partner), against the oracle."""
    cases = [
        (1, 300, 192, 64),   # 300 slabs: more workgroups than CUs -> whole blocks
        (2, 4, 1000, 128),   # one round -> pairs; 16 half blocks of 64 rows (v3)
        (1, 3, 1100, 64),    # one round -> pairs; 18 half blocks (v3), 35 (v3b): odd
        (1, 1, 2049, 128),   # one slab, tail row in its own half block
    ]
    for (B, H, N, D) in cases:
        q, k, v = oracle_mod.make_inputs(B, H, N, D, seeds={"q": 41, "k": 42, "v": 43})
        ref = oracle_mod.attention(q, k, v, True, threads=HOST_THREADS)
        for kernel in kernels_for(D, FUSED_KERNELS):
            say("causal layout", kernel, B, H, N, D)
            check(oracle_mod, run_bits(fa, kernel, q, k, v, True), ref, f"causal layout {kernel} {(B, H, N, D)}")


def growing_logit_inputs(oracle_mod, B, H, N, D, seed, top=60.0):
    """Q ~ 0.5 + noise, K rows growing linearly along the sequence: every
    query's logits rise key after key, to about `top` at the last key. The
    fused kernels move their exponent base to the row max when a tile's row
    sum passes 2^48, so a move follows about every 44-48 log2 units (about
    31 natural) of growth: `top` 60 moves it about twice per row, `top` 500
    on every tile at N 256 and about every second tile at N 1000. The same
    keys in falling order (largest first) never move it."""
    rng = np.random.default_rng(seed)
    kappa = 2.0 * top / np.sqrt(D)  # scale * D * 0.5 * kappa = top at the last key
    ramp = kappa * np.arange(N, dtype=np.float64) / N
    q = 0.5 + 0.05 * rng.standard_normal((B, H, N, D))
    k = ramp[None, None, :, None] + 0.25 * rng.standard_normal((B, H, N, D))
    v = rng.uniform(-1.0, 1.0, (B, H, N, D))
    return (oracle_mod.bf16_bits(q), oracle_mod.bf16_bits(k), oracle_mod.bf16_bits(v))


def test_base_moves(fa, oracle_mod):
    """Inputs whose row max keeps growing (the exponent base moves once or
    twice per row, or on most tiles for the steep ramp), the same keys in
    falling order (it never moves after the first tile), and N(0, 3^2)
    logits at a short length: all against the oracle, dense and causal,
    every fused configuration, both head dims."""
    for D in (64, 128):
        for N in (256, 1000):
            q, k, v = growing_logit_inputs(oracle_mod, 1, 2, N, D, seed=N + D)
            cases = [("growing", q, k, v), ("falling", q, k[:, :, ::-1].copy(), v[:, :, ::-1].copy())]
            cases.append(("steep",) + growing_logit_inputs(oracle_mod, 1, 2, N, D, seed=N + D + 1, top=500.0))
            cases.append(("stress",) + tuple(oracle_mod.make_inputs(1, 2, N, D, "stress")))
            for name, qq, kk, vv in cases:
                for causal in (False, True):
                    ref = oracle_mod.attention(qq, kk, vv, causal, threads=HOST_THREADS)
                    for kernel in kernels_for(D, FUSED_KERNELS):
                        say("base moves", name, kernel, N, D, causal)
                        check(oracle_mod, run_bits(fa, kernel, qq, kk, vv, causal), ref,
                              f"base moves {name} {kernel} {(N, D, causal)}")


def test_value_range(fa, oracle_mod):
    """V scaled across bf16's range (2^-120, subnormal 2^-130, 2^100, 2^115),
    Q and K scaled to subnormals or to opposite extremes, and Q and K both
    scaled by 2^12 to 2^56 (scores up to about 2^118), against the oracle,
    every kernel, both head dims and masks. The softmax weights do not
    depend on V's scale, so the V cases exercise the P V products at the
    edges of fp32: the fused kernels keep P <= 1 outside base moves, so
    their products neither underflow for tiny V nor overflow for huge V.
    Large Q and K push the exponent base past 2^28, where the fused
    exponent's exact product minus the rounded base loses the row max, and
    below the old empty-row sentinel; those waves recompute every tile from
    rounded products, also when the huge scores only start mid-walk (one
    key, or the last quarter of the keys)."""
    B, H, N = 1, 2, 300
    for D in (64, 128):
        q, k, v = oracle_mod.make_inputs(B, H, N, D, seeds={"q": 1, "k": 2, "v": 3})
        qf, kf, vf = (oracle_mod.bf16_to_f32(x).astype(np.float64) for x in (q, k, v))
        cases = [("v 2^-120", q, k, oracle_mod.bf16_bits(vf * 2.0 ** -120)),
                 ("v 2^-130", q, k, oracle_mod.bf16_bits(vf * 2.0 ** -130)),
                 ("v 2^100", q, k, oracle_mod.bf16_bits(vf * 2.0 ** 100)),
                 ("v 2^115", q, k, oracle_mod.bf16_bits(vf * 2.0 ** 115)),
                 ("qk 2^-130", oracle_mod.bf16_bits(qf * 2.0 ** -130), oracle_mod.bf16_bits(kf * 2.0 ** -130), v),
                 ("q 2^100 k 2^-128", oracle_mod.bf16_bits(qf * 2.0 ** 100), oracle_mod.bf16_bits(kf * 2.0 ** -128), v)]
        cases += [(f"qk 2^{e}", oracle_mod.bf16_bits(qf * 2.0 ** e), oracle_mod.bf16_bits(kf * 2.0 ** e), v)
                  for e in (12, 16, 24, 40, 56)]
        # huge scores from the middle of the walk on: the base turns coarse after a move
        one, late = kf.copy(), kf.copy()
        one[:, :, N // 2, :] *= 2.0 ** 40
        late[:, :, 3 * N // 4:, :] *= 2.0 ** 24
        cases += [("one key 2^40", q, oracle_mod.bf16_bits(one), v), ("late keys 2^24", q, oracle_mod.bf16_bits(late), v)]
        for name, qq, kk, vv in cases:
            for causal in (False, True):
                ref = oracle_mod.attention(qq, kk, vv, causal, threads=HOST_THREADS)
                for kernel in kernels_for(D):
                    say("value range", name, kernel, D, causal)
                    check(oracle_mod, run_bits(fa, kernel, qq, kk, vv, causal), ref,
                          f"value range {name} {kernel} {(D, causal)}")


def bf16_is_nan(bits):
    return ((bits & 0x7F80) == 0x7F80) & ((bits & 0x7F) != 0)


def test_non_finite_inputs(fa, oracle_mod):
    """A NaN in one query row (head 0, row 5), a NaN in one key (head 1, key
    200) and +Inf in one element of another key (head 0, key 100, dim 3).
    Exactly the rows whose FP64 oracle output is NaN come out NaN, in every
    element, and every other row passes the gate. The Inf key scores +Inf
    for the rows with q[3] > 0 (NaN outputs: the exponent base moves to
    infinity, as the oracle's max does), NaN where q[3] is zero, and -Inf
    where q[3] < 0 (P = 0: those rows stay finite). Causal rows that share a
    bad key's diagonal tile without seeing it stay finite: the mask replaces
    scores rather than adding to them. (A non-finite V is not meaningful
    here: a masked or underflowed P of 0 times Inf or NaN is NaN in any
    matrix product, while the oracle never multiplies it.)"""
    B, H, N = 1, 2, 300
    for D in (64, 128):
        q, k, v = oracle_mod.make_inputs(B, H, N, D, seeds={"q": 81, "k": 82, "v": 83})
        q[0, 0, 5, 7] = 0x7FC0
        k[0, 1, 200, 3] = 0x7FC0
        k[0, 0, 100, 3] = 0x7F80
        q3 = oracle_mod.bf16_to_f32(q[0, 0, :, 3])
        for causal in (False, True):
            ref = oracle_mod.attention(q, k, v, causal, threads=HOST_THREADS).reshape(-1, D)
            nan_rows = np.isnan(ref).any(axis=1)
            assert np.isnan(ref[nan_rows]).all()
            sees_inf = np.arange(N) >= (100 if causal else 0)
            expected = ({5} | set(np.flatnonzero(sees_inf & (q3 >= 0)).tolist())
                        | set(range(N + (200 if causal else 0), 2 * N)))
            assert set(np.flatnonzero(nan_rows).tolist()) == expected
            assert (sees_inf & (q3 < 0)).sum() > 50  # rows that see -Inf and stay finite
            for kernel in kernels_for(D):
                say("non-finite", kernel, D, causal)
                got = run_bits(fa, kernel, q, k, v, causal).reshape(-1, D)
                assert bf16_is_nan(got[nan_rows]).all(), (kernel, D, causal)
                assert not bf16_is_nan(got[~nan_rows]).any(), (kernel, D, causal)
                check(oracle_mod, got[~nan_rows], ref[~nan_rows], f"non-finite {kernel} {(D, causal)}")


def test_v3_and_v3b_agree(fa, oracle_mod):
    """The 128-row (v3_128) and 64-row (v3b) configurations. Dense: each wave
    computes its 32 rows identically whatever the workgroup size (both
    configurations split the same KV range the same way), so the outputs are
    bitwise equal. Causal: the KV range a workgroup walks ends at its own last
    row, so the two configurations split it between their two wave groups at
    different tiles and sum in a different order; both must pass the oracle
    gate and agree to one bf16 ulp of the row scale."""
    for (B, H, N, D) in [(1, 2, 300, 64), (2, 2, 513, 128)]:
        qb, kb, vb = oracle_mod.make_inputs(B, H, N, D)
        q, k, v = to_dev(qb), to_dev(kb), to_dev(vb)
        for causal in (False, True):
            say("v3-v3b", B, H, N, D, causal)
            a = from_dev(run(fa, "v3_128", q, k, v, causal))
            b = from_dev(run(fa, "v3b_mfma", q, k, v, causal))
            if not causal:
                assert np.array_equal(a, b)
                continue
            ref = oracle_mod.attention(qb, kb, vb, True, threads=HOST_THREADS)
            check(oracle_mod, a, ref, "v3 causal")
            check(oracle_mod, b, ref, "v3b causal")
            af = oracle_mod.bf16_to_f32(a).astype(np.float64).reshape(-1, D)
            bf = oracle_mod.bf16_to_f32(b).astype(np.float64).reshape(-1, D)
            row_scale = np.abs(ref.reshape(-1, D)).max(axis=1, keepdims=True)
            assert np.all(np.abs(af - bf) <= 2.0 ** -7 * row_scale)


def test_v3_picks_the_configuration_by_grid(fa, oracle_mod):
    """The v3 entry's configuration rule: 64 rows per workgroup when the
    128-row grid has fewer workgroups than the device has CUs (four KV groups
    at head_dim 64 with seq_len >= 1024, else two); 256 rows in one group when
    even 256-row workgroups give every CU one (dense), or, causal, for
    seq_len >= 8192 with two rounds of them, or when one round of them
    replaces more than one of 128-row workgroups at seq_len <= 2048 (head_dim
    128) or <= 1024 (64); at head_dim 64, causal, exactly one round and
    seq_len >= 2048, the four-group list layout (128, 4); at head_dim 64,
    causal, more than one round and seq_len <= 2048, 64 rows in two groups;
    else 128 rows in two groups. Its output equals the pinned configuration's
    bit for bit on each side of each threshold."""
    cus = fa.query_tensorcore_v3(64)["compute_units"]
    assert cus > 0
    cases = [
        ((1, 2, 700, 64), (False, True), "v3b_mfma"),           # 12 workgroups of 128 rows, seq_len < 1024
        ((1, 4, 1024, 64), (False, True), "v3_64x4"),           # 32 workgroups of 128 rows, head_dim 64
        ((1, 4, 1024, 128), (False, True), "v3b_mfma"),         # the same at head_dim 128
        ((1, cus // 2, 256, 64), (False, True), "v3_128"),      # `cus` of 128 rows, head_dim 64
        ((1, cus // 2, 256, 128), (False, True), "v3_128"),     # `cus` of 128 rows, `cus`/2 of 256
        ((1, cus, 256, 128), (False, True), "v3_256"),          # `cus` workgroups of 256 rows (causal:
        ((1, cus, 256, 64), (False, True), "v3_256"),           #   one round of them instead of two of 128)
        ((1, cus // 16, 2048, 64), (True,), "v3_128x4"),        # head_dim 64 causal, one round, seq_len 2048
        ((1, cus // 16, 2048, 64), (False,), "v3_128"),         # ... dense
        ((1, cus // 8, 2048, 64), (True,), "v3b_mfma"),         # head_dim 64 causal, 2 rounds, seq_len 2048
        ((1, cus // 16, 4096, 64), (True,), "v3_128"),          # ... and seq_len 4096
        ((1, 2 * cus // 32, 8192, 128), (True,), "v3_256"),     # causal, 2 * `cus` of 256 rows
        ((1, 2 * cus // 32, 8192, 64), (True,), "v3_256"),      # ... at head_dim 64
        ((1, cus // 16, 4096, 128), (True,), "v3_128"),         # one round of 256 rows, seq_len 4096
        ((1, 4 * cus // 16, 4096, 128), (True,), "v3_128"),     # causal below 8192 keys
    ]
    for (B, H, N, D), masks, pinned in cases:
        q, k, v = (to_dev(x) for x in oracle_mod.make_inputs(B, H, N, D))
        for causal in masks:
            shape = fa.AttentionShape(B, H, N, D)
            assert fa.tensorcore_v3_config(shape, causal) == fa.FUSED_CONFIGS[pinned], (shape, causal, pinned)
            assert fa.tensorcore_v3_rows_per_block(shape, causal) == fa.FUSED_CONFIGS[pinned][0]
            say("v3 dispatch", B, H, N, D, causal, pinned)
            a = from_dev(run(fa, "v3_mfma", q, k, v, causal))
            b = from_dev(run(fa, pinned, q, k, v, causal))
            assert np.array_equal(a, b), (B, H, N, D, causal, pinned)


def test_deterministic(fa, oracle_mod):
    for D in (64, 128):
        q, k, v = (to_dev(x) for x in oracle_mod.make_inputs(2, 4, 1000, D))
        for kernel in kernels_for(D):
            for causal in (False, True):
                say("determinism", kernel, D, causal)
                a = from_dev(run(fa, kernel, q, k, v, causal))
                b = from_dev(run(fa, kernel, q, k, v, causal))
                assert np.array_equal(a, b)


def test_non_default_stream(fa, oracle_mod):
    import torch

    s = torch.cuda.Stream()
    for D in (64, 128):
        q, k, v = oracle_mod.make_inputs(1, 2, 257, D)
        ref = oracle_mod.attention(q, k, v, True)
        qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
        torch.cuda.synchronize()
        for kernel in kernels_for(D):
            say("stream", kernel, D)
            with torch.cuda.stream(s):
                o = run(fa, kernel, qd, kd, vd, True, stream=s)
            check(oracle_mod, from_dev(o), ref, f"stream {kernel} D={D}")


def test_v0_profile_bitwise_equal(fa, oracle_mod):
    """benchmarks/profile_attention_v0.cu:98-122: the instrumented launch equals
    the plain launch bitwise, with and without events, at N in {1, 17, 256}."""
    import torch

    for n in (1, 17, 256):
        for d in (64, 128):
            for causal in (False, True):
                qb, kb, vb = oracle_mod.make_inputs(1, 2, n, d, "normal_mt19937")
                q, k, v = to_dev(qb), to_dev(kb), to_dev(vb)
                say("v0-profile", n, d, causal)
                plain = from_dev(run(fa, "v0_unfused", q, k, v, causal))
                shape = fa.AttentionShape(1, 2, n, d)
                ws = torch.empty(fa.unfused_workspace_bytes(shape) // 4, dtype=torch.float32, device="cuda")
                events = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
                o1 = nan_like(q)
                assert fa.launch_attention_unfused_profile(q, k, v, o1, ws, shape, causal, events=events)
                torch.cuda.synchronize()
                o2 = nan_like(q)
                assert fa.launch_attention_unfused_profile(q, k, v, o2, ws, shape, causal, events=None)
                torch.cuda.synchronize()
                assert np.array_equal(from_dev(o1), plain) and np.array_equal(from_dev(o2), plain)
                stages = [events[i].elapsed_time(events[i + 1]) for i in range(3)]
                assert all(t >= 0.0 for t in stages)


def test_softmax_rows_inplace(fa):
    import torch

    rng = np.random.default_rng(9)
    for rows, cols in [(5, 1), (7, 3), (4, 1000), (3, 2048), (2, 8192), (2, 9000), (3, 4097)]:
        x = rng.normal(0, 4, size=(rows, cols)).astype(np.float32)
        x[0, : cols // 2] = -np.finfo(np.float32).max  # masked entries
        if rows > 2:
            x[2, :] = -np.finfo(np.float32).max        # fully masked row -> uniform
        t = torch.from_numpy(x.copy()).cuda()
        say("softmax", rows, cols)
        assert fa.launch_softmax_rows_inplace(t, rows, cols)
        torch.cuda.synchronize()
        got = t.cpu().numpy().astype(np.float64)
        xd = x.astype(np.float64)
        e = np.exp(xd - xd.max(axis=1, keepdims=True))
        want = e / e.sum(axis=1, keepdims=True)
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=1e-7)
    # unaligned base pointer takes the scalar path
    x = rng.normal(size=(3, 65)).astype(np.float32)
    t = torch.from_numpy(np.concatenate([np.zeros(1, np.float32), x.reshape(-1)])).cuda()
    assert fa.launch_softmax_rows_inplace(t.data_ptr() + 4, 3, 65)
    torch.cuda.synchronize()
    got = t.cpu().numpy()[1:].reshape(3, 65).astype(np.float64)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    np.testing.assert_allclose(got, e / e.sum(axis=1, keepdims=True), rtol=2e-5, atol=1e-7)


def test_error_paths_leave_output_untouched(fa, oracle_mod):
    import torch

    q = to_dev(oracle_mod.make_inputs(1, 1, 64, 96)[0])
    o = nan_like(q)
    shape = fa.AttentionShape(1, 1, 64, 96)
    assert fa.launch_attention_tensorcore_v3(q, q, q, o, shape, False) is False
    assert fa.launch_attention_tensorcore_v3b(q, q, q, o, shape, True) is False
    torch.cuda.synchronize()
    assert np.all(from_dev(o) == 0xFFFF)
    # empty sequence: success, no launch
    assert fa.launch_attention_tensorcore_v3(q, q, q, o, fa.AttentionShape(1, 1, 0, 64), False)
    # misaligned base pointer is rejected on the host, and kept for the
    # thread's get_last_error (what a caller of the void C++ launcher reads)
    fa.get_last_error()
    with pytest.raises(fa.FaError):
        fa.launch_attention_tensorcore_v3(q.data_ptr() + 2, q, q, o, fa.AttentionShape(1, 1, 16, 64), False)
    assert fa.get_last_error() == 1 and fa.get_last_error() == 0
    torch.cuda.synchronize()
    assert np.all(from_dev(o) == 0xFFFF)
    # v0 handles any head_dim, including 96
    qb, kb, vb = oracle_mod.make_inputs(1, 2, 50, 96)
    ref = oracle_mod.attention(qb, kb, vb, True)
    check(oracle_mod, run_bits(fa, "v0_unfused", qb, kb, vb, True), ref, "v0 D=96")
    qb, kb, vb = oracle_mod.make_inputs(1, 1, 37, 5)  # odd D -> scalar load path
    ref = oracle_mod.attention(qb, kb, vb, False)
    check(oracle_mod, run_bits(fa, "v0_unfused", qb, kb, vb, False), ref, "v0 D=5")


def test_query_reports_resources(fa):
    for rows, groups in fa.FUSED_CONFIGS.values():
        for d in (64, 128):
            assert fa.query_fused_groups(d, rows, groups) == fa.query_fused_config(d, rows, groups, False)
            for causal in (False, True):
                info = fa.query_fused_config(d, rows, groups, causal)
                if groups == 4 and d == 128:
                    assert info["supported"] == 0
                    continue
                assert info["supported"] == 1 and info["rows_per_block"] == rows and info["kv_groups"] == groups
                assert info["waves_per_block"] * 64 == info["block_size"]
                assert info["agprs_per_thread"] == 0 and info["max_blocks_per_sm"] >= 1
                if (d, groups, causal) == (64, 1, False):
                    # the dense head_dim-64 one-group kernel is built for two
                    # workgroups per CU (at most 128 VGPRs); the compiler may
                    # spill a few values, which lie outside the step loop
                    # (test_capi_host.py::test_no_spill_traffic_in_step_loops)
                    assert info["max_blocks_per_sm"] == 2 and info["local_bytes_per_thread"] <= 64
                    assert info["registers_per_thread"] <= 128
                else:
                    assert info["local_bytes_per_thread"] == 0, ("register spill", rows, groups, d, causal)


def test_query_describes_the_launched_kernel(fa):
    """query_tensorcore_v3(shape, causal) reports the instantiation v3 runs:
    at the four metric shapes, the configuration fa_tensorcore_v3_config
    names with the mask's own build (c2 causal: the (128, 4) list kernel)."""
    seen = {}
    for d in (64, 128):
        for causal in (False, True):
            shape = fa.AttentionShape(2, 8, 2048, d)
            rows, groups = fa.tensorcore_v3_config(shape, causal)
            info = fa.query_tensorcore_v3_shape(shape, causal)
            print((2, 8, 2048, d), "causal" if causal else "dense", (rows, groups), info)
            assert info == fa.query_fused_config(d, rows, groups, causal)
            assert info["rows_per_block"] == rows and info["kv_groups"] == groups
            assert info["local_bytes_per_thread"] == 0 and info["agprs_per_thread"] == 0
            seen[(d, causal)] = (rows, groups)
    assert seen[(64, True)] == (128, 4)
    assert fa.query_tensorcore_v3_shape(fa.AttentionShape(2, 8, 2048, 96), False)["supported"] == 0
    for d in (64, 128):
        wide = fa.query_fused(d, 256)
        assert wide["rows_per_block"] == 256 and wide["waves_per_block"] == 8 and wide["block_size"] == 512
        infos = [fa.query_tensorcore_v3(d), fa.query_tensorcore_v3b(d), wide]
        for info in infos:
            print(d, info)
            assert info["supported"] == 1
            assert info["registers_per_thread"] > 0
            if not (d == 64 and info is wide):
                assert info["local_bytes_per_thread"] == 0, "register spill"
            assert info["shared_bytes_per_block"] >= 2 * 2 * 32 * d * 2
            assert info["max_blocks_per_sm"] >= 1
            assert info["device_shared_bytes_per_sm"] >= 64 * 1024
            assert info["compute_units"] > 0
            # AGPRs from the compiler's report of the kernel (the kernels
            # accumulate MFMA results in architectural VGPRs: 0)
            assert info["agprs_per_thread"] == 0
