"""CPU pins of the FP64 oracle (oracle/oracle.cpp).

Each check is chosen so that a plausible mistake in the oracle (a dropped
term, a wrong sign, scale or index, a transposed operand, a wrong rounding)
fails at least one of them:
  * bit-level bf16 RNE: exhaustive (2^32 patterns) agreement of two
    independent implementations, plus agreement with torch's converter;
  * bf16_ulp against the spacing of adjacent bf16 values;
  * closed forms: default_scale bits, FLOP / workspace identities;
  * special inputs with textbook answers (N=1, Q=K=0, all ones, constant V,
    one-hot logits);
  * an independent numpy long-double brute force on tiny shapes;
  * the C++-standard mt19937 known answer and SplitMix64's published output;
  * the reference's own published accuracy statistics
    (results/raw/flash_attention/accuracy.csv:2-21), reproduced to 1e-15 from
    regenerated reference inputs — which also fails if the oracle is fed a
    transposed operand or the wrong mask (planted below).
"""
import json
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def brute_force(qb, kb, vb, causal, oracle):
    """Independent restatement: vectorised long-double softmax(QK^T*scale)V with
    the normalisation applied to P before the product."""
    q = oracle.bf16_to_f32(qb).astype(np.longdouble)
    k = oracle.bf16_to_f32(kb).astype(np.longdouble)
    v = oracle.bf16_to_f32(vb).astype(np.longdouble)
    B, H, N, D = q.shape
    scale = np.longdouble(np.float32(1.0) / np.sqrt(np.float32(D)))
    out = np.empty((B, H, N, D), dtype=np.longdouble)
    for b in range(B):
        for h in range(H):
            s = np.einsum("qd,kd->qk", q[b, h], k[b, h]) * scale
            if causal:
                s = np.where(np.tril(np.ones((N, N), dtype=bool)), s, -np.inf)
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p = p / p.sum(axis=1, keepdims=True)
            out[b, h] = np.einsum("qk,kd->qd", p, v[b, h])
    return out


def test_rne_exhaustive_two_implementations(oracle_mod):
    assert oracle_mod.rne_exhaustive_mismatches(8) == 0


def test_rne_matches_torch(oracle_mod):
    torch = pytest.importorskip("torch")
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x3FFF, 0x7FFF, 0x8000, 0x8001, 0xBFFF, 0xC000, 0xFFFF, 0x1234,
                     0x7FFE, 0x8002, 0x4000, 0xA5A5, 0x5A5A, 0xEFFF], dtype=np.uint32)
    bits = (hi[:, None] | lows[None, :]).reshape(-1)
    x = bits.view(np.float32)
    ours = oracle_mod.bf16_bits(x)
    theirs = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    finite_or_inf = ~np.isnan(x)
    assert np.array_equal(ours[finite_or_inf], theirs[finite_or_inf])
    # NaN stays NaN
    back = oracle_mod.bf16_to_f32(ours[~finite_or_inf])
    assert np.all(np.isnan(back))


def test_rne_ties_and_overflow(oracle_mod):
    L = oracle_mod.lib()
    f = lambda u: np.array([u], dtype=np.uint32).view(np.float32)[0]
    assert L.fa_oracle_bf16_from_float(f(0x3F808000)) == 0x3F80  # tie, even kept
    assert L.fa_oracle_bf16_from_float(f(0x3F818000)) == 0x3F82  # tie, odd rounds up
    assert L.fa_oracle_bf16_from_float(f(0x7F7FFFFF)) == 0x7F80  # overflow -> +inf
    assert L.fa_oracle_bf16_from_float(f(0xFF7FFFFF)) == 0xFF80  # -> -inf
    assert L.fa_oracle_bf16_from_float(f(0x00000001)) == 0x0000  # tiny subnormal -> 0


def test_bf16_ulp_is_bf16_spacing(oracle_mod):
    rng = np.random.default_rng(3)
    bits = rng.integers(0x0001, 0x7F7F, size=4000, dtype=np.uint16)  # positive finite, not max
    x = oracle_mod.bf16_to_f32(bits)
    spacing = oracle_mod.bf16_to_f32(bits + 1).astype(np.float64) - x.astype(np.float64)
    for xv, sp in zip(x, spacing):
        assert oracle_mod.bf16_ulp(float(xv)) == pytest.approx(sp, rel=0, abs=0), (xv, sp)
    assert oracle_mod.bf16_ulp(1.0) == 2.0 ** -7
    assert oracle_mod.bf16_ulp(0.75) == 2.0 ** -8
    assert oracle_mod.bf16_ulp(0.0) == 2.0 ** -133
    assert oracle_mod.bf16_ulp(float("inf")) == 2.0 ** -133


def test_default_scale_bits(oracle_mod):
    s128 = np.float32(oracle_mod.default_scale(128))
    assert s128.view(np.uint32) == 0x3DB504F3
    assert oracle_mod.default_scale(64) == 0.125


def test_flops_and_workspace_identities(oracle_mod):
    L = oracle_mod.lib()
    assert oracle_mod.attention_flops(2, 8, 2048, 64, False) == 4.0 * 2048 ** 2 * 64 * 16 == 17179869184.0
    assert oracle_mod.attention_flops(2, 8, 2048, 128, True) == 4.0 * 2048 * 2049 / 2 * 128 * 16
    assert L.fa_oracle_unfused_workspace_bytes(2, 8, 2048) == 2 * 8 * 2048 * 2048 * 4 == 268435456
    assert L.fa_oracle_qkvo_bytes(2, 8, 2048, 64) == 8 * 2 * 8 * 2048 * 64
    # v3 traffic model at one query block equals Q+O + one pass of K/V tiles
    assert L.fa_oracle_blocked_kv_hbm_bytes(1, 1, 64, 64, 0, 64, 64) == 4 * 64 * 64 * 2


def _reference_hbm_rows():
    with open(os.path.join(HERE, "golden", "reference_hbm_model.json")) as fh:
        return json.load(fh)["rows"]


def _oracle_model_bytes(L, kernel, B, H, N, D, causal, rows=None, tile=None):
    """The oracle's byte model for one kernel of the reference's summary.csv
    (benchmarks/bench_flash_attention.cu:641-648), with the reference's
    tiling unless `rows` / `tile` override it."""
    if kernel == "v0_unfused":
        return L.fa_oracle_qkvo_bytes(B, H, N, D) + L.fa_oracle_unfused_score_bytes(B, H, N)
    if kernel in ("v2a_fused_tiled", "v2b_fused_tiled"):  # 256 threads / 32 = 8 rows, tileKV 64
        rows, tile = rows or 8, tile or 64
    else:  # v3: q_rows 64, v3_tile_kv(D) = 64 (D <= 64) or 32
        rows, tile = rows or 64, tile or (64 if D <= 64 else 32)
    return L.fa_oracle_blocked_kv_hbm_bytes(B, H, N, D, causal, rows, tile)


def test_byte_models_reproduce_reference_published_hbm(oracle_mod):
    """All 240 published algorithmic_hbm_gb values (v0, v2a, v2b, v3 rows of
    results/raw/flash_attention/summary.csv, 60 shapes each) come out of the
    oracle's byte models to 1e-12."""
    L = oracle_mod.lib()
    rows = _reference_hbm_rows()
    assert len(rows) == 240
    for r in rows:
        got = _oracle_model_bytes(L, r["kernel"], r["batch"], r["heads"], r["seq_len"], r["head_dim"], r["causal"])
        want = float(r["algorithmic_hbm_gb"]) * 1e9
        assert got == pytest.approx(want, rel=1e-12), r


def test_byte_model_fixture_rejects_planted_mistakes(oracle_mod):
    """The fixture discriminates the model's parameters: the wrong rows per
    block, or v0 without the softmax passes, each miss published values.
    (The tile size cancels on the published grid, whose rows per block are
    multiples of the tile; test_byte_model_closed_forms pins it.)"""
    L = oracle_mod.lib()
    rows = _reference_hbm_rows()

    def misses(fn):
        return sum(1 for r in rows if fn(r) != pytest.approx(float(r["algorithmic_hbm_gb"]) * 1e9, rel=1e-12))

    assert misses(lambda r: _oracle_model_bytes(L, r["kernel"], r["batch"], r["heads"], r["seq_len"], r["head_dim"],
                                                r["causal"], rows=128) if r["kernel"] != "v0_unfused" else
                  float(r["algorithmic_hbm_gb"]) * 1e9) > 100
    assert misses(lambda r: L.fa_oracle_qkvo_bytes(r["batch"], r["heads"], r["seq_len"], r["head_dim"]) +
                  3.0 / 5.0 * L.fa_oracle_unfused_score_bytes(r["batch"], r["heads"], r["seq_len"])
                  if r["kernel"] == "v0_unfused" else float(r["algorithmic_hbm_gb"]) * 1e9) == 60


def test_byte_model_closed_forms(oracle_mod):
    """Branches the published grid (N a multiple of every tile) leaves open:
    ragged N and the causal clamp of the last block's key limit to N-1."""
    L = oracle_mod.lib()
    assert L.fa_oracle_unfused_score_bytes(2, 8, 2048) == 20.0 * 2 * 8 * 2048 ** 2
    for (B, H, N, D, rows, tile) in [(1, 1, 1, 64, 64, 32), (2, 3, 77, 128, 128, 32), (1, 2, 1000, 64, 64, 64),
                                     (3, 1, 4097, 128, 256, 32), (1, 1, 33, 64, 8, 64)]:
        nb = -(-N // rows)
        qo = 2.0 * B * H * N * D * 2
        # dense: every block loads ceil(N / tile) whole tiles
        dense = qo + 2.0 * B * H * nb * (-(-N // tile)) * tile * D * 2
        assert L.fa_oracle_blocked_kv_hbm_bytes(B, H, N, D, 0, rows, tile) == dense
        # causal: block b loads tiles up to min(last row of b, N-1)
        tiles = sum(min(b * rows + rows - 1, N - 1) // tile + 1 for b in range(nb))
        assert L.fa_oracle_blocked_kv_hbm_bytes(B, H, N, D, 1, rows, tile) == qo + 2.0 * B * H * tiles * tile * D * 2
    # causal, rows == tile, N a multiple: triangular number of tiles
    assert L.fa_oracle_blocked_kv_hbm_bytes(1, 1, 64 * 10, 64, 1, 64, 64) == (2 * 640 * 64 * 2 +
                                                                               2 * 55 * 64 * 64 * 2)


def test_package_quantiles_and_summary_match_numpy(fa_lib):
    """The package's type-7 quantile and median/IQR summary (every median in
    bench.py's line) against numpy's default (linear = type 7) percentile."""
    rng = np.random.default_rng(11)
    for n in (1, 2, 3, 7, 30, 31):
        xs = list(rng.random(n) * 10)
        for p in (0.0, 0.1, 0.25, 0.5, 0.75, 0.9, 1.0):
            assert fa_lib.quantile_type7(xs, p) == pytest.approx(float(np.percentile(xs, 100 * p)), rel=1e-14)
        s = fa_lib.summarize(xs)
        q1, med, q3 = np.percentile(xs, [25, 50, 75])
        assert s["median_ms"] == pytest.approx(med, rel=1e-14)
        assert s["q1_ms"] == pytest.approx(q1, rel=1e-14) and s["q3_ms"] == pytest.approx(q3, rel=1e-14)
        assert s["iqr_ms"] == pytest.approx(q3 - q1, rel=1e-12, abs=1e-15)
    # order of the samples does not matter; ties and a known small case
    assert fa_lib.quantile_type7([4.0, 1.0, 3.0, 2.0], 0.25) == 1.75
    assert fa_lib.summarize([2.0, 2.0, 2.0])["iqr_ms"] == 0.0


def test_quantile_type7(oracle_mod):
    rng = np.random.default_rng(5)
    for n in (1, 2, 7, 30):
        xs = np.sort(rng.random(n))
        for p in (0.0, 0.25, 0.5, 0.75, 1.0):
            assert oracle_mod.quantile_sorted(xs, p) == pytest.approx(np.percentile(xs, 100 * p), rel=1e-15)


def test_known_answers_generators(oracle_mod):
    assert oracle_mod.lib().fa_oracle_mt19937_10000th() == 4123659995
    assert int(oracle_mod.splitmix64(0, 1)[0]) == 0xE220A8397B1DCDAF
    u = oracle_mod.bf16_to_f32(oracle_mod.fill_uniform((1 << 16,), 11))
    assert u.min() >= -1.0 and u.max() <= 1.0
    assert abs(float(u.mean())) < 0.01 and abs(float(u.var()) - 1.0 / 3.0) < 0.01
    z = oracle_mod.bf16_to_f32(oracle_mod.fill_normal((1 << 16,), 22, 3.0)).astype(np.float64)
    assert abs(z.mean()) < 0.05 and abs(z.std() - 3.0) < 0.05


def test_single_key_returns_v_row(oracle_mod):
    q, k, v = oracle_mod.make_inputs(1, 2, 1, 64)
    for causal in (False, True):
        out = oracle_mod.attention(q, k, v, causal)
        assert np.array_equal(out, oracle_mod.bf16_to_f32(v).astype(np.float64))


def test_causal_row0_and_zero_logits(oracle_mod):
    B, H, N, D = 1, 2, 33, 64
    q, k, v = oracle_mod.make_inputs(B, H, N, D, "zeros")
    vf = oracle_mod.bf16_to_f32(v).astype(np.float64)
    dense = oracle_mod.attention(q, k, v, False)
    causal = oracle_mod.attention(q, k, v, True)
    np.testing.assert_allclose(dense, np.broadcast_to(vf.mean(axis=2, keepdims=True), dense.shape), rtol=1e-13, atol=1e-15)
    prefix = np.cumsum(vf, axis=2) / np.arange(1, N + 1)[None, None, :, None]
    np.testing.assert_allclose(causal, prefix, rtol=1e-13, atol=1e-15)
    qr, kr, vr = oracle_mod.make_inputs(B, H, N, D)
    out = oracle_mod.attention(qr, kr, vr, True)
    assert np.array_equal(out[:, :, 0], oracle_mod.bf16_to_f32(vr[:, :, 0]).astype(np.float64))


def test_all_ones_and_constant_v(oracle_mod):
    q, k, v = oracle_mod.make_inputs(1, 1, 17, 128, "ones")
    for causal in (False, True):
        assert np.array_equal(oracle_mod.attention(q, k, v, causal), np.ones((1, 1, 17, 128)))
    q, k, _ = oracle_mod.make_inputs(1, 2, 40, 64)
    c = oracle_mod.bf16_bits(np.full((1, 2, 40, 64), -0.3125, dtype=np.float32))
    for causal in (False, True):
        np.testing.assert_allclose(oracle_mod.attention(q, k, c, causal), -0.3125, rtol=1e-15)


def test_one_hot_logit_selects_v_row(oracle_mod):
    N, D = 24, 64
    q = np.zeros((1, 1, N, D), dtype=np.uint16)
    k = np.zeros((1, 1, N, D), dtype=np.uint16)
    big = oracle_mod.bf16_bits(np.array([64.0], dtype=np.float32))[0]
    q[..., 0] = big           # every query points along dim 0
    winner = 5
    k[0, 0, winner, 0] = big  # logit 64*64/8 = 512 for key 5, 0 elsewhere
    _, _, v = oracle_mod.make_inputs(1, 1, N, D)
    out = oracle_mod.attention(q, k, v, False)
    np.testing.assert_allclose(out[0, 0], np.broadcast_to(oracle_mod.bf16_to_f32(v[0, 0, winner]), (N, D)), rtol=1e-15)
    outc = oracle_mod.attention(q, k, v, True)
    np.testing.assert_allclose(outc[0, 0, winner:], np.broadcast_to(oracle_mod.bf16_to_f32(v[0, 0, winner]), (N - winner, D)), rtol=1e-15)


def test_reference_boundary_families(oracle_mod):
    """The reference's five boundary families (kernels/ablation/experiments.cu:
    283-289) as the oracle builds them: the normal(0,1) mt19937 base with
    seeds 11/22/33, Q=K=V=0 (every output exactly 0: uniform weights over a
    zero V), all ones (every output 1), the ramp V (integers -D/2 .. D/2-1
    along the head dim) over the same normal Q and K, and the normal Q and K
    times 4 (exact in bf16; logits of standard deviation about 16)."""
    shape = (1, 2, 129, 64)
    base = oracle_mod.make_inputs(*shape, "normal_mt19937")
    normal = oracle_mod.make_inputs(*shape, "ref_normal")
    for a, b in zip(base, normal):
        assert np.array_equal(a, b)
    q, k, v = oracle_mod.make_inputs(*shape, "ref_zeros")
    assert not q.any() and not k.any() and not v.any()
    for causal in (False, True):
        assert np.array_equal(oracle_mod.attention(q, k, v, causal), np.zeros(shape))
    q, k, v = oracle_mod.make_inputs(*shape, "ref_ramp")
    assert np.array_equal(q, base[0]) and np.array_equal(k, base[1])
    vf = oracle_mod.bf16_to_f32(v)
    assert np.array_equal(vf[0, 1, 7], np.arange(64, dtype=np.float32) - 32)
    q, k, v = oracle_mod.make_inputs(*shape, "ref_scaled")
    assert np.array_equal(oracle_mod.bf16_to_f32(q), 4 * oracle_mod.bf16_to_f32(base[0]))
    assert np.array_equal(oracle_mod.bf16_to_f32(k), 4 * oracle_mod.bf16_to_f32(base[1]))
    assert np.array_equal(v, base[2])
    logits = np.einsum("hnd,hmd->hnm", oracle_mod.bf16_to_f32(q)[0].astype(np.float64),
                       oracle_mod.bf16_to_f32(k)[0].astype(np.float64)) / np.sqrt(64.0)
    assert 13.0 < logits.std() < 19.0
    for causal in (False, True):
        assert np.all(np.isfinite(oracle_mod.attention(q, k, v, causal)))


@pytest.mark.parametrize("family", ["uniform", "scaled", "ramp", "stress", "normal_mt19937", "ref_ramp",
                                    "ref_scaled"])
@pytest.mark.parametrize("causal", [False, True])
def test_brute_force_long_double(oracle_mod, family, causal):
    for (B, H, N, D) in [(1, 2, 9, 64), (2, 1, 33, 128), (1, 1, 64, 64)]:
        q, k, v = oracle_mod.make_inputs(B, H, N, D, family)
        got = oracle_mod.attention(q, k, v, causal)
        want = brute_force(q, k, v, causal, oracle_mod).astype(np.float64)
        scale = np.maximum(np.abs(want).max(axis=-1, keepdims=True), 1e-30)
        assert np.all(np.isfinite(got))
        assert np.max(np.abs(got - want) / scale) < 1e-12, (B, H, N, D, family, causal)


def test_row_subset_matches_full(oracle_mod):
    q, k, v = oracle_mod.make_inputs(2, 2, 70, 64)
    full = oracle_mod.attention(q, k, v, True).reshape(-1, 64)
    rows = np.array([0, 1, 69, 70, 139, 200, 279], dtype=np.int64)
    part = oracle_mod.attention(q, k, v, True, rows=rows, threads=3)
    assert np.array_equal(part, full[rows])
    with pytest.raises(ValueError):
        oracle_mod.attention(q, k, v, True, rows=np.array([280], dtype=np.int64))


@pytest.mark.parametrize("causal", [False, True])
def test_blocked_path_equals_scalar_restatement(oracle_mod, causal):
    """The default (cache-blocked) oracle reorders only which independent sums
    advance first; every output must equal the row-by-row restatement of
    bench_flash_attention.cu:117-142 bit for bit: ragged N (tails of the
    4-query, 8-key and 256-key blocks), head dims that are not a multiple of
    8, several slabs, unsorted and repeated row lists, several families."""
    cases = [((1, 1, 1, 64), "uniform"), ((2, 3, 37, 128), "uniform"), ((1, 2, 300, 64), "stress"),
             ((1, 1, 513, 128), "normal_mt19937"), ((2, 1, 77, 5), "uniform"), ((1, 2, 260, 80), "scaled"),
             ((1, 1, 129, 3), "ramp")]
    for shape, family in cases:
        q, k, v = oracle_mod.make_inputs(*shape, family)
        fast = oracle_mod.attention(q, k, v, causal, threads=4)
        slow = oracle_mod.attention(q, k, v, causal, threads=4, scalar=True)
        assert np.array_equal(fast.view(np.uint64), slow.view(np.uint64)), (shape, family, causal)
        total = shape[0] * shape[1] * shape[2]
        rows = np.random.default_rng(total).integers(0, total, size=min(total, 50)).astype(np.int64)
        rows = np.concatenate([rows, rows[:3]])  # repeats and any order
        part = oracle_mod.attention(q, k, v, causal, rows=rows, threads=3)
        assert np.array_equal(part.view(np.uint64), slow.reshape(-1, shape[3])[rows].view(np.uint64))


def _reference_cases():
    with open(os.path.join(HERE, "golden", "reference_accuracy.json")) as fh:
        return json.load(fh)["cases"]


@pytest.mark.parametrize("case", _reference_cases(), ids=lambda c: f"D{c['head_dim']}_c{c['causal']}")
def test_reference_accuracy_csv_known_answer(oracle_mod, case):
    """Regenerate the reference's inputs (mt19937 + normal<float>, seeds 11/22/33,
    B=1 H=2 N=256) and reproduce its published error statistics, which are set
    by rounding the FP64 oracle output to bf16."""
    D, causal = case["head_dim"], bool(case["causal"])
    q, k, v = oracle_mod.make_inputs(1, 2, 256, D, "normal_mt19937")
    ref = oracle_mod.attention(q, k, v, causal)
    acc = oracle_mod.compare(oracle_mod.bf16_bits(ref.astype(np.float32)), ref)
    assert acc.max_abs == pytest.approx(case["max_abs_error"], rel=1e-15)
    assert acc.row_scaled == pytest.approx(case["row_scaled_error"], rel=1e-15)
    if D == 64:  # v0 returned exactly bf16(O_ref) there, so vs_double matches too
        assert acc.vs_double == pytest.approx(case["v0_vs_double"], rel=1e-15)
    assert acc.passed and acc.ulp == 0.0


def test_known_answer_catches_planted_mistakes(oracle_mod):
    """The published statistics reject an oracle fed a transposed operand
    (K and V swapped), the wrong mask, or the wrong seed order."""
    case = _reference_cases()[0]  # D=64 dense
    q, k, v = oracle_mod.make_inputs(1, 2, 256, 64, "normal_mt19937")

    def stat(qq, kk, vv, causal):
        ref = oracle_mod.attention(qq, kk, vv, causal)
        return oracle_mod.compare(oracle_mod.bf16_bits(ref.astype(np.float32)), ref).max_abs

    assert stat(q, k, v, False) == pytest.approx(case["max_abs_error"], rel=1e-15)
    for planted in (stat(q, v, k, False), stat(q, k, v, True), stat(k, q, v, False)):
        assert planted != pytest.approx(case["max_abs_error"], rel=1e-6)


def test_comparator_planted_errors(oracle_mod):
    ref = np.array([[0.5, -0.25, 0.125, 0.0]], dtype=np.float64)
    good = oracle_mod.bf16_bits(ref.astype(np.float32))
    acc = oracle_mod.compare(good, ref)
    assert acc.passed and acc.max_abs == 0.0 and acc.ulp == 0.0
    # one bf16 ulp of the row scale (0.5 -> ulp 2^-8) on the largest element: ulp = 1
    off = good.copy()
    off[0, 0] += 1
    acc = oracle_mod.compare(off, ref)
    assert acc.ulp == 1.0 and acc.passed
    # three ulps fail the reference gate; 2^-7 * 0.5 = 2^-8 abs gate also fails
    off[0, 0] += 2
    acc = oracle_mod.compare(off, ref)
    assert acc.ulp == 3.0 and not acc.passed_ulp and not acc.passed_abs
    # NaN output is counted and fails
    nan = good.copy()
    nan[0, 2] = 0x7FC0
    acc = oracle_mod.compare(nan, ref)
    assert acc.output_nan == 1 and not acc.passed and acc.max_abs == float("inf")
    # unwritten 0xFFFF prefill is NaN
    acc = oracle_mod.compare(np.full_like(good, 0xFFFF), ref)
    assert acc.output_nan == 4 and not acc.passed
