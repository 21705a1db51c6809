"""Maximum sizes: tensors past 4 GiB, and a 65536-key sequence.

(1, 8192, 4096, 64) bf16 is 4 GiB per tensor, so the last (batch, head) slabs
start beyond 2^32 bytes: every slab offset, K/V descriptor base and output row
address must be 64-bit. The inputs are drawn uniform[-1,1) on the device (no
4 GiB host arrays); the first, a middle and the last slab are copied back and
every row of them is checked against the FP64 oracle, dense and causal, for the v3 entry
(256-row configuration at this grid size for dense, 128-row for causal) and
the pinned 128-row configuration. The output starts as NaN-pattern fill, so a
slab the kernel skips fails the check."""
import numpy as np
import pytest

from gpu_common import FUSED_KERNELS, HOST_THREADS, from_dev, kernels_for, nan_like, run, say, to_dev
from test_gpu_parity import check, fa  # noqa: F401 (fa: fixture)

pytestmark = [pytest.mark.gpu, pytest.mark.slow]


def test_tensors_past_4_gib(fa, oracle_mod):
    import torch

    B, H, N, D = 1, 8192, 4096, 64
    assert B * H * N * D * 2 >= 2 ** 32
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)
    say("large inputs", B, H, N, D)
    q, k, v = (torch.empty((B, H, N, D), dtype=torch.bfloat16, device="cuda").uniform_(-1.0, 1.0, generator=gen)
               for _ in range(3))
    slabs = (0, H // 2 + 1, H - 1)
    host = {s: tuple(from_dev(t[0, s]).reshape(1, 1, N, D) for t in (q, k, v)) for s in slabs}
    for causal in (False, True):
        refs = {s: oracle_mod.attention(*host[s], causal).reshape(N, D) for s in slabs}
        for kernel in ("v3_mfma", "v3_128", "v3_64x4", "v3_128x4"):
            say("large", kernel, causal)
            o = run(fa, kernel, q, k, v, causal, out=nan_like(q))
            for s in slabs:
                got = from_dev(o[0, s]).reshape(N, D)
                check(oracle_mod, got, refs[s], f"large {kernel} causal={causal} slab {s}")
            del o
            torch.cuda.empty_cache()


def test_list_layout_long_sequence(fa, oracle_mod):
    """(1,2,16384,64) causal is one round of 128-row workgroups (2 slabs x
    128 blocks = 256), so v3 runs the list layout: each workgroup's two half
    blocks are far apart in length (the first pair's tile lists are 2 and 512
    long), so quarters cross from the early to the late half block at every
    position. Every row of both slabs against the FP64 oracle, for v3 and the
    pinned configuration (bitwise equal)."""
    B, H, N, D = 1, 2, 16384, 64
    cus = fa.query_tensorcore_v3(64)["compute_units"]
    qb, kb, vb = oracle_mod.make_inputs(B, H, N, D, seeds={"q": 91, "k": 92, "v": 93})
    ref = oracle_mod.attention(qb, kb, vb, True)
    say("list long", B, H, N, D)
    if cus == 256:
        assert fa.tensorcore_v3_config(fa.AttentionShape(B, H, N, D), True) == (128, 4)
    got = from_dev(run(fa, "v3_mfma", *(to_dev(x) for x in (qb, kb, vb)), True))
    check(oracle_mod, got, ref, "list long v3")
    pinned = from_dev(run(fa, "v3_128x4", *(to_dev(x) for x in (qb, kb, vb)), True))
    assert cus != 256 or np.array_equal(got, pinned)
    check(oracle_mod, pinned, ref, "list long pinned")


@pytest.mark.parametrize("D", [64, 128])
def test_sequence_65536(fa, oracle_mod, D):
    """N = 65536 in one slab, four times the longest BASELINE sequence (c5):
    2048 K/V tiles in a walk. Dense on uniform inputs, and causal on the
    stress family (Q, K ~ N(0, 3^2)), whose logits keep raising the row
    maximum along the whole walk, so the exponent base moves again and again.
    Every fused configuration. The first and last query tiles and 64 seeded
    random rows are checked against the FP64 oracle, and every output element
    must be finite after the NaN prefill."""
    B, H, N = 1, 1, 65536
    rows = oracle_mod.sample_rows(B, H, N)
    for family, causal in (("uniform", False), ("stress", True)):
        qb, kb, vb = oracle_mod.make_inputs(B, H, N, D, family, seeds={"q": 71 + D, "k": 72 + D, "v": 73 + D})
        ref = oracle_mod.attention(qb, kb, vb, causal, rows=rows, threads=HOST_THREADS)
        q, k, v = to_dev(qb), to_dev(kb), to_dev(vb)
        for kernel in kernels_for(D, FUSED_KERNELS):
            say("seq 65536", kernel, D, family, causal)
            out = from_dev(run(fa, kernel, q, k, v, causal)).reshape(-1, D)
            assert int(np.count_nonzero((out & 0x7F80) == 0x7F80)) == 0, (kernel, causal)
            acc = check(oracle_mod, out[rows], ref, f"seq 65536 {kernel} D={D} {family} causal={causal}")
            print(f"seq 65536 {kernel} D={D} {family} causal={causal} rows {len(rows)} ulp={acc.ulp:.2f} "
                  f"row_scaled={acc.row_scaled:.2e}")
        del q, k, v
