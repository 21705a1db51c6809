"""The allocation-free v0 entry point (fa_launch_attention_unfused_noalloc)
against the workspace entry it shares its kernels with: bit-for-bit equal
outputs on two calls in a row, the second smaller than the first (the
library's one scratch array per GPU keeps the first call's contents), a
shape at the scratch limit, and a shape past it rejected with nothing
written. Called through the C ABI."""
import ctypes

import numpy as np
import pytest

from gpu_common import from_dev, nan_like, say, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fa(fa_lib):
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    return fa_lib


def _stream():
    import torch

    return ctypes.c_void_p(int(torch.cuda.current_stream().cuda_stream))


def _noalloc(fa, q, k, v, o, shape, causal):
    import torch

    st = fa.lib().fa_launch_attention_unfused_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                                     *shape, int(causal), _stream())
    torch.cuda.synchronize()
    return st


def _with_workspace(fa, q, k, v, shape, causal):
    import torch

    ws = torch.empty(max(1, fa.unfused_workspace_bytes(fa.AttentionShape(*shape)) // 4), dtype=torch.float32,
                     device="cuda")
    o = nan_like(q)
    st = fa.lib().fa_launch_attention_unfused(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                              ws.data_ptr(), *shape, int(causal), _stream())
    torch.cuda.synchronize()
    assert st == 0
    return from_dev(o)


def test_noalloc_matches_workspace_entry(fa, oracle_mod):
    limit = fa.lib().fa_unfused_noalloc_max_workspace_bytes()
    assert limit == 64 << 20
    # two calls in a row, the second smaller; then the largest shape that fits
    cases = [((2, 4, 700, 128), True), ((1, 2, 130, 64), False), ((1, 3, 77, 5), True),
             ((2, 8, 1024, 64), False)]
    for shape, causal in cases:
        B, H, N, D = shape
        assert B * H * N * N * 4 <= limit
        qb, kb, vb = oracle_mod.make_inputs(*shape, seeds={"q": N + 1, "k": N + 2, "v": N + 3})
        q, k, v = to_dev(qb), to_dev(kb), to_dev(vb)
        say("noalloc", shape, causal)
        o = nan_like(q)
        assert _noalloc(fa, q, k, v, o, shape, causal) == 0
        got = from_dev(o)
        want = _with_workspace(fa, q, k, v, shape, causal)
        assert np.array_equal(got, want), (shape, causal)
        # and it is correct on its own terms
        acc = oracle_mod.compare(got.reshape(-1, D), oracle_mod.attention(qb, kb, vb, causal).reshape(-1, D))
        assert acc.passed, (shape, causal, acc)


def test_noalloc_rejects_shapes_past_its_scratch(fa, oracle_mod):
    import torch

    shape = (2, 8, 1025, 64)  # 2*8*1025^2*4 bytes > 64 MiB
    q, k, v = (to_dev(x) for x in oracle_mod.make_inputs(*shape))
    o = nan_like(q)
    fa.get_last_error()
    say("noalloc over the limit", shape)
    assert _noalloc(fa, q, k, v, o, shape, False) == 1  # hipErrorInvalidValue, nothing launched
    assert fa.get_last_error() == 1
    torch.cuda.synchronize()
    assert np.all(from_dev(o) == 0xFFFF)
    # empty shape: success, no launch
    assert fa.lib().fa_launch_attention_unfused_noalloc(None, None, None, None, 0, 8, 64, 64, 0, _stream()) == 0
