"""HIP graph capture of the launches: the fused and unfused entry points
allocate nothing and never synchronise, so a caller can capture them into a
graph (torch.cuda.CUDAGraph records the kernels launched on its capture
stream). Each graph is replayed several times with eager work and host
synchronisations between the replays (O refilled with NaN), and every replay
must equal the eager launch bit for bit."""
import numpy as np
import pytest

from gpu_common import from_dev, run, say, to_dev
from test_gpu_parity import check, fa  # noqa: F401 (fa: fixture)

pytestmark = pytest.mark.gpu


def _capture_and_replay(fa, launch, q, reference, replays=4):
    import torch

    o = torch.empty_like(q)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up launch off the capture stream
        launch(o, side)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch(o, torch.cuda.current_stream())
    for _ in range(replays):
        o.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(from_dev(o), reference)


@pytest.mark.parametrize("B,H,N,D,causal", [(2, 4, 1000, 64, False), (1, 2, 513, 128, True), (1, 3, 300, 64, True)])
def test_fused_launch_replays_in_a_graph(fa, oracle_mod, B, H, N, D, causal):
    qb, kb, vb = oracle_mod.make_inputs(B, H, N, D, seeds={"q": 61, "k": 62, "v": 63})
    q, k, v = to_dev(qb), to_dev(kb), to_dev(vb)
    shape = fa.AttentionShape(B, H, N, D)
    eager = from_dev(run(fa, "v3_mfma", q, k, v, causal))
    check(oracle_mod, eager, oracle_mod.attention(qb, kb, vb, causal), f"graph eager {(B, H, N, D, causal)}")
    say("graph fused", B, H, N, D, causal)

    def launch(o, stream):
        assert fa.launch_attention_tensorcore_v3(q, k, v, o, shape, causal, stream=stream)

    _capture_and_replay(fa, launch, q, eager)


def test_pinned_configurations_replay_in_a_graph(fa, oracle_mod):
    """Every pinned fused configuration at head_dim 64 (the four-group ones,
    the list layout's moving waves and LDS merge included), captured and
    replayed, causal and dense."""
    B, H, N, D = 2, 3, 1000, 64
    qb, kb, vb = oracle_mod.make_inputs(B, H, N, D, seeds={"q": 64, "k": 65, "v": 66})
    q, k, v = to_dev(qb), to_dev(kb), to_dev(vb)
    shape = fa.AttentionShape(B, H, N, D)
    for name, (rows, groups) in fa.FUSED_CONFIGS.items():
        for causal in (True, False):
            eager = from_dev(run(fa, name, q, k, v, causal))
            say("graph pinned", name, causal)

            def launch(o, stream, rows=rows, groups=groups, causal=causal):
                assert fa.launch_attention_fused_groups(q, k, v, o, shape, causal, rows, groups, stream=stream)

            _capture_and_replay(fa, launch, q, eager)


def test_unfused_launch_replays_in_a_graph(fa, oracle_mod):
    import torch

    B, H, N, D = 1, 2, 300, 64
    qb, kb, vb = oracle_mod.make_inputs(B, H, N, D)
    q, k, v = to_dev(qb), to_dev(kb), to_dev(vb)
    shape = fa.AttentionShape(B, H, N, D)
    ws = torch.empty(fa.unfused_workspace_bytes(shape) // 4, dtype=torch.float32, device="cuda")
    for causal in (False, True):
        eager = from_dev(run(fa, "v0_unfused", q, k, v, causal))
        say("graph unfused", causal)

        def launch(o, stream):
            assert fa.launch_attention_unfused(q, k, v, o, ws, shape, causal, stream=stream)

        _capture_and_replay(fa, launch, q, eager)
