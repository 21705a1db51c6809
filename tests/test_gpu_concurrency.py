"""Concurrent launches: the launchers keep no state (include/flash_attention.h
callers may launch from any host thread on any stream; the reference's
launchers are reentrant). Two host threads, each with its own stream and its
own inputs, launch the fused and unfused kernels repeatedly at the same time;
every output must equal the same launch run alone, bit for bit."""
import threading

import numpy as np
import pytest

from gpu_common import from_dev, nan_like, run, say, to_dev
from test_gpu_parity import fa  # noqa: F401 (fa: fixture)

pytestmark = pytest.mark.gpu


def test_two_threads_two_streams(fa, oracle_mod):
    import torch

    cases = [((2, 4, 777, 64), True, "v3_mfma"), ((1, 3, 1024, 128), False, "v3_mfma"),
             ((1, 2, 300, 64), True, "v0_unfused"), ((2, 2, 513, 128), True, "v3_256"),
             ((1, 4, 900, 64), False, "v3_64x4"), ((2, 3, 1000, 64), True, "v3_128x4")]
    inputs, alone = [], []
    for i, (shape, causal, kernel) in enumerate(cases):
        q, k, v = (to_dev(x) for x in oracle_mod.make_inputs(*shape, seeds={"q": 70 + i, "k": 80 + i, "v": 90 + i}))
        inputs.append((q, k, v))
        say("concurrency alone", shape, causal, kernel)
        alone.append(from_dev(run(fa, kernel, q, k, v, causal)))
    torch.cuda.synchronize()

    errors = []

    def worker(indices):
        try:
            stream = torch.cuda.Stream()
            for _ in range(5):
                for i in indices:
                    shape, causal, kernel = cases[i]
                    q, k, v = inputs[i]
                    with torch.cuda.stream(stream):
                        o = run(fa, kernel, q, k, v, causal, stream=stream, out=nan_like(q))
                    if not np.array_equal(from_dev(o), alone[i]):
                        errors.append((i, shape, causal, kernel))
        except Exception as exc:  # reported below, not lost in the thread
            errors.append(repr(exc))

    say("concurrency threads")
    # every case runs in a thread, the two head_dim-64 four-group
    # configurations (64, 4) and the (128, 4) list layout included
    threads = [threading.Thread(target=worker, args=([0, 2, 4],)), threading.Thread(target=worker, args=([1, 3, 5],))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a launch thread did not finish"
    assert not errors, errors
