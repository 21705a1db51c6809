"""Helpers shared by the GPU parity tests: move bf16 bit arrays to the device,
launch a kernel through the C ABI (ctypes), read the result back. Outputs are
prefilled with 0xFFFF (bf16 NaN) so an unwritten element fails the check
(benchmarks/bench_flash_attention.cu:555-556)."""
import os
import sys

import numpy as np

HOST_THREADS = max(1, min(16, os.cpu_count() or 1))


def to_dev(bits: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


def from_dev(t) -> np.ndarray:
    import torch

    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def nan_like(t):
    import torch

    return torch.full(t.shape, -1, dtype=torch.int16, device=t.device).view(torch.bfloat16)


def say(*parts):
    """Name the case before a GPU step (flushed, so a fault still shows it)."""
    print(*parts, flush=True)
    sys.stdout.flush()


def run(fa, kernel: str, q, k, v, causal: bool, stream=None, out=None):
    """Launch `kernel` on device tensors and return the output tensor."""
    import torch

    shape = fa.AttentionShape(*q.shape)
    o = nan_like(q) if out is None else out
    st = stream if stream is not None else torch.cuda.current_stream()
    if kernel == "v0_unfused":
        ws = torch.empty(max(1, fa.unfused_workspace_bytes(shape) // 4), dtype=torch.float32, device=q.device)
        assert fa.launch_attention_unfused(q, k, v, o, ws, shape, causal, stream=st)
    elif kernel == "v3_mfma":
        assert fa.launch_attention_tensorcore_v3(q, k, v, o, shape, causal, stream=st)
    elif kernel == "v3b_mfma":
        assert fa.launch_attention_tensorcore_v3b(q, k, v, o, shape, causal, stream=st)
    elif kernel == "v3_128":
        assert fa.launch_attention_fused(q, k, v, o, shape, causal, rows_per_block=128, stream=st)
    elif kernel == "v3_256":
        assert fa.launch_attention_fused(q, k, v, o, shape, causal, rows_per_block=256, stream=st)
    elif kernel in ("v3_64x4", "v3_128x4"):
        rows, groups = fa.FUSED_CONFIGS[kernel]
        assert fa.launch_attention_fused_groups(q, k, v, o, shape, causal, rows, groups, stream=st)
    else:
        raise ValueError(kernel)
    torch.cuda.synchronize()
    return o


def run_bits(fa, kernel, qb, kb, vb, causal):
    q, k, v = to_dev(qb), to_dev(kb), to_dev(vb)
    return from_dev(run(fa, kernel, q, k, v, causal))


# v3_mfma picks its workgroup configuration from the shape (64 rows for
# grids that leave CUs idle); v3_128, v3_256, v3_64x4 and v3_128x4 pin the
# 128-row, the one-group 256-row, the four-group 64-row and the four-group
# 128-row list configurations, so every shape exercises each (the last two
# exist for head_dim 64 only).
KERNELS = ["v0_unfused", "v3_mfma", "v3b_mfma", "v3_128", "v3_256", "v3_64x4", "v3_128x4"]
FUSED_KERNELS = ["v3_mfma", "v3b_mfma", "v3_128", "v3_256", "v3_64x4", "v3_128x4"]


def supports(kernel: str, head_dim: int) -> bool:
    """Whether `kernel` handles head_dim (the four-group configurations'
    stage sets fit LDS at head_dim 64 only)."""
    return not (kernel in ("v3_64x4", "v3_128x4") and head_dim != 64)


def kernels_for(head_dim: int, kernels=None):
    return [k for k in (KERNELS if kernels is None else kernels) if supports(k, head_dim)]
