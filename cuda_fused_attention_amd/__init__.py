"""MI355X-native BF16 attention forward — Python host mirror of the C ABI.

The product is ``libfa_mi355x.so`` (HIP kernels for gfx950 + the C ABI of
``include/fa_mi355x.h`` + the C++ interface of ``include/flash_attention.h``).
This module binds the C ABI with ctypes and mirrors the reference's launch
interface (``include/flash_attention.h:9-109`` of RichterWang/cuda_fused_attention)
for Python callers and tests: the same function names, the same argument
meaning ([batch, heads, seq_len, head_dim] contiguous bf16, caller-owned
buffers, stream-ordered launches).

Error behaviour: a non-zero HIP status raises :class:`FaError`; an
unsupported head_dim launches nothing and returns ``False`` (the reference
returns silently, ``kernels/v3/v3_tensorcore.cu:743-744``). There is no CPU
fallback: if the library is missing, :func:`lib` raises.

PyTorch is used only as the allocator / stream provider; any object with a
device pointer (an ``int``) works as well.
"""
from __future__ import annotations

import ctypes
import os
from typing import NamedTuple, Optional

from . import _build

LIB_PATH = _build.LIB_PATH
FA_ERROR_UNSUPPORTED = 801

# kernel ids for fa_time_launches / fa_time_batch
KERNEL_UNFUSED = 0
KERNEL_V3 = 1
KERNEL_V3B = 2
KERNEL_V3_128 = 3  # the fused forward pinned to 128 rows per workgroup
KERNEL_V3_256 = 4  # pinned to 256 rows per workgroup (one wave group)
KERNEL_V3_64X4 = 5  # pinned to 64 rows per workgroup split over four KV groups (head_dim 64)
KERNEL_V3_128X4 = 6  # pinned to 128 rows (two half blocks) walked as one list by four KV groups (head_dim 64)
KERNEL_IDS = {"v0_unfused": KERNEL_UNFUSED, "v3_mfma": KERNEL_V3, "v3b_mfma": KERNEL_V3B, "v3_128": KERNEL_V3_128,
              "v3_256": KERNEL_V3_256, "v3_64x4": KERNEL_V3_64X4, "v3_128x4": KERNEL_V3_128X4}
# (rows per workgroup, KV groups) of each pinned fused configuration
FUSED_CONFIGS = {"v3b_mfma": (64, 2), "v3_128": (128, 2), "v3_256": (256, 1), "v3_64x4": (64, 4),
                 "v3_128x4": (128, 4)}

_lib = None


class FaError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what} failed with HIP status {status}")
        self.status = status


class AttentionShape(NamedTuple):
    """include/flash_attention.h:12-18"""

    batch: int
    heads: int
    seq_len: int
    head_dim: int


class TilingInfo(ctypes.Structure):
    """fa_tiling_info: the reference's FusedTilingInfo (include/flash_attention.h:60-72)
    plus AGPRs, waves per workgroup and the CU count."""

    _fields_ = [
        (name, ctypes.c_int)
        for name in (
            "supported", "block_size", "tile_kv", "rows_per_block", "shared_bytes_per_block",
            "registers_per_thread", "local_bytes_per_thread", "max_blocks_per_sm",
            "device_shared_bytes_per_sm", "shared_limited_blocks_per_sm", "agprs_per_thread",
            "waves_per_block", "compute_units", "kv_groups",
        )
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


# Every symbol include/fa_mi355x.h declares, with its ctypes signature.
_vp = ctypes.c_void_p
_i = ctypes.c_int
_SIGNATURES = {
    "fa_get_last_error": (_i, []),
    "fa_peek_at_last_error": (_i, []),
    "fa_default_scale": (ctypes.c_float, [_i]),
    "fa_attention_flops": (ctypes.c_double, [_i, _i, _i, _i, _i]),
    "fa_unfused_workspace_bytes": (ctypes.c_size_t, [_i, _i, _i, _i]),
    "fa_launch_attention_unfused": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "fa_launch_attention_unfused_noalloc": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "fa_unfused_noalloc_max_workspace_bytes": (ctypes.c_size_t, []),
    "fa_launch_softmax_rows_inplace": (_i, [_vp, _i, _i, _vp]),
    "fa_launch_attention_unfused_profile": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp]),
    "fa_tensorcore_v3_supported": (_i, [_i]),
    "fa_launch_attention_tensorcore_v3": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "fa_launch_attention_fused": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "fa_query_fused": (_i, [_i, _i, ctypes.POINTER(TilingInfo)]),
    "fa_launch_attention_fused_groups": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "fa_query_fused_groups": (_i, [_i, _i, _i, ctypes.POINTER(TilingInfo)]),
    "fa_query_fused_config": (_i, [_i, _i, _i, _i, ctypes.POINTER(TilingInfo)]),
    "fa_query_tensorcore_v3_shape": (_i, [_i, _i, _i, _i, _i, ctypes.POINTER(TilingInfo)]),
    "fa_tensorcore_v3_rows_per_block": (_i, [_i, _i, _i, _i, _i]),
    "fa_tensorcore_v3_config": (_i, [_i, _i, _i, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "fa_query_tensorcore_v3": (_i, [_i, ctypes.POINTER(TilingInfo)]),
    "fa_tensorcore_v3_hbm_bytes": (ctypes.c_double, [_i, _i, _i, _i, _i]),
    "fa_tensorcore_v3b_supported": (_i, [_i]),
    "fa_launch_attention_tensorcore_v3b": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "fa_query_tensorcore_v3b": (_i, [_i, ctypes.POINTER(TilingInfo)]),
    "fa_tensorcore_v3b_hbm_bytes": (ctypes.c_double, [_i, _i, _i, _i, _i]),
    "fa_time_launches": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i,
                              ctypes.POINTER(ctypes.c_float), _vp]),
    "fa_time_batch": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i,
                           ctypes.POINTER(ctypes.c_float), _vp]),
    "fa_mfma_peak_records_bytes": (ctypes.c_size_t, []),
    "fa_mfma_peak": (_i, [_vp, _i, _i, _vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double), _vp]),
    "fa_build_info": (ctypes.c_char_p, []),
}


def lib() -> ctypes.CDLL:
    """Load libfa_mi355x.so (in-tree). Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "(hipcc, gfx950). There is no CPU fallback.")
        # PyTorch-ROCm ships its own libamdhip64.so.7. Load it first so this
        # library binds to the HIP runtime already in the process (by soname)
        # instead of pulling a second runtime from /opt/rocm, which then finds
        # no device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(x) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return int(x.data_ptr())


def _stream(stream) -> Optional[int]:
    if stream is None:
        import torch

        return int(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return stream
    return int(stream.cuda_stream)


def _check(status: int, what: str) -> bool:
    if status == 0:
        return True
    if status == FA_ERROR_UNSUPPORTED:
        return False
    raise FaError(status, what)


def _shape_of(shape) -> AttentionShape:
    return shape if isinstance(shape, AttentionShape) else AttentionShape(*shape)


# ---------------------------------------------------------------- host helpers
def default_scale(head_dim: int) -> float:
    """include/flash_attention.h:21-24"""
    return float(lib().fa_default_scale(head_dim))


def attention_flops(shape, causal: bool) -> float:
    """kernels/v0_unfused.cu:118-126 (causal pairs N(N+1)/2)."""
    s = _shape_of(shape)
    return float(lib().fa_attention_flops(s.batch, s.heads, s.seq_len, s.head_dim, int(causal)))


def unfused_workspace_bytes(shape) -> int:
    """kernels/v0_unfused.cu:128-131"""
    s = _shape_of(shape)
    return int(lib().fa_unfused_workspace_bytes(s.batch, s.heads, s.seq_len, s.head_dim))


def tensorcore_v3_supported(head_dim: int) -> bool:
    return bool(lib().fa_tensorcore_v3_supported(head_dim))


def tensorcore_v3b_supported(head_dim: int) -> bool:
    return bool(lib().fa_tensorcore_v3b_supported(head_dim))


def query_tensorcore_v3(head_dim: int) -> dict:
    info = TilingInfo()
    _check(lib().fa_query_tensorcore_v3(head_dim, ctypes.byref(info)), "fa_query_tensorcore_v3")
    return info.as_dict()


def query_fused(head_dim: int, rows_per_block: int) -> dict:
    info = TilingInfo()
    _check(lib().fa_query_fused(head_dim, rows_per_block, ctypes.byref(info)), "fa_query_fused")
    return info.as_dict()


def query_fused_groups(head_dim: int, rows_per_block: int, kv_groups: int) -> dict:
    info = TilingInfo()
    _check(lib().fa_query_fused_groups(head_dim, rows_per_block, kv_groups, ctypes.byref(info)),
           "fa_query_fused_groups")
    return info.as_dict()


def query_fused_config(head_dim: int, rows_per_block: int, kv_groups: int, causal: bool) -> dict:
    """Resources of the kernel (rows_per_block, kv_groups) runs with this mask."""
    info = TilingInfo()
    _check(lib().fa_query_fused_config(head_dim, rows_per_block, kv_groups, int(causal), ctypes.byref(info)),
           "fa_query_fused_config")
    return info.as_dict()


def query_tensorcore_v3_shape(shape, causal: bool) -> dict:
    """Resources of the kernel the v3 entry launches at this shape and mask."""
    s = _shape_of(shape)
    info = TilingInfo()
    _check(lib().fa_query_tensorcore_v3_shape(s.batch, s.heads, s.seq_len, s.head_dim, int(causal),
                                              ctypes.byref(info)), "fa_query_tensorcore_v3_shape")
    return info.as_dict()


def query_tensorcore_v3b(head_dim: int) -> dict:
    info = TilingInfo()
    _check(lib().fa_query_tensorcore_v3b(head_dim, ctypes.byref(info)), "fa_query_tensorcore_v3b")
    return info.as_dict()


def tensorcore_v3_hbm_bytes(shape, causal: bool) -> float:
    s = _shape_of(shape)
    return float(lib().fa_tensorcore_v3_hbm_bytes(s.batch, s.heads, s.seq_len, s.head_dim, int(causal)))


def tensorcore_v3b_hbm_bytes(shape, causal: bool) -> float:
    s = _shape_of(shape)
    return float(lib().fa_tensorcore_v3b_hbm_bytes(s.batch, s.heads, s.seq_len, s.head_dim, int(causal)))


def tensorcore_v3_rows_per_block(shape, causal: bool) -> int:
    """Query rows per workgroup the v3 entry runs at this shape (64, 128 or 256;
    tensorcore_v3_config also gives the KV groups)."""
    s = _shape_of(shape)
    return int(lib().fa_tensorcore_v3_rows_per_block(s.batch, s.heads, s.seq_len, s.head_dim, int(causal)))


def tensorcore_v3_config(shape, causal: bool):
    """(rows per workgroup, KV wave groups) the v3 entry runs at this shape,
    or None for an unsupported head_dim."""
    s = _shape_of(shape)
    rows, groups = ctypes.c_int(), ctypes.c_int()
    st = lib().fa_tensorcore_v3_config(s.batch, s.heads, s.seq_len, s.head_dim, int(causal), ctypes.byref(rows),
                                       ctypes.byref(groups))
    if not _check(st, "fa_tensorcore_v3_config"):
        return None
    return rows.value, groups.value


def get_last_error() -> int:
    """The calling thread's last non-zero C-ABI status (reset to 0)."""
    return int(lib().fa_get_last_error())


def peek_at_last_error() -> int:
    return int(lib().fa_peek_at_last_error())


def build_info() -> str:
    return lib().fa_build_info().decode()


# ---------------------------------------------------------------- launchers
def launch_attention_unfused(q, k, v, o, workspace, shape, causal: bool, stream=None) -> bool:
    """include/flash_attention.h:33 — v0: S, softmax, PV; workspace >= unfused_workspace_bytes."""
    s = _shape_of(shape)
    st = lib().fa_launch_attention_unfused(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(workspace), s.batch,
                                           s.heads, s.seq_len, s.head_dim, int(causal), _stream(stream))
    return _check(st, "fa_launch_attention_unfused")


def launch_softmax_rows_inplace(s_buf, rows: int, cols: int, stream=None) -> bool:
    st = lib().fa_launch_softmax_rows_inplace(_ptr(s_buf), rows, cols, _stream(stream))
    return _check(st, "fa_launch_softmax_rows_inplace")


def launch_attention_unfused_profile(q, k, v, o, workspace, shape, causal: bool, events=None, stream=None) -> bool:
    """include/flash_attention_v0_profile.h:20-23. `events`: four torch.cuda.Event
    (enable_timing=True) or raw hipEvent_t ints, in the order qk_start, qk_end,
    softmax_end, pv_end; None records no markers."""
    s = _shape_of(shape)
    ev = None
    if events is not None:
        handles = []
        for e in events:
            if not isinstance(e, int) and int(e.cuda_event) == 0:
                # torch creates the underlying hipEvent_t on first record()
                e.record(stream) if stream is not None else e.record()
            handles.append(e if isinstance(e, int) else int(e.cuda_event))
        if len(handles) != 4:
            raise ValueError("need exactly four events")
        ev = (ctypes.c_void_p * 4)(*handles)
    st = lib().fa_launch_attention_unfused_profile(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(workspace), s.batch,
                                                   s.heads, s.seq_len, s.head_dim, int(causal),
                                                   ctypes.cast(ev, ctypes.c_void_p) if ev is not None else None,
                                                   _stream(stream))
    return _check(st, "fa_launch_attention_unfused_profile")


def launch_attention_tensorcore_v3(q, k, v, o, shape, causal: bool, stream=None) -> bool:
    """include/flash_attention.h:92 — the fused MFMA forward in the workgroup
    configuration tensorcore_v3_config(shape, causal) names."""
    s = _shape_of(shape)
    st = lib().fa_launch_attention_tensorcore_v3(_ptr(q), _ptr(k), _ptr(v), _ptr(o), s.batch, s.heads,
                                                 s.seq_len, s.head_dim, int(causal), _stream(stream))
    return _check(st, "fa_launch_attention_tensorcore_v3")


def launch_attention_fused(q, k, v, o, shape, causal: bool, rows_per_block: int = 0, stream=None) -> bool:
    """The fused forward with a pinned workgroup configuration (no counterpart in
    the reference): rows_per_block 128 (v3), 64 (v3b), 256 (one wave group) or 0
    (the v3 entry's choice)."""
    s = _shape_of(shape)
    st = lib().fa_launch_attention_fused(_ptr(q), _ptr(k), _ptr(v), _ptr(o), s.batch, s.heads, s.seq_len,
                                         s.head_dim, int(causal), int(rows_per_block), _stream(stream))
    return _check(st, "fa_launch_attention_fused")


def launch_attention_fused_groups(q, k, v, o, shape, causal: bool, rows_per_block: int, kv_groups: int,
                                  stream=None) -> bool:
    """The fused forward in a pinned (rows per workgroup, KV groups)
    configuration: (128, 2), (64, 2), (256, 1), or at head_dim 64 (64, 4) and (128, 4)."""
    s = _shape_of(shape)
    st = lib().fa_launch_attention_fused_groups(_ptr(q), _ptr(k), _ptr(v), _ptr(o), s.batch, s.heads, s.seq_len,
                                                s.head_dim, int(causal), int(rows_per_block), int(kv_groups),
                                                _stream(stream))
    return _check(st, "fa_launch_attention_fused_groups")


def launch_attention_tensorcore_v3b(q, k, v, o, shape, causal: bool, stream=None) -> bool:
    """include/flash_attention.h:103 — the fused MFMA forward (64 query rows / workgroup)."""
    s = _shape_of(shape)
    st = lib().fa_launch_attention_tensorcore_v3b(_ptr(q), _ptr(k), _ptr(v), _ptr(o), s.batch, s.heads,
                                                  s.seq_len, s.head_dim, int(causal), _stream(stream))
    return _check(st, "fa_launch_attention_tensorcore_v3b")


# ---------------------------------------------------------------- timing
def time_launches(kernel: str, q, k, v, o, workspace, shape, causal: bool, warmup: int = 5, iters: int = 30,
                  stream=None):
    """benchmarks/bench_flash_attention.cu:265-299: `warmup` launches, sync, then
    `iters` launches each bracketed by hipEvents on the launch stream. Returns
    the per-launch milliseconds in measurement order."""
    s = _shape_of(shape)
    samples = (ctypes.c_float * iters)()
    st = lib().fa_time_launches(KERNEL_IDS[kernel], _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(workspace),
                                s.batch, s.heads, s.seq_len, s.head_dim, int(causal), warmup, iters, samples,
                                _stream(stream))
    if not _check(st, "fa_time_launches"):
        return None
    return [float(x) for x in samples]


def time_batch(kernel: str, q, k, v, o, workspace, shape, causal: bool, iters: int, stream=None) -> Optional[float]:
    """Total milliseconds of `iters` back-to-back launches between one event pair."""
    s = _shape_of(shape)
    total = ctypes.c_float()
    st = lib().fa_time_batch(KERNEL_IDS[kernel], _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(workspace), s.batch,
                             s.heads, s.seq_len, s.head_dim, int(causal), iters, ctypes.byref(total),
                             _stream(stream))
    if not _check(st, "fa_time_batch"):
        return None
    return float(total.value)


def mfma_peak(mfma_per_wave: int = 8192, launches: int = 5, operands=None, stream=None) -> dict:
    """Same-run calibration of the dense bf16 matrix rate the device sustains
    (fa_mfma_peak): every wave of two per SIMD issuing back-to-back MFMAs.
    `operands`: None, or a bf16 CUDA tensor whose first 4096 values the
    MFMA operands are drawn from (the sustained clock depends on the data).
    Returns {"tflops", "clock_ghz", "mfma_per_wave", "launches"}."""
    import torch

    if operands is not None:
        if operands.dtype != torch.bfloat16 or not operands.is_cuda or operands.numel() < 4096:
            raise ValueError("operands must be a CUDA bf16 tensor of at least 4096 values")
        operands = operands.reshape(-1)[:4096].contiguous()

    nbytes = lib().fa_mfma_peak_records_bytes()
    if nbytes == 0:
        raise FaError(0, "fa_mfma_peak_records_bytes (no device)")
    records = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    tf, ghz = ctypes.c_double(), ctypes.c_double()
    st = lib().fa_mfma_peak(_ptr(operands), mfma_per_wave, launches, _ptr(records), ctypes.byref(tf),
                            ctypes.byref(ghz), _stream(stream))
    _check(st, "fa_mfma_peak")
    return {"tflops": tf.value, "clock_ghz": ghz.value, "mfma_per_wave": mfma_per_wave - mfma_per_wave % 8,
            "launches": launches}


def quantile_type7(values, p: float) -> float:
    """benchmarks/bench_flash_attention.cu:243-249 — linear interpolation at (n-1)p."""
    xs = sorted(values)
    index = (len(xs) - 1) * p
    lo = int(index)
    hi = min(lo + 1, len(xs) - 1)
    return xs[lo] + (xs[hi] - xs[lo]) * (index - lo)


def summarize(samples_ms) -> dict:
    """median / q1 / q3 / iqr of raw samples (bench_flash_attention.cu:251-262)."""
    q1 = quantile_type7(samples_ms, 0.25)
    med = quantile_type7(samples_ms, 0.5)
    q3 = quantile_type7(samples_ms, 0.75)
    return {"median_ms": med, "q1_ms": q1, "q3_ms": q3, "iqr_ms": q3 - q1}


# ---------------------------------------------------------------- torch convenience
def attention_forward(q, k, v, causal: bool = False, kernel: str = "v3_mfma", out=None, workspace=None):
    """Run one kernel on torch bf16 CUDA tensors [B,H,N,D]; returns O."""
    import torch

    for t in (q, k, v):
        if t.dtype != torch.bfloat16 or not t.is_cuda or not t.is_contiguous():
            raise ValueError("q, k, v must be contiguous bf16 CUDA tensors")
    shape = AttentionShape(*q.shape)
    o = out if out is not None else torch.empty_like(q)
    if kernel == "v0_unfused":
        ws = workspace
        if ws is None:
            ws = torch.empty(max(1, unfused_workspace_bytes(shape) // 4), dtype=torch.float32, device=q.device)
        launch_attention_unfused(q, k, v, o, ws, shape, causal)
    elif kernel == "v3_mfma":
        if not launch_attention_tensorcore_v3(q, k, v, o, shape, causal):
            raise ValueError(f"head_dim {shape.head_dim} is not supported by the fused kernel")
    elif kernel == "v3b_mfma":
        if not launch_attention_tensorcore_v3b(q, k, v, o, shape, causal):
            raise ValueError(f"head_dim {shape.head_dim} is not supported by the fused kernel")
    elif kernel in ("v3_128", "v3_256", "v3_64x4", "v3_128x4"):
        rows, groups = FUSED_CONFIGS[kernel]
        if not launch_attention_fused_groups(q, k, v, o, shape, causal, rows, groups):
            raise ValueError(f"head_dim {shape.head_dim} is not supported by the {kernel} configuration")
    else:
        raise ValueError(f"unknown kernel {kernel!r}")
    return o
