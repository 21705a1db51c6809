"""TEST INFRASTRUCTURE — the CPU FP64 oracle (checker), never the product.

ctypes/numpy wrapper over ``oracle/liboracle.so`` (built from ``oracle.cpp``
by ``oracle/Makefile``). Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module.

The C++ source restates the reference's CPU oracle and comparator
(``benchmarks/bench_flash_attention.cu:86-231``); see the citations there.
bf16 tensors cross this boundary as ``numpy.uint16`` bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


class _Accuracy(ctypes.Structure):
    _fields_ = [
        ("vs_double", ctypes.c_double),
        ("row_scaled", ctypes.c_double),
        ("max_abs", ctypes.c_double),
        ("ulp", ctypes.c_double),
        ("abs_gate", ctypes.c_double),
        ("output_nan", ctypes.c_int64),
        ("output_inf", ctypes.c_int64),
        ("reference_nan", ctypes.c_int64),
        ("reference_inf", ctypes.c_int64),
        ("passed_ulp", ctypes.c_int32),
        ("passed_abs", ctypes.c_int32),
    ]


@dataclass
class Accuracy:
    """Mirror of the reference's ``Accuracy`` (bench_flash_attention.cu:148-164)
    plus ``abs_gate`` = max |err| / (2^-7 * row scale) (passes when <= 1)."""

    vs_double: float
    row_scaled: float
    max_abs: float
    ulp: float
    abs_gate: float
    output_nan: int
    output_inf: int
    reference_nan: int
    reference_inf: int
    passed_ulp: bool
    passed_abs: bool

    @property
    def passed(self) -> bool:
        return self.passed_ulp and self.passed_abs


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (g++)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "liboracle.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        u16p = ctypes.POINTER(ctypes.c_uint16)
        f64p = ctypes.POINTER(ctypes.c_double)
        i64p = ctypes.POINTER(ctypes.c_int64)
        L.fa_oracle_bf16_from_float.restype = ctypes.c_uint16
        L.fa_oracle_bf16_from_float.argtypes = [ctypes.c_float]
        L.fa_oracle_bf16_from_float_slow.restype = ctypes.c_uint16
        L.fa_oracle_bf16_from_float_slow.argtypes = [ctypes.c_float]
        L.fa_oracle_float_from_bf16.restype = ctypes.c_float
        L.fa_oracle_float_from_bf16.argtypes = [ctypes.c_uint16]
        L.fa_oracle_bf16_from_float_array.restype = None
        L.fa_oracle_bf16_from_float_array.argtypes = [ctypes.POINTER(ctypes.c_float), u16p, ctypes.c_int64]
        L.fa_oracle_bf16_ulp.restype = ctypes.c_float
        L.fa_oracle_bf16_ulp.argtypes = [ctypes.c_float]
        L.fa_oracle_default_scale.restype = ctypes.c_float
        L.fa_oracle_default_scale.argtypes = [ctypes.c_int]
        L.fa_oracle_attention_flops.restype = ctypes.c_double
        L.fa_oracle_attention_flops.argtypes = [ctypes.c_int] * 5
        L.fa_oracle_unfused_workspace_bytes.restype = ctypes.c_uint64
        L.fa_oracle_unfused_workspace_bytes.argtypes = [ctypes.c_int] * 3
        L.fa_oracle_qkvo_bytes.restype = ctypes.c_double
        L.fa_oracle_qkvo_bytes.argtypes = [ctypes.c_int] * 4
        L.fa_oracle_unfused_score_bytes.restype = ctypes.c_double
        L.fa_oracle_unfused_score_bytes.argtypes = [ctypes.c_int] * 3
        L.fa_oracle_blocked_kv_hbm_bytes.restype = ctypes.c_double
        L.fa_oracle_blocked_kv_hbm_bytes.argtypes = [ctypes.c_int] * 7
        L.fa_oracle_fill_uniform.restype = None
        L.fa_oracle_fill_uniform.argtypes = [u16p, ctypes.c_int64, ctypes.c_uint64]
        L.fa_oracle_fill_normal.restype = None
        L.fa_oracle_fill_normal.argtypes = [u16p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_double]
        L.fa_oracle_fill_normal_mt19937.restype = None
        L.fa_oracle_fill_normal_mt19937.argtypes = [u16p, ctypes.c_int64, ctypes.c_uint32]
        L.fa_oracle_mt19937_10000th.restype = ctypes.c_uint32
        L.fa_oracle_mt19937_10000th.argtypes = []
        L.fa_oracle_attention.restype = ctypes.c_int
        L.fa_oracle_attention.argtypes = [u16p, u16p, u16p, f64p] + [ctypes.c_int] * 5 + [i64p, ctypes.c_int64, ctypes.c_int]
        L.fa_oracle_attention_scalar.restype = ctypes.c_int
        L.fa_oracle_attention_scalar.argtypes = L.fa_oracle_attention.argtypes
        L.fa_oracle_compare.restype = None
        L.fa_oracle_compare.argtypes = [u16p, f64p, ctypes.c_int64, ctypes.c_int, ctypes.POINTER(_Accuracy)]
        L.fa_oracle_quantile_sorted.restype = ctypes.c_double
        L.fa_oracle_quantile_sorted.argtypes = [f64p, ctypes.c_int64, ctypes.c_double]
        _lib = L
    return _lib


def _u16(a: np.ndarray):
    assert a.dtype == np.uint16 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


def _f64(a: np.ndarray):
    assert a.dtype == np.float64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


# ---------------------------------------------------------------- bf16 helpers
def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, IEEE round-to-nearest-even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().fa_oracle_bf16_from_float_array(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), _u16(out), x.size)
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_ulp(value: float) -> float:
    return float(lib().fa_oracle_bf16_ulp(value))


def default_scale(head_dim: int) -> float:
    return float(lib().fa_oracle_default_scale(head_dim))


def attention_flops(batch, heads, seq_len, head_dim, causal) -> float:
    """Reference convention: 4 * pairs * D * B * H, causal pairs N(N+1)/2."""
    return float(lib().fa_oracle_attention_flops(batch, heads, seq_len, head_dim, int(causal)))


# ---------------------------------------------------------------- inputs
SEEDS = {"q": 11, "k": 22, "v": 33}


def fill_uniform(shape, seed: int) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint16)
    lib().fa_oracle_fill_uniform(_u16(out), out.size, seed)
    return out


def fill_normal(shape, seed: int, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint16)
    lib().fa_oracle_fill_normal(_u16(out), out.size, seed, sigma)
    return out


def fill_normal_mt19937(shape, seed: int) -> np.ndarray:
    """The reference's own generator (bench_flash_attention.cu:86-92)."""
    out = np.empty(shape, dtype=np.uint16)
    lib().fa_oracle_fill_normal_mt19937(_u16(out), out.size, seed)
    return out


def make_inputs(batch, heads, seq_len, head_dim, family: str = "uniform", seeds=None):
    """Q, K, V bf16 bit arrays [B,H,N,D] for a named input family.

    Families: uniform (BASELINE), normal_mt19937 (the reference's inputs),
    stress (Q,K ~ N(0, 3^2), V uniform), zeros (Q=K=0, V uniform), ones,
    ramp (V[i] = (i mod D) - D/2, Q/K uniform), scaled (Q,K uniform x4).
    The reference's own five boundary families
    (kernels/ablation/experiments.cu:283-289), all on its normal(0,1)
    mt19937 inputs with seeds 11/22/33: ref_normal (that base), ref_zeros
    (Q=K=V=0), ones (shared with the list above), ref_ramp (V[i] =
    (i mod D) - D/2 over the normal Q and K) and ref_scaled (the normal Q
    and K times 4, rounded to bf16 again: exact, a power of two; logits of
    standard deviation about 16 at the 1/sqrt(D) scale).
    """
    shape = (batch, heads, seq_len, head_dim)
    s = dict(SEEDS)
    if seeds:
        s.update(seeds)
    if family == "uniform":
        return fill_uniform(shape, s["q"]), fill_uniform(shape, s["k"]), fill_uniform(shape, s["v"])
    if family == "normal_mt19937":
        return (fill_normal_mt19937(shape, s["q"]), fill_normal_mt19937(shape, s["k"]),
                fill_normal_mt19937(shape, s["v"]))
    if family == "stress":
        return fill_normal(shape, s["q"], 3.0), fill_normal(shape, s["k"], 3.0), fill_uniform(shape, s["v"])
    if family == "zeros":
        z = np.zeros(shape, dtype=np.uint16)
        return z, z.copy(), fill_uniform(shape, s["v"])
    if family == "ones":
        one = np.full(shape, 0x3F80, dtype=np.uint16)
        return one, one.copy(), one.copy()
    if family == "ramp":
        idx = np.arange(batch * heads * seq_len * head_dim, dtype=np.int64).reshape(shape)
        ramp = (idx % head_dim - head_dim // 2).astype(np.float32)
        return fill_uniform(shape, s["q"]), fill_uniform(shape, s["k"]), bf16_bits(ramp)
    if family in ("ref_normal", "ref_ramp", "ref_scaled"):
        q, k, v = (fill_normal_mt19937(shape, s["q"]), fill_normal_mt19937(shape, s["k"]),
                   fill_normal_mt19937(shape, s["v"]))
        if family == "ref_ramp":
            idx = np.arange(batch * heads * seq_len * head_dim, dtype=np.int64).reshape(shape)
            v = bf16_bits((idx % head_dim - head_dim // 2).astype(np.float32))
        elif family == "ref_scaled":
            q = bf16_bits(bf16_to_f32(q) * 4.0)
            k = bf16_bits(bf16_to_f32(k) * 4.0)
        return q, k, v
    if family == "ref_zeros":
        z = np.zeros(shape, dtype=np.uint16)
        return z, z.copy(), z.copy()
    if family == "scaled":
        q = bf16_bits(bf16_to_f32(fill_uniform(shape, s["q"])) * 4.0)
        k = bf16_bits(bf16_to_f32(fill_uniform(shape, s["k"])) * 4.0)
        return q, k, fill_uniform(shape, s["v"])
    raise ValueError(f"unknown input family {family!r}")


# ---------------------------------------------------------------- the oracle
def attention(q, k, v, causal: bool, rows=None, threads: int = 0, scalar: bool = False) -> np.ndarray:
    """FP64 attention (bench_flash_attention.cu:105-145).

    q, k, v: uint16 bf16 bits [B,H,N,D]. rows: optional global row ids
    (bh*N + query); returns float64 [len(rows), D], else [B,H,N,D].
    scalar: compute row by row with the direct restatement (slow; the pin of
    the default blocked path, which must agree with it bit for bit).
    """
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    B, H, N, D = q.shape
    assert k.shape == q.shape and v.shape == q.shape
    fn = lib().fa_oracle_attention_scalar if scalar else lib().fa_oracle_attention
    if rows is None:
        out = np.empty((B, H, N, D), dtype=np.float64)
        rc = fn(_u16(q), _u16(k), _u16(v), _f64(out), B, H, N, D, int(causal),
                                       None, 0, threads)
    else:
        rows = np.ascontiguousarray(rows, dtype=np.int64)
        out = np.empty((rows.size, D), dtype=np.float64)
        rc = fn(_u16(q), _u16(k), _u16(v), _f64(out), B, H, N, D, int(causal),
                                       rows.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), rows.size, threads)
    if rc != 0:
        raise ValueError("fa_oracle_attention rejected its arguments")
    return out


def compare(got_bits: np.ndarray, ref: np.ndarray) -> Accuracy:
    """Reference comparator (bench_flash_attention.cu:167-218) over rows of D."""
    got_bits = np.ascontiguousarray(got_bits, dtype=np.uint16)
    ref = np.ascontiguousarray(ref, dtype=np.float64)
    D = ref.shape[-1]
    assert got_bits.size == ref.size
    acc = _Accuracy()
    lib().fa_oracle_compare(_u16(got_bits), _f64(ref), ref.size // D, D, ctypes.byref(acc))
    return Accuracy(
        acc.vs_double, acc.row_scaled, acc.max_abs, acc.ulp, acc.abs_gate,
        acc.output_nan, acc.output_inf, acc.reference_nan, acc.reference_inf,
        bool(acc.passed_ulp), bool(acc.passed_abs),
    )


def sample_rows(batch, heads, seq_len, rows_per_slab: int = 64, tile: int = 128, seed: int = 7) -> np.ndarray:
    """Stratified row sample for shapes too large for the full oracle: in every
    (b,h) slab, all rows of the first and last query tiles plus seeded random
    rows (which land in interior and diagonal tiles alike)."""
    rng = np.random.default_rng(seed)
    rows = []
    for bh in range(batch * heads):
        base = bh * seq_len
        first = np.arange(min(tile, seq_len))
        last = np.arange(max(0, seq_len - tile), seq_len)
        rand = rng.integers(0, seq_len, size=rows_per_slab)
        rows.append(base + np.unique(np.concatenate([first, last, rand])))
    return np.concatenate(rows).astype(np.int64)


def quantile_sorted(sorted_values, p: float) -> float:
    a = np.ascontiguousarray(sorted_values, dtype=np.float64)
    return float(lib().fa_oracle_quantile_sorted(_f64(a), a.size, p))


def splitmix64(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint64)
    L = lib()
    L.fa_oracle_splitmix64.restype = None
    L.fa_oracle_splitmix64.argtypes = [ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64), ctypes.c_int64]
    L.fa_oracle_splitmix64(seed, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)), n)
    return out


def rne_exhaustive_mismatches(threads: int = 0) -> int:
    L = lib()
    L.fa_oracle_rne_exhaustive_mismatches.restype = ctypes.c_uint64
    L.fa_oracle_rne_exhaustive_mismatches.argtypes = [ctypes.c_int]
    return int(L.fa_oracle_rne_exhaustive_mismatches(threads))
