"""Synthetic input generation for benchmarks and callers that need seeded
Q/K/V tensors in the [batch, heads, seq_len, head_dim] bf16 layout.

Uniform[-1,1) family: a SplitMix64 stream (Steele, Lea, Flood, "Fast
splittable pseudorandom number generators", OOPSLA 2014) seeded with the
tensor's seed; draw i takes the top 24 bits of output i as u in [0,1) on the
2^-24 grid (exact in binary32), x = 2u - 1 (exact), rounded to bf16 with
round-to-nearest-even. Per-tensor seeds follow the reference's seed values
(Q 11, K 22, V 33; benchmarks/bench_flash_attention.cu:528-530), not its
normal distribution.

Vectorised with numpy uint64 arithmetic (wrapping modulo 2^64, as the
generator's definition requires): draw i is the mix of seed + (i+1)*gamma.
"""
from __future__ import annotations

import numpy as np

SEEDS = {"q": 11, "k": 22, "v": 33}

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Outputs start .. start+n-1 of SplitMix64(seed)."""
    idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + idx * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns, for finite inputs."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    r = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return r.astype(np.uint16)


def fill_uniform(shape, seed: int, chunk: int = 1 << 22) -> np.ndarray:
    """bf16 bit patterns (uint16) of `shape`, uniform[-1,1) from SplitMix64(seed)."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.uint16)
    for start in range(0, n, chunk):
        m = min(chunk, n - start)
        z = _splitmix64(seed, m, start)
        u = (z >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
        out[start:start + m] = _f32_to_bf16_bits(np.float32(2.0) * u - np.float32(1.0))
    return out.reshape(shape)


def fill_normal(shape, seed: int, sigma: float = 1.0, chunk: int = 1 << 21) -> np.ndarray:
    """bf16 bit patterns of `shape`, N(0, sigma^2) by Box-Muller on SplitMix64(seed):
    draw i takes outputs 2i and 2i+1 as u1, u2 on the 2^-53 grid and gives
    sigma * sqrt(-2 log(1 - u1)) * cos(2 pi u2) in binary64, rounded to binary32, then to bf16 (RNE)."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.uint16)
    two_pi = 6.283185307179586
    for start in range(0, n, chunk):
        m = min(chunk, n - start)
        z = _splitmix64(seed, 2 * m, 2 * start)
        u = (z >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
        radius = np.sqrt(-2.0 * np.log1p(-u[0::2]))
        out[start:start + m] = _f32_to_bf16_bits((sigma * radius * np.cos(two_pi * u[1::2])).astype(np.float32))
    return out.reshape(shape)


def make_stress_inputs(batch: int, heads: int, seq_len: int, head_dim: int, seeds=None):
    """BASELINE's long-sequence stress family: Q and K ~ N(0, 3^2), V uniform[-1,1)."""
    s = dict(SEEDS)
    if seeds:
        s.update(seeds)
    shape = (batch, heads, seq_len, head_dim)
    return fill_normal(shape, s["q"], 3.0), fill_normal(shape, s["k"], 3.0), fill_uniform(shape, s["v"])


def make_uniform_inputs(batch: int, heads: int, seq_len: int, head_dim: int, seeds=None):
    """(q, k, v) uint16 bf16 bit arrays [B,H,N,D] of the uniform family."""
    s = dict(SEEDS)
    if seeds:
        s.update(seeds)
    shape = (batch, heads, seq_len, head_dim)
    return fill_uniform(shape, s["q"]), fill_uniform(shape, s["k"]), fill_uniform(shape, s["v"])


def to_device(bits: np.ndarray, device="cuda"):
    """A torch bf16 tensor on `device` holding the given bf16 bit patterns."""
    import torch

    return torch.from_numpy(bits.view(np.int16)).to(device).view(torch.bfloat16)
