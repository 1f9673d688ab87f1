"""Deterministic input generators restated from the reference's tests.

Each mirrors one generator of amazingvince/falcon-ocr-cpu so that the parity
tests use the same inputs the reference's own tests use:
  values      src/kernels/tests.rs:6-14 (LCG in [-1, 1))
  att_values  src/kernels/attention/prefill64/tests.rs:4-20 (LCG with signed
              zeros and a subnormal every 97 elements)
  noise       src/kernels/panels/panel_i16/tests.rs:8-12 (SplitMix-style)
  matrix      src/kernels/panels/panel.rs:236-240 (hash)
  normalized  src/kernels/attention/prefill64/test_data.rs:14-23 (norm-8 heads)
and the BASELINE synthetic data (seeded numpy PCG64: normals, uniforms).
"""
import numpy as np

M32 = 0xFFFFFFFF
M64 = 0xFFFFFFFFFFFFFFFF


def values(n, seed, scale=1.0):
    out = np.empty(n, dtype=np.float32)
    state = seed & M32
    for i in range(n):
        state = (state * 1664525 + 1013904223) & M32
        out[i] = np.float32(((state >> 8) / 16777216.0 * 2.0 - 1.0))
    if scale != 1.0:
        out *= np.float32(scale)
    return out


def att_values(n, seed, rng=1.0):
    out = np.empty(n, dtype=np.float32)
    state = seed & M32
    sub = np.array([3], dtype=np.uint32).view(np.float32)[0]
    for i in range(n):
        state = (state * 1664525 + 1013904223) & M32
        x = np.float32(np.float32((state >> 8) / 16777216.0 * 2.0 - 1.0) * np.float32(rng))
        m = i % 97
        out[i] = np.float32(-0.0) if m == 0 else (np.float32(0.0) if m == 1 else (sub if m == 2 else x))
    return out


def noise(i, seed):
    i = np.asarray(i, dtype=np.uint64)
    with np.errstate(over="ignore"):
        h = (i ^ np.uint64((seed << 40) & M64)) * np.uint64(0x9E3779B97F4A7C15)
        h = (h ^ (h >> np.uint64(29))) * np.uint64(0xBF58476D1CE4E5B9)
    return (h >> np.uint64(40)).astype(np.float32) / np.float32(1 << 24) - np.float32(0.5)


def matrix(length, seed):
    i = np.arange(length, dtype=np.int64)
    return (((i * 2654435761 + seed * 97) % 2003).astype(np.float32) - np.float32(1001.0)) / np.float32(977.0)


def normalized(n, seed):
    x = values(n, seed)
    heads = x.reshape(-1, 64)
    for h in heads:
        norm = np.float32(np.sqrt(np.float32(np.sum(h * h, dtype=np.float32))))
        h *= np.float32(8.0) / norm
    return x


def i16_activations(m, k):
    """panel_i16/tests.rs:16-29: a 700x outlier channel, zero first group in row 2."""
    idx = np.arange(m * k, dtype=np.uint64)
    v = noise(idx, 1) * np.float32(4.0)
    r, c = idx // k, idx % k
    v = np.where((r == 2) & (c < 64), np.float32(0.0), np.where(c == 37, v * np.float32(700.0), v))
    return v.astype(np.float32)


def i16_weights(n, k):
    """panel_i16/tests.rs:32-38: int8 codes in [-127,127], positive group scales."""
    codes = np.clip(np.round(noise(np.arange(n * k, dtype=np.uint64), 2) * np.float32(254.0)), -127, 127).astype(np.int8)
    scales = (np.float32(0.001) + np.abs(noise(np.arange(n * k // 64, dtype=np.uint64), 3)) * np.float32(0.01)).astype(np.float32)
    return codes.reshape(n, k), scales.reshape(n, k // 64)


# ---- BASELINE.json synthetic data (seeded) ---------------------------------
def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def normal(shape, std, seed):
    return (rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def codes_uniform(shape, lo, hi, dtype, seed):
    return rng(seed).integers(lo, hi + 1, size=shape, dtype=np.int64).astype(dtype)


def uniform(shape, lo, hi, seed):
    return rng(seed).uniform(lo, hi, size=shape).astype(np.float32)
