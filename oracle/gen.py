"""Portable seeded inputs for parity fixtures -- TEST INFRASTRUCTURE ONLY.

The golden fixtures in tests/golden/ record digests of quantizer outputs on
inputs drawn here, so the same bytes must come out on any x86 host and any
numpy version.  Only integer arithmetic, IEEE add/multiply/divide and sqrt
are used (all correctly rounded, hence identical everywhere); no log/cos.

  uniform : splitmix64(seed, counter) -> 24-bit uniform in [0, 1)
  normal  : Irwin-Hall, sum of 12 uniforms - 6  (mean 0, variance 1, |z| < 6)
  student : Z / sqrt(chi2_3 / 3), chi2_3 = sum of three squared normals
"""

import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix64(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int, stream: int = 0) -> np.ndarray:
    """n float64 values k * 2^-24, k uniform in [0, 2^24)."""
    base = (np.uint64(seed) << np.uint64(40)) ^ (np.uint64(stream) << np.uint64(36))
    ctr = np.arange(n, dtype=np.uint64) + base
    bits = _splitmix64(ctr) >> np.uint64(40)
    return bits.astype(np.float64) * (2.0 ** -24)


def normal(seed: int, shape, std: float = 1.0, stream: int = 0) -> np.ndarray:
    """float32 array of approximately N(0, std^2) values (Irwin-Hall 12)."""
    n = int(np.prod(shape))
    acc = np.zeros(n, dtype=np.float64)
    for j in range(12):
        acc += uniform(seed, n, stream * 16 + j)
    acc -= 6.0
    return (acc * std).astype(np.float32).reshape(shape)


def student_t3(seed: int, shape, scale: float = 1.0) -> np.ndarray:
    """float32 Student-t (df=3) values times `scale`: heavy tails that stress
    the E8M0 scale range."""
    z = normal(seed, shape, stream=0).astype(np.float64)
    chi = np.zeros(z.shape, dtype=np.float64)
    for j in range(3):
        g = normal(seed, shape, stream=1 + j).astype(np.float64)
        chi += g * g
    t = z / np.sqrt(chi / 3.0)
    return (t * scale).astype(np.float32)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even (NaN kept)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u >> 16) & 1) + np.uint32(0x7FFF)
    out = ((u + r) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)
