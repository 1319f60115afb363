"""Seeded synthetic inputs: bf16 tensors ~ N(0, 1) and U(lo, hi).

The benchmark configurations ask for "bf16 ~ N(0,1) from a fixed seed".  The
generator here is counter based and built only from IEEE-754 operations that
are exactly rounded everywhere (integer ops, +, -, *, /, sqrt, frexp), so the
same seed gives the same bits on every CPU, whatever SIMD paths numpy picks
for its transcendental functions:

* SplitMix64: word i of stream ``s`` is ``mix64(s + (i + 1) * 0x9E3779B97F4A7C15)``.
* Box-Muller on word pairs (2j, 2j+1): u1 = ((w >> 11) + 1) * 2**-53 in (0, 1],
  u2 = (w >> 11) * 2**-53 in [0, 1); z0 = r cos(2 pi u2), z1 = r sin(2 pi u2),
  r = sqrt(-2 ln u1).  ln and sin/cos are evaluated with fixed polynomials
  (atanh series for ln on [sqrt(1/2), sqrt(2)); Taylor series on [0, pi/4]
  after an exact octant reduction of u2), accurate to a few ulp of float64.
* float64 -> float32 (RNE) -> bf16 (RNE).

Streams: tensor ``name`` of a workload uses stream ``mix64(seed ^ fnv1a(name))``.

The numpy code below is the specification.  ``csrc/synth.c`` runs the same
operation sequence in C with OpenMP (``lib/libtoyinfer_synth.so``) and is
used when built; tests check both produce identical bits.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib",
                         "libtoyinfer_synth.so")
_clib = None


def _c():
    global _clib
    if _clib is None and os.path.exists(_LIB_PATH):
        lib = ctypes.CDLL(_LIB_PATH)
        lib.ti_synth_normal_bf16.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_void_p]
        lib.ti_synth_normal_bf16.restype = None
        lib.ti_synth_uniform_bf16.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_double,
                                              ctypes.c_double, ctypes.c_void_p]
        lib.ti_synth_uniform_bf16.restype = None
        lib.ti_synth_scale_bf16.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_float,
                                            ctypes.c_void_p]
        lib.ti_synth_scale_bf16.restype = None
        _clib = lib
    return _clib

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_LN2 = 0.6931471805599453
_HALF_PI = 1.5707963267948966
_TWO53 = 2.0 ** -53
_CHUNK = 1 << 20


def _mix64(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def fnv1a64(text: str) -> int:
    h = 0xCBF29CE484222325
    for b in text.encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def stream_key(seed: int, name: str) -> int:
    with np.errstate(over="ignore"):
        return int(_mix64(np.array([(seed ^ fnv1a64(name)) & 0xFFFFFFFFFFFFFFFF],
                                   dtype=np.uint64))[0])


def _words(key: int, start: int, count: int) -> np.ndarray:
    idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix64(np.uint64(key) + idx * _GAMMA)


def _ln(u: np.ndarray) -> np.ndarray:
    """ln(u) for u in (0, 1] from frexp and an atanh series (exact ops only)."""
    m, e = np.frexp(u)                      # u = m * 2**e, m in [0.5, 1)
    small = m < 0.7071067811865476
    m = np.where(small, m * 2.0, m)
    e = np.where(small, e - 1, e).astype(np.float64)
    z = (m - 1.0) / (m + 1.0)               # |z| <= 0.1716
    z2 = z * z
    acc = np.full_like(z, 1.0 / 25.0)
    for k in range(11, -1, -1):             # sum_{k=0..12} z^(2k+1)/(2k+1)
        acc = acc * z2 + 1.0 / (2 * k + 1)
    return e * _LN2 + 2.0 * z * acc


def _sincos_2pi(u: np.ndarray):
    """(sin, cos)(2*pi*u) for u in [0, 1) with an exact quadrant reduction."""
    t = u * 4.0                              # exact (power of two)
    quad = np.floor(t)
    f = t - quad                             # exact, in [0, 1)
    flip = f > 0.5
    y = np.where(flip, 1.0 - f, f)           # exact, in [0, 0.5]
    x = y * _HALF_PI                         # in [0, pi/4]
    x2 = x * x
    s = np.full_like(x, 1.0 / _fact(17))
    for k in (15, 13, 11, 9, 7, 5, 3, 1):
        s = s * (-x2) + 1.0 / _fact(k)
    s = s * x
    c = np.full_like(x, 1.0 / _fact(16))
    for k in (14, 12, 10, 8, 6, 4, 2, 0):
        c = c * (-x2) + 1.0 / _fact(k)
    s, c = np.where(flip, c, s), np.where(flip, s, c)
    q = quad.astype(np.int64) & 3
    sin = np.select([q == 0, q == 1, q == 2], [s, c, -s], -c)
    cos = np.select([q == 0, q == 1, q == 2], [c, -s, -c], s)
    return sin, cos


def _fact(k: int) -> float:
    out = 1.0
    for i in range(2, k + 1):
        out *= i
    return out


def normal_f64(key: int, n: int) -> np.ndarray:
    """n standard normals (float64) of stream ``key``."""
    out = np.empty(n, np.float64)
    npairs = (n + 1) // 2
    for p0 in range(0, npairs, _CHUNK):
        pc = min(_CHUNK, npairs - p0)
        w = _words(key, 2 * p0, 2 * pc)
        u1 = ((w[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * _TWO53
        u2 = (w[1::2] >> np.uint64(11)).astype(np.float64) * _TWO53
        r = np.sqrt(-2.0 * _ln(u1))
        sn, cs = _sincos_2pi(u2)
        z = np.empty(2 * pc, np.float64)
        z[0::2] = r * cs
        z[1::2] = r * sn
        lo = 2 * p0
        hi = min(n, lo + 2 * pc)
        out[lo:hi] = z[: hi - lo]
    return out


def uniform_f64(key: int, n: int, lo: float, hi: float) -> np.ndarray:
    w = _words(key, 0, n)
    u = (w >> np.uint64(11)).astype(np.float64) * _TWO53
    return lo + (hi - lo) * u


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even, NaN kept quiet."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    r = np.where(nan, (u >> np.uint32(16)) | np.uint32(0x40), r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(
        np.float32)


def normal_bf16(seed: int, name: str, shape, use_c: bool = True) -> np.ndarray:
    """bf16 bit patterns ~ N(0, 1), shape ``shape``, stream (seed, name)."""
    n = int(np.prod(shape))
    key = stream_key(seed, name)
    lib = _c() if use_c else None
    if lib is not None:
        out = np.empty(n, np.uint16)
        lib.ti_synth_normal_bf16(key, n, out.ctypes.data)
        return out.reshape(shape)
    z = normal_f64(key, n).astype(np.float32)
    return f32_to_bf16_bits(z).reshape(shape)


def scale_bf16(bits: np.ndarray, scale: float, use_c: bool = True) -> np.ndarray:
    """bf16 bits of float32(bits) * float32(scale), rounded to nearest even."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    lib = _c() if use_c else None
    if lib is not None:
        out = np.empty_like(b)
        lib.ti_synth_scale_bf16(b.ctypes.data, b.size, float(np.float32(scale)), out.ctypes.data)
        return out
    return f32_to_bf16_bits(bf16_bits_to_f32(b) * np.float32(scale))


def uniform_bf16(seed: int, name: str, shape, lo: float, hi: float,
                 use_c: bool = True) -> np.ndarray:
    n = int(np.prod(shape))
    key = stream_key(seed, name)
    lib = _c() if use_c else None
    if lib is not None:
        out = np.empty(n, np.uint16)
        lib.ti_synth_uniform_bf16(key, n, float(lo), float(hi), out.ctypes.data)
        return out.reshape(shape)
    z = uniform_f64(key, n, lo, hi).astype(np.float32)
    return f32_to_bf16_bits(z).reshape(shape)
