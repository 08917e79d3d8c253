"""Seeded synthetic GGUF weights and activations (host side, numpy).

The byte recipe is shared with the device generator (csrc/kernels/synth.hip,
``hh_synth_weights_dev``); the GPU tests check that both produce identical bytes:

* stream byte j of seed s = byte (j % 8), little endian, of
  ``mix64(s + (j // 8 + 1) * 0x9E3779B97F4A7C15)`` (splitmix64 evaluated at a counter);
* every f16 scale field k of the format (Q4_K: d = field 2b, dmin = field 2b+1 of block b;
  Q4_0 / Q8_0 / IQ2_XXS / IQ3_XXS: d = field b at the block start; Q6_K: d = field b at
  byte 208) is then overwritten with
  ``f16_rne(f32(lo + (hi - lo) * u_k))``, ``u_k = (mix64 stream of s ^ SCALE_SALT at k) >> 11
  * 2**-53`` computed in double, lo/hi being f32 values.

Uniform bytes make every 4-bit code, 6-bit scale/min, grid index, sign pattern and IQ
scale nibble uniform, which is the input distribution BASELINE.json names.  Activations
are N(0, 1) by Box-Muller in double, rounded to f32.
"""
from __future__ import annotations

import numpy as np

GOLDEN = 0x9E3779B97F4A7C15
SCALE_SALT = 0xD1B54A32D192ED03
M64 = (1 << 64) - 1

# GGML type ids
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS = 0, 1, 2, 8, 12, 14, 16, 18
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), IQ2_XXS: (256, 66),
         IQ3_XXS: (256, 98), F32: (1, 4), F16: (1, 2)}
# Default U(lo, hi) ranges of the f16 scales per format (project choices).
SCALE_RANGE = {Q4_0: (0.001, 0.02), Q8_0: (0.001, 0.01), Q4_K: (2e-4, 2e-3), Q6_K: (5e-5, 5e-4),
               IQ2_XXS: (0.001, 0.01), IQ3_XXS: (0.001, 0.01)}


def _mix64(z: np.ndarray) -> np.ndarray:
    z = z.astype(np.uint64, copy=True)
    with np.errstate(over="ignore"):
        z ^= z >> np.uint64(30)
        z *= np.uint64(0xBF58476D1CE4E5B9)
        z ^= z >> np.uint64(27)
        z *= np.uint64(0x94D049BB133111EB)
        z ^= z >> np.uint64(31)
    return z


def synth_u64(seed: int, idx: np.ndarray) -> np.ndarray:
    idx = np.asarray(idx, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & M64) + (idx + np.uint64(1)) * np.uint64(GOLDEN)
    return _mix64(z)


def stream_bytes(seed: int, nbytes: int) -> np.ndarray:
    words = synth_u64(seed, np.arange((nbytes + 7) // 8, dtype=np.uint64))
    return words.astype("<u8").view(np.uint8)[:nbytes].copy()


def scale_values(seed: int, fields: np.ndarray, lo: float, hi: float) -> np.ndarray:
    """f16 bit patterns of the scale fields (see module docstring)."""
    u = (synth_u64(seed ^ SCALE_SALT, fields) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
    lo_d, hi_d = float(np.float32(lo)), float(np.float32(hi))
    v = (lo_d + (hi_d - lo_d) * u).astype(np.float32)
    return v.astype(np.float16).view(np.uint16)


def quant_weights(t: int, n_blocks: int, seed: int, lo: float | None = None, hi: float | None = None) -> np.ndarray:
    """n_blocks GGUF blocks of format t (bytes), exactly as hh_synth_weights_dev writes them."""
    block, bb = BLOCK[t]
    out = stream_bytes(seed, n_blocks * bb)
    if t in (F32, F16):
        return out
    if lo is None or hi is None:
        lo, hi = SCALE_RANGE[t]
    b = np.arange(n_blocks, dtype=np.uint64)
    view = out.reshape(n_blocks, bb)
    if t == Q4_K:
        d = scale_values(seed, 2 * b, lo, hi)
        dm = scale_values(seed, 2 * b + 1, lo, hi)
        view[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
        view[:, 2:4] = dm.view(np.uint8).reshape(-1, 2)
    elif t == Q6_K:
        d = scale_values(seed, b, lo, hi)
        view[:, 208:210] = d.view(np.uint8).reshape(-1, 2)
    else:
        d = scale_values(seed, b, lo, hi)
        view[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    return out


def matrix(t: int, rows: int, cols: int, seed: int, lo: float | None = None, hi: float | None = None) -> np.ndarray:
    block, bb = BLOCK[t]
    assert cols % block == 0
    return quant_weights(t, rows * cols // block, seed, lo, hi)


def normal(seed: int, n: int) -> np.ndarray:
    """n samples of N(0,1) as f32 (Box-Muller in double)."""
    i = np.arange(n, dtype=np.uint64)
    u1 = ((synth_u64(seed, 2 * i) >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)
    u2 = (synth_u64(seed, 2 * i + 1) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
    return (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)).astype(np.float32)


def seed_for(config: int, layer: int, matrix_id: int) -> int:
    """Seed = hash(config, layer, matrix) (splitmix64 finaliser of a packed key)."""
    key = np.uint64(((config & 0xFFFF) << 40) ^ ((layer & 0xFFFFFF) << 8) ^ (matrix_id & 0xFF) ^ 0x5EED0000000000)
    return int(_mix64(np.array([key], dtype=np.uint64))[0])


# matrix ids
GATE, UP, DOWN, ACT = 0, 1, 2, 3
