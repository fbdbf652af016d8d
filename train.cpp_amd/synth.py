"""Seeded synthetic inputs for the benchmark configurations (numpy, vectorised).

Random numbers come from splitmix64, the generator of the reference library
(src/core/trc_rng.cpp:38-68), with one independent stream per block (or per
element for dense F32 tensors): stream i starts at state `seed + i`. This makes
the data independent of how the work is split. The draws mirror the
reference's rng_uniform01 (top 24 bits), rng_uniform (lo + (hi-lo)*u) and
rng_normal (Box-Muller, u1 clamped to 1e-7) in float32 arithmetic.

Block contents follow the benchmark configurations:
  d  fp16(uniform[2e-4, 1e-3])             every format
  m  fp16(uniform[-0.05, 0])               Q4_1, Q5_1
  qh one 32-bit draw                       Q5_0, Q5_1
  qs 4 x 32-bit draws -> 16 nibble pairs   Q4_*, Q5_*
  qs 32 int8 in [-127, 127] by rejection   Q8_0 (top byte of a draw, 255 rejected)
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)

BLOCK_DTYPES = {
    2: np.dtype([("d", "<u2"), ("qs", "u1", 16)]),                               # Q4_0, 18 B
    3: np.dtype([("d", "<u2"), ("m", "<u2"), ("qs", "u1", 16)]),                 # Q4_1, 20 B
    6: np.dtype([("d", "<u2"), ("qh", "<u4"), ("qs", "u1", 16)]),                # Q5_0, 22 B
    7: np.dtype([("d", "<u2"), ("m", "<u2"), ("qh", "<u4"), ("qs", "u1", 16)]),  # Q5_1, 24 B
    8: np.dtype([("d", "<u2"), ("qs", "i1", 32)]),                               # Q8_0, 34 B
}
TYPE_NAMES = {2: "q4_0", 3: "q4_1", 6: "q5_0", 7: "q5_1", 8: "q8_0"}


def config_seed(cfg: int, tensor_id: int) -> int:
    return (0x7261696E ^ (cfg << 32) ^ tensor_id) & 0xFFFFFFFFFFFFFFFF


def next_u64(state: np.ndarray) -> np.ndarray:
    """Advances every stream in `state` (uint64 array, in place) by one draw."""
    with np.errstate(over="ignore"):
        state += GOLDEN
        z = state.copy()
        z ^= z >> np.uint64(30)
        z *= M1
        z ^= z >> np.uint64(27)
        z *= M2
        z ^= z >> np.uint64(31)
    return z


def next_u32(state: np.ndarray) -> np.ndarray:
    return (next_u64(state) >> np.uint64(32)).astype(np.uint32)


def uniform01(state: np.ndarray) -> np.ndarray:
    return (next_u64(state) >> np.uint64(40)).astype(np.float32) * np.float32(1.0 / 16777216.0)


def uniform(state: np.ndarray, lo: float, hi: float) -> np.ndarray:
    lo32, hi32 = np.float32(lo), np.float32(hi)
    return lo32 + (hi32 - lo32) * uniform01(state)


def streams(seed: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        return np.uint64(seed) + np.arange(n, dtype=np.uint64)


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """n float32 draws of N(mean, std), element i from stream seed + i."""
    st = streams(seed, n)
    u1 = np.maximum(uniform01(st), np.float32(1e-7))
    u2 = uniform01(st)
    r = np.sqrt(np.float32(-2.0) * np.log(u1))
    return (np.float32(mean) + np.float32(std) * r * np.cos(np.float32(6.28318530717958647692) * u2)).astype(np.float32)


def quant_blocks(type_: int, n_blocks: int, seed: int) -> np.ndarray:
    """n_blocks blocks of a legacy quant type as a structured array (raw bytes via .view(np.uint8))."""
    dt = BLOCK_DTYPES[type_]
    out = np.zeros(n_blocks, dtype=dt)
    st = streams(seed, n_blocks)
    out["d"] = uniform(st, 2e-4, 1e-3).astype(np.float16).view(np.uint16)
    if "m" in dt.names:
        out["m"] = uniform(st, -0.05, 0.0).astype(np.float16).view(np.uint16)
    if "qh" in dt.names:
        out["qh"] = next_u32(st)
    if type_ == 8:
        q = np.zeros((n_blocks, 32), dtype=np.int8)
        count = np.zeros(n_blocks, dtype=np.int64)
        idx = np.arange(n_blocks)
        while idx.size:
            sub = st[idx]
            v = (next_u32(sub) >> np.uint32(24)).astype(np.int16)
            st[idx] = sub
            ok = v < 255
            acc = idx[ok]
            q[acc, count[acc]] = (v[ok] - 127).astype(np.int8)
            count[acc] += 1
            idx = idx[count[idx] < 32]
        out["qs"] = q
    else:
        words = np.stack([next_u32(st) for _ in range(4)], axis=1)  # (n, 4) little-endian words
        out["qs"] = words.view(np.uint8).reshape(n_blocks, 16)
    return out


def block_bytes(blocks: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
