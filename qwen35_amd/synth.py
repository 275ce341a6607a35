"""Seeded synthetic weights and activations for the benchmark configurations.

Every byte comes from a counter-based SplitMix64 stream (seed 0 by default,
one sub-stream per tensor), so the host-side checker and the GPU read the same
inputs.  Block contents follow the generation rules of each configuration:

* Q8_0    32 int8 uniform in [-127, 127], f16 d = f16(|N(0,1)| * 2e-4)
* Q4_K    random nibbles and packed 6-bit scales/mins, f16 d and dmin = |N(0,1)| * 1e-3
* Q6_K    random ql/qh bits, int8 sub-scales uniform in [-64, 63], f16 d = |N(0,1)| * 1e-3
* IQ4_NL  random 4-bit codebook indices, f16 d = |N(0,1)| * 1e-3
* Q5_K    as Q4_K plus random high bits; Q3_K random 2-bit values, high-bit
          mask and packed 6-bit scales; Q2_K random 2-bit values and 4-bit
          scale/min bytes; IQ4_XS random indices and 6-bit scales; f16 d (and
          dmin) = |N(0,1)| * 1e-3 (formats beyond the benchmark configurations,
          same generation style)
* Q4_0    random nibbles, f16 d = |N(0,1)| * 1e-3; Q4_1 the same plus an f16
          min m = N(0,1) * 8e-3
* IQ3_XXS, IQ3_S  random grid indices, sign words and scale nibbles, f16 d =
          |N(0,1)| * 1e-3
* activations f32 ~ N(0,1) (Box-Muller)
"""
from __future__ import annotations

import hashlib

import numpy as np

TT_Q8_0, TT_Q4_K, TT_Q6_K, TT_IQ4_NL = 8, 12, 14, 20
TT_Q2_K, TT_Q3_K, TT_Q5_K, TT_IQ4_XS = 10, 11, 13, 23
TT_Q4_0, TT_Q4_1 = 2, 3
TT_IQ3_XXS, TT_IQ3_S = 18, 21
GEOM = {TT_Q8_0: (32, 34), TT_IQ4_NL: (32, 18), TT_Q4_K: (256, 144), TT_Q6_K: (256, 210),
        TT_Q2_K: (256, 84), TT_Q3_K: (256, 110), TT_Q5_K: (256, 176), TT_IQ4_XS: (256, 136),
        TT_Q4_0: (32, 18), TT_Q4_1: (32, 20), TT_IQ3_XXS: (256, 98), TT_IQ3_S: (256, 110)}
D_SCALE = {TT_Q8_0: 2e-4, TT_IQ4_NL: 1e-3, TT_Q4_K: 1e-3, TT_Q6_K: 1e-3, TT_Q2_K: 1e-3, TT_Q3_K: 1e-3,
           TT_Q5_K: 1e-3, TT_IQ4_XS: 1e-3, TT_Q4_0: 1e-3, TT_Q4_1: 1e-3, TT_IQ3_XXS: 1e-3, TT_IQ3_S: 1e-3}

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def substream(seed: int, tag: int) -> int:
    """Seed of the independent stream `tag` derived from `seed`."""
    with np.errstate(over="ignore"):
        z = np.array([(seed * 0x9E3779B97F4A7C15 + tag * 0xD1B54A32D192ED03 + 1) % (1 << 64)],
                     np.uint64)
        return int(_mix(z)[0])


def splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Outputs start..start+n-1 of SplitMix64 seeded with `seed`."""
    with np.errstate(over="ignore"):
        i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        return _mix(np.uint64(seed % (1 << 64)) + i * _GAMMA)


def rand_bytes(seed: int, n: int) -> np.ndarray:
    words = splitmix64(seed, (n + 7) // 8)
    return words.view(np.uint8)[:n].copy()


def rand_uniform_int(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """n integers uniform on [lo, hi] (multiply-shift range reduction)."""
    z = splitmix64(seed, n) >> np.uint64(32)
    span = np.uint64(hi - lo + 1)
    return ((z * span) >> np.uint64(32)).astype(np.int64) + lo


def rand_normal(seed: int, n: int) -> np.ndarray:
    """n standard normals (float64) by Box-Muller on pairs of 53-bit uniforms."""
    m = (n + 1) // 2
    z = splitmix64(seed, 2 * m)
    u = ((z >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * m)
    out[0::2] = r * np.cos(2 * np.pi * u2)
    out[1::2] = r * np.sin(2 * np.pi * u2)
    return out[:n]


def f16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float64).astype(np.float16).view(np.uint16)


def make_weight(ttype: int, rows: int, cols: int, seed: int = 0, tag: int = 1) -> np.ndarray:
    """Packed weight [rows, row_bytes] (uint8) in GGUF block layout."""
    be, bb = GEOM[ttype]
    assert cols % be == 0
    nb = rows * (cols // be)
    s = substream(seed, tag)
    blocks = np.empty((nb, bb), np.uint8)
    d = f16_bits(np.abs(rand_normal(substream(s, 1), nb)) * D_SCALE[ttype])
    if ttype == TT_Q8_0:
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        q = rand_uniform_int(substream(s, 2), nb * 32, -127, 127).astype(np.int8)
        blocks[:, 2:] = q.view(np.uint8).reshape(nb, 32)
    elif ttype == TT_IQ4_NL:
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blocks[:, 2:] = rand_bytes(substream(s, 2), nb * 16).reshape(nb, 16)
    elif ttype == TT_Q4_K:
        dmin = f16_bits(np.abs(rand_normal(substream(s, 3), nb)) * D_SCALE[ttype])
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blocks[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
        blocks[:, 4:16] = rand_bytes(substream(s, 4), nb * 12).reshape(nb, 12)
        blocks[:, 16:] = rand_bytes(substream(s, 2), nb * 128).reshape(nb, 128)
    elif ttype == TT_Q6_K:
        blocks[:, 0:192] = rand_bytes(substream(s, 2), nb * 192).reshape(nb, 192)
        sc = rand_uniform_int(substream(s, 4), nb * 16, -64, 63).astype(np.int8)
        blocks[:, 192:208] = sc.view(np.uint8).reshape(nb, 16)
        blocks[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    elif ttype == TT_Q5_K:
        dmin = f16_bits(np.abs(rand_normal(substream(s, 3), nb)) * D_SCALE[ttype])
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blocks[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
        blocks[:, 4:16] = rand_bytes(substream(s, 4), nb * 12).reshape(nb, 12)
        blocks[:, 16:] = rand_bytes(substream(s, 2), nb * 160).reshape(nb, 160)
    elif ttype == TT_Q3_K:
        blocks[:, 0:108] = rand_bytes(substream(s, 2), nb * 108).reshape(nb, 108)
        blocks[:, 108:110] = d.view(np.uint8).reshape(nb, 2)
    elif ttype == TT_Q2_K:
        dmin = f16_bits(np.abs(rand_normal(substream(s, 3), nb)) * D_SCALE[ttype])
        blocks[:, 0:80] = rand_bytes(substream(s, 2), nb * 80).reshape(nb, 80)
        blocks[:, 80:82] = d.view(np.uint8).reshape(nb, 2)
        blocks[:, 82:84] = dmin.view(np.uint8).reshape(nb, 2)
    elif ttype == TT_IQ4_XS:
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blocks[:, 2:] = rand_bytes(substream(s, 2), nb * 134).reshape(nb, 134)
    elif ttype in (TT_IQ3_XXS, TT_IQ3_S):
        # every byte after d is free: grid indices, sign indices / masks, scales
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blocks[:, 2:] = rand_bytes(substream(s, 2), nb * (bb - 2)).reshape(nb, bb - 2)
    elif ttype == TT_Q4_0:
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blocks[:, 2:] = rand_bytes(substream(s, 2), nb * 16).reshape(nb, 16)
    elif ttype == TT_Q4_1:
        # m: the block minimum, signed, of the magnitude of 8 * d
        m = f16_bits(rand_normal(substream(s, 3), nb) * (8 * D_SCALE[ttype]))
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blocks[:, 2:4] = m.view(np.uint8).reshape(nb, 2)
        blocks[:, 4:] = rand_bytes(substream(s, 2), nb * 16).reshape(nb, 16)
    else:
        raise ValueError(f"unsupported ttype {ttype}")
    return blocks.reshape(rows, cols // be * bb)


def make_act(cols: int, k: int = 1, seed: int = 0, tag: int = 100) -> np.ndarray:
    """Activations [k, cols] f32 ~ N(0,1)."""
    return rand_normal(substream(seed, tag), k * cols).astype(np.float32).reshape(k, cols)


def ragged_lengths(nseq: int = 8, lo: int = 16, hi: int = 256, seed: int = 0,
                   tag: int = 200) -> np.ndarray:
    """Sequence lengths uniform on [lo, hi] (config 4's ragged prefill batch)."""
    return rand_uniform_int(substream(seed, tag), nseq, lo, hi).astype(np.int32)


def offsets_from_lengths(lengths: np.ndarray) -> np.ndarray:
    """Prefix-sum offset table: offsets[i] = first packed token of sequence i, offsets[n] = total."""
    off = np.zeros(len(lengths) + 1, np.int32)
    np.cumsum(lengths, out=off[1:])
    return off


def sha256(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()
