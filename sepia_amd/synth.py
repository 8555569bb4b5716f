"""Seeded synthetic inputs for the benchmark configurations (host side, numpy).

Quantized blocks are uniform random bytes (so every packed field -- 6-bit
sub-scales, quants, grid indices, sign bits -- is uniform over its range),
with each block's f16 scale fields replaced by values drawn uniformly from
[lo, hi] and rounded to f16, as the benchmark configurations specify
(2^-10 .. 2^-6). Activations are N(0, 1) float32; the router is N(0, 0.02).
Large weight sets are generated on the GPU instead (sepia_hip_synth_blocks).
"""
import numpy as np

# (elements per block, bytes per block) and the byte offsets of each block's
# f16 scale fields, per GGUF type id.
GEOM = {0: (1, 4), 1: (1, 2), 8: (32, 34), 10: (256, 84), 11: (256, 110), 12: (256, 144),
        13: (256, 176), 14: (256, 210), 16: (256, 66), 17: (256, 74), 18: (256, 98), 23: (256, 136)}
F16_FIELDS = {8: (0,), 10: (80, 82), 11: (108,), 12: (0, 2), 13: (0, 2), 14: (208,),
              16: (0,), 17: (0,), 18: (0,), 23: (0,)}

SCALE_LO = 2.0 ** -10
SCALE_HI = 2.0 ** -6


def row_bytes(t, n):
    be, bb = GEOM[t]
    if n % be:
        raise ValueError("row length %d is not a multiple of the block size %d" % (n, be))
    return n // be * bb


def f16_bits_uniform(rng, n, lo=SCALE_LO, hi=SCALE_HI):
    v = rng.uniform(lo, hi, size=n).astype(np.float16)
    return v.view(np.uint16)


def random_blocks(t, n_blocks, rng, lo=SCALE_LO, hi=SCALE_HI):
    """n_blocks random blocks of type t as a flat uint8 array."""
    be, bb = GEOM[t]
    raw = rng.integers(0, 256, size=(n_blocks, bb), dtype=np.uint8)
    for off in F16_FIELDS.get(t, ()):
        raw[:, off:off + 2] = f16_bits_uniform(rng, n_blocks, lo, hi).view(np.uint8).reshape(n_blocks, 2)
    return raw.reshape(-1)


def random_matrix(t, out_dim, in_dim, rng, lo=SCALE_LO, hi=SCALE_HI):
    be, _ = GEOM[t]
    return random_blocks(t, out_dim * (in_dim // be), rng, lo, hi)


def normal_vector(rng, n, scale=1.0):
    return (rng.standard_normal(n) * scale).astype(np.float32)
