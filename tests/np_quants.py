"""Second, independent decoder for the formats the reference does not carry
(Q2_K, Q3_K, IQ2_XXS), written vectorised over whole blocks from the public
ggml layout. It shares no code or loop structure with the C oracle, so an
index, shift or sign mistake in either shows up as a mismatch. float32
numpy arithmetic rounds each product/difference separately (no FMA), the
same rounding the oracle and the GPU dequantizers use.
"""
import numpy as np


def _f16(raw, off):
    return raw[:, off:off + 2].copy().view(np.float16).astype(np.float32)  # (nb, 1)


def q2_k(raw):
    raw = raw.reshape(-1, 84)
    nb = raw.shape[0]
    sc = raw[:, :16]                                   # 16 groups of 16 weights
    qs = raw[:, 16:80].reshape(nb, 2, 1, 32)           # half, (shift), byte
    d, dmin = _f16(raw, 80), _f16(raw, 82)
    shifts = np.array([0, 2, 4, 6], dtype=np.uint8).reshape(1, 1, 4, 1)
    q = ((qs >> shifts) & 3).reshape(nb, 16, 16)        # group index = 8*half + 2*shift + byte//16
    dl = (d * (sc & 15).astype(np.float32)).reshape(nb, 16, 1)
    ml = (dmin * (sc >> 4).astype(np.float32)).reshape(nb, 16, 1)
    return (dl * q.astype(np.float32) - ml).reshape(-1)


def q3_k(raw):
    raw = raw.reshape(-1, 110)
    nb = raw.shape[0]
    hmask = raw[:, 0:32]
    qs = raw[:, 32:96].reshape(nb, 2, 1, 32)
    s12 = raw[:, 96:108]
    d = _f16(raw, 108)
    low = np.concatenate([s12[:, 0:8] & 15, s12[:, 0:8] >> 4], axis=1)           # (nb, 16)
    high = (s12[:, 8:12].reshape(nb, 1, 4) >> np.array([0, 2, 4, 6], dtype=np.uint8).reshape(1, 4, 1)) & 3
    scales = (low | (high.reshape(nb, 16) << 4)).astype(np.int32) - 32
    shifts = np.array([0, 2, 4, 6], dtype=np.uint8).reshape(1, 1, 4, 1)
    q2 = ((qs >> shifts) & 3).reshape(nb, 2, 4, 32).astype(np.int32)
    bits = (hmask.reshape(nb, 1, 1, 32) >> np.arange(8, dtype=np.uint8).reshape(1, 2, 4, 1)) & 1
    q = q2 - 4 * (1 - bits.astype(np.int32))
    dl = (d * scales.astype(np.float32)).reshape(nb, 16, 1)
    return (dl * q.reshape(nb, 16, 16).astype(np.float32)).reshape(-1)


def _sign_table():
    s = np.arange(128)
    par = np.array([bin(i).count("1") & 1 for i in range(128)])
    full = (s | (par << 7)).astype(np.uint8)
    return np.unpackbits(full.reshape(-1, 1), axis=1, bitorder="little")  # (128, 8)


def iq2_xxs(raw, grid):
    raw = raw.reshape(-1, 66)
    nb = raw.shape[0]
    d = _f16(raw, 0)
    q = raw[:, 2:66].reshape(nb, 8, 8)
    idx = q[:, :, 0:4]                                     # grid indices
    s = q[:, :, 4:8].copy().view("<u4").reshape(nb, 8)     # signs + scale
    db = (d * (0.5 + (s >> 28).astype(np.float32))) * np.float32(0.25)      # (nb, 8)
    g = np.asarray(grid, dtype="<u8")[idx].view(np.uint8).reshape(nb, 8, 4, 8).astype(np.float32)
    sidx = (s.reshape(nb, 8, 1) >> (7 * np.arange(4, dtype=np.uint32)).reshape(1, 1, 4)) & 127
    neg = _sign_table()[sidx]                              # (nb, 8, 4, 8)
    sign = np.where(neg == 1, np.float32(-1.0), np.float32(1.0))
    return ((db.reshape(nb, 8, 1, 1).astype(np.float32) * g) * sign).reshape(-1)
