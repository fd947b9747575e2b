"""Independent numpy restatement of the GGUF block layouts used on this path.

Written from the ggml block descriptions (block_q8_0, block_q4_K, block_q3_K and
dequantize_row_*), separately from the C oracle, so that two implementations
must agree. Also builds blocks from explicit field values (known-answer blocks).
"""
import numpy as np


def f16_to_f32(h):
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


# ---------------------------------------------------------------- Q8_0
def q8_0_fields(raw, rows, n):
    b = np.asarray(raw, np.uint8).reshape(rows, n // 32, 34)
    d = b[:, :, 0:2].copy().view(np.uint16)[:, :, 0]
    q = b[:, :, 2:].view(np.int8)
    return d, q


def q8_0_dequant(raw, rows, n):
    d, q = q8_0_fields(raw, rows, n)
    return (f16_to_f32(d)[:, :, None] * q.astype(np.float32)).reshape(rows, n)


def q8_0_pack(d_f16_bits, q):
    rows, nb = d_f16_bits.shape
    out = np.zeros((rows, nb, 34), np.uint8)
    out[:, :, 0:2] = np.asarray(d_f16_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:] = np.asarray(q, np.int8).reshape(rows, nb, 32).view(np.uint8)
    return out.reshape(-1)


# ---------------------------------------------------------------- Q4_K
def q4_k_pack(d, dmin, sc, mn, q):
    """One superblock: d/dmin fp16 bit patterns, sc/mn 8 ints 0..63, q 256 ints 0..15."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([d], np.uint16).view(np.uint8)
    blk[2:4] = np.array([dmin], np.uint16).view(np.uint8)
    s = np.zeros(12, np.int64)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    blk[4:16] = s.astype(np.uint8)
    q = np.asarray(q, np.int64).reshape(4, 2, 32)  # [pair j][nibble h][l]
    blk[16:] = (q[:, 0, :] | (q[:, 1, :] << 4)).reshape(-1).astype(np.uint8)
    return blk


def q4_k_unpack(blk):
    blk = np.asarray(blk, np.uint8)
    d = int(blk[0:2].view(np.uint16)[0])
    dmin = int(blk[2:4].view(np.uint16)[0])
    s = blk[4:16].astype(np.int64)
    sc, mn = np.zeros(8, np.int64), np.zeros(8, np.int64)
    for j in range(8):
        if j < 4:
            sc[j], mn[j] = s[j] & 63, s[j + 4] & 63
        else:
            sc[j] = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4)
            mn[j] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
    qs = blk[16:].astype(np.int64).reshape(4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=1).reshape(256)
    return d, dmin, sc, mn, q


def q4_k_dequant(raw, rows, n):
    raw = np.asarray(raw, np.uint8).reshape(rows, n // 256, 144)
    out = np.zeros((rows, n), np.float32)
    for r in range(rows):
        for s in range(n // 256):
            d, dmin, sc, mn, q = q4_k_unpack(raw[r, s])
            df, mf = f16_to_f32(d), f16_to_f32(dmin)
            for a in range(8):
                d1 = np.float32(df * np.float32(sc[a]))
                m1 = np.float32(mf * np.float32(mn[a]))
                vals = np.float32(d1 * q[a * 32:(a + 1) * 32].astype(np.float32)) - m1
                out[r, s * 256 + a * 32:s * 256 + (a + 1) * 32] = vals
    return out


# ---------------------------------------------------------------- Q3_K
def q3_k_pack(q3, scales, d):
    """One superblock: q3 256 ints 0..7 (value = q3 - 4), scales 16 ints 0..63, d fp16 bits."""
    blk = np.zeros(110, np.uint8)
    hm, qs = np.zeros(32, np.int64), np.zeros(64, np.int64)
    for i in range(256):
        v = int(q3[i])
        n, j, h, l = i // 128, (i // 32) % 4, (i // 16) % 2, i % 16
        qs[32 * n + 16 * h + l] |= (v & 3) << (2 * j)
        if v & 4:
            hm[16 * h + l] |= 1 << (4 * n + j)
    sc = np.zeros(12, np.int64)
    for k in range(16):
        if k < 8:
            sc[k] |= scales[k] & 15
        else:
            sc[k - 8] |= (scales[k] & 15) << 4
        sc[8 + k % 4] |= ((scales[k] >> 4) & 3) << (2 * (k // 4))
    blk[0:32] = hm.astype(np.uint8)
    blk[32:96] = qs.astype(np.uint8)
    blk[96:108] = sc.astype(np.uint8)
    blk[108:110] = np.array([d], np.uint16).view(np.uint8)
    return blk


def q3_k_unpack(blk):
    """Returns (q3 values -4..3 as ints, 16 scales 0..63, d bits) via the kmask form."""
    blk = np.asarray(blk, np.uint8)
    aux = blk[96:108].copy().view(np.uint32).astype(np.uint64)
    k1, k2 = 0x03030303, 0x0F0F0F0F
    tmp = int(aux[2])
    a0, a1 = int(aux[0]), int(aux[1])
    w = [(a0 & k2) | (((tmp >> 0) & k1) << 4), (a1 & k2) | (((tmp >> 2) & k1) << 4),
         ((a0 >> 4) & k2) | (((tmp >> 4) & k1) << 4), ((a1 >> 4) & k2) | (((tmp >> 6) & k1) << 4)]
    scales = np.array(w, np.uint32).view(np.uint8).astype(np.int64)
    hm, qs = blk[0:32].astype(np.int64), blk[32:96].astype(np.int64)
    vals = np.zeros(256, np.int64)
    i = 0
    m = 1
    for n in range(2):
        shift = 0
        for j in range(4):
            for h in range(2):
                for l in range(16):
                    low = (qs[32 * n + 16 * h + l] >> shift) & 3
                    vals[i] = low - (0 if hm[16 * h + l] & m else 4)
                    i += 1
            shift += 2
            m <<= 1
    d = int(blk[108:110].view(np.uint16)[0])
    return vals, scales, d


def q3_k_dequant(raw, rows, n):
    raw = np.asarray(raw, np.uint8).reshape(rows, n // 256, 110)
    out = np.zeros((rows, n), np.float32)
    for r in range(rows):
        for s in range(n // 256):
            vals, scales, d = q3_k_unpack(raw[r, s])
            df = f16_to_f32(d)
            for k in range(16):
                dl = np.float32(df * np.float32(scales[k] - 32))
                out[r, s * 256 + 16 * k:s * 256 + 16 * (k + 1)] = dl * vals[16 * k:16 * (k + 1)].astype(np.float32)
    return out
