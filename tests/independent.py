"""Second restatements of the block formats, written from other texts than the oracle's, to pin it.

* Q2_0, Q3_K, IQ4_NL, IQ4_XS, IQ3_S: the affine form of strata_mlx/gguf.py:182-276 (`to_affine`), which reads the
  blocks as bit strings and words (little-endian bit order over the qh and sign bytes, 32-bit scale words with
  masks for Q3_K) where strata_mlx/blocks.py:57-194 (the oracle's text) indexes bytes.
* IQ3_XXS, IQ2_S, IQ2_XS, IQ2_XXS, IQ1_M, Q6_K: ggml's published scalar dequantizers (ggml-quants
  `dequantize_row_*`, as gguf-py 0.19.0 ports them), loops over sub-blocks with their own indexing.

Pure Python per block: slow, for a few blocks only. Returns float64 weights (exact).
"""

import struct

import numpy as np

KV = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]


def f16(bs: bytes) -> float:
    return float(np.frombuffer(bs, dtype="<f2")[0])


def bits_le(bs: bytes):
    """The bits of a byte string, least significant of the first byte first."""
    return [(byte >> i) & 1 for byte in bs for i in range(8)]


def q2_0(b: bytes, t):
    d = f16(b[0:2])
    return [d * (((b[2 + i // 4] >> (2 * (i % 4))) & 3) - 1) for i in range(64)]


def iq4_nl(b: bytes, t):
    d = f16(b[0:2])
    nib = [q & 15 for q in b[2:18]] + [q >> 4 for q in b[2:18]]
    return [d * KV[c] for c in nib]


def iq4_xs(b: bytes, t):
    d = f16(b[0:2])
    high = struct.unpack("<H", b[2:4])[0]
    out = []
    for ib in range(8):
        low = (b[4 + ib // 2] >> (4 * (ib % 2))) & 15
        ls = low | (((high >> (2 * ib)) & 3) << 4)
        run = b[8 + 16 * ib: 24 + 16 * ib]
        nib = [q & 15 for q in run] + [q >> 4 for q in run]
        out += [d * (ls - 32) * KV[c] for c in nib]
    return out


def q3_k(b: bytes, t):
    hmask, qs = b[0:32], b[32:96]
    d = f16(b[108:110])
    a0, a1, tmp = struct.unpack("<III", b[96:108])
    k1, k2 = 0x03030303, 0x0F0F0F0F
    words = [(a0 & k2) | ((tmp & k1) << 4), (a1 & k2) | (((tmp >> 2) & k1) << 4),
             ((a0 >> 4) & k2) | (((tmp >> 4) & k1) << 4), ((a1 >> 4) & k2) | (((tmp >> 6) & k1) << 4)]
    sub = [((w >> (8 * i)) & 0xFF) - 32 for w in words for i in range(4)]
    out = []
    for i in range(256):
        r, pos = i // 32, i % 32
        half, j = r // 4, r % 4
        two = (qs[32 * half + pos] >> (2 * j)) & 3
        value = two - (0 if (hmask[pos] >> r) & 1 else 4)
        out.append(d * sub[i // 16] * value)
    return out


def iq3_s(b: bytes, t):
    grid = t["iq3s_grid"].reshape(512, 4)
    d = f16(b[0:2])
    hbits = bits_le(b[66:74])
    negative = bits_le(b[74:106])
    nib = [v for s in b[106:110] for v in (s & 15, s >> 4)]
    out = []
    for i in range(256):
        entry = i // 4
        index = b[2 + entry] | (hbits[entry] << 8)
        value = int(grid[index][i % 4]) * (-1 if negative[i] else 1)
        out.append(d * (1 + 2 * nib[i // 32]) * value)
    return out


def iq3_xxs(b: bytes, t):  # ggml dequantize_row_iq3_xxs
    grid = t["iq3xxs_grid"].reshape(256, 4)
    ksigns = t["ksigns"]
    d = f16(b[0:2])
    qs, sas = b[2:66], b[66:98]
    y = []
    for ib32 in range(8):
        aux32 = struct.unpack("<I", sas[4 * ib32: 4 * ib32 + 4])[0]
        db = d * (0.5 + (aux32 >> 28)) * 0.5
        q3 = qs[8 * ib32: 8 * ib32 + 8]
        for l in range(4):
            signs = int(ksigns[(aux32 >> (7 * l)) & 127])
            g1, g2 = grid[q3[2 * l]], grid[q3[2 * l + 1]]
            y += [db * int(g1[j]) * (-1 if signs & (1 << j) else 1) for j in range(4)]
            y += [db * int(g2[j]) * (-1 if signs & (1 << (j + 4)) else 1) for j in range(4)]
    return y


def iq2_s(b: bytes, t):  # ggml dequantize_row_iq2_s
    grid = t["iq2s_grid"].reshape(1024, 8)
    d = f16(b[0:2])
    qs, signs, qh, scales = b[2:34], b[34:66], b[66:74], b[74:82]
    y = []
    for ib32 in range(8):
        db = [d * (0.5 + (scales[ib32] & 15)) * 0.25, d * (0.5 + (scales[ib32] >> 4)) * 0.25]
        for l in range(4):
            dl = db[l // 2]
            g = grid[qs[4 * ib32 + l] | ((qh[ib32] << (8 - 2 * l)) & 0x300)]
            s = signs[4 * ib32 + l]
            y += [dl * int(g[j]) * (-1 if s & (1 << j) else 1) for j in range(8)]
    return y


def iq2_xs(b: bytes, t):  # ggml dequantize_row_iq2_xs
    grid = t["iq2xs_grid"].reshape(512, 8)
    ksigns = t["ksigns"]
    d = f16(b[0:2])
    qs = struct.unpack("<32H", b[2:66])
    scales = b[66:74]
    y = []
    for ib32 in range(8):
        db = [d * (0.5 + (scales[ib32] & 15)) * 0.25, d * (0.5 + (scales[ib32] >> 4)) * 0.25]
        for l in range(4):
            q = qs[4 * ib32 + l]
            g = grid[q & 511]
            s = int(ksigns[q >> 9])
            y += [db[l // 2] * int(g[j]) * (-1 if s & (1 << j) else 1) for j in range(8)]
    return y


def iq2_xxs(b: bytes, t):  # ggml dequantize_row_iq2_xxs
    grid = t["iq2xxs_grid"].reshape(256, 8)
    ksigns = t["ksigns"]
    d = f16(b[0:2])
    y = []
    for ib32 in range(8):
        part = b[2 + 8 * ib32: 10 + 8 * ib32]
        aux8 = part[0:4]
        aux32 = struct.unpack("<I", part[4:8])[0]
        db = d * (0.5 + (aux32 >> 28)) * 0.25
        for l in range(4):
            g = grid[aux8[l]]
            s = int(ksigns[(aux32 >> (7 * l)) & 127])
            y += [db * int(g[j]) * (-1 if s & (1 << j) else 1) for j in range(8)]
    return y


def iq1_m(b: bytes, t):  # ggml dequantize_row_iq1_m (grid values -1, 0, 1; the table holds them + 1)
    grid = t["iq1_grid"].reshape(2048, 8).astype(np.int64) - 1
    qs, qh = b[0:32], b[32:48]
    sc = struct.unpack("<4H", b[48:56])
    u = (sc[0] >> 12) | ((sc[1] >> 8) & 0x00F0) | ((sc[2] >> 4) & 0x0F00) | (sc[3] & 0xF000)
    d = float(np.array([u], dtype="<u2").view("<f2")[0])
    y = []
    for ib in range(8):
        dl1 = d * (2 * ((sc[ib // 2] >> (6 * (ib % 2) + 0)) & 7) + 1)
        dl2 = d * (2 * ((sc[ib // 2] >> (6 * (ib % 2) + 3)) & 7) + 1)
        q, h = qs[4 * ib: 4 * ib + 4], qh[2 * ib: 2 * ib + 2]
        idx = [q[0] | ((h[0] << 8) & 0x700), q[1] | ((h[0] << 4) & 0x700),
               q[2] | ((h[1] << 8) & 0x700), q[3] | ((h[1] << 4) & 0x700)]
        delta = [-0.125 if h[0] & 0x08 else 0.125, -0.125 if h[0] & 0x80 else 0.125,
                 -0.125 if h[1] & 0x08 else 0.125, -0.125 if h[1] & 0x80 else 0.125]
        for l in range(4):
            dl = dl1 if l < 2 else dl2
            y += [dl * (int(grid[idx[l]][j]) + delta[l]) for j in range(8)]
    return y


DECODE = {"Q2_0": q2_0, "IQ4_NL": iq4_nl, "IQ4_XS": iq4_xs, "Q3_K": q3_k, "IQ3_S": iq3_s, "IQ3_XXS": iq3_xxs,
          "IQ2_S": iq2_s, "IQ2_XS": iq2_xs, "IQ2_XXS": iq2_xxs, "IQ1_M": iq1_m}


def q6_k(b: bytes, t=None):  # ggml dequantize_row_q6_K: two halves of 128, four runs of 32 a half
    ql, qh, sc = b[0:128], b[128:192], [x - 256 if x > 127 else x for x in b[192:208]]
    d = f16(b[208:210])
    y = [0.0] * 256
    for half in range(2):
        L, H, S, Y = 64 * half, 32 * half, 8 * half, 128 * half
        for l in range(32):
            s = l // 16
            q1 = ((ql[L + l] & 15) | (((qh[H + l] >> 0) & 3) << 4)) - 32
            q2 = ((ql[L + l + 32] & 15) | (((qh[H + l] >> 2) & 3) << 4)) - 32
            q3 = ((ql[L + l] >> 4) | (((qh[H + l] >> 4) & 3) << 4)) - 32
            q4 = ((ql[L + l + 32] >> 4) | (((qh[H + l] >> 6) & 3) << 4)) - 32
            y[Y + l] = d * sc[S + s] * q1
            y[Y + l + 32] = d * sc[S + s + 2] * q2
            y[Y + l + 64] = d * sc[S + s + 4] * q3
            y[Y + l + 96] = d * sc[S + s + 6] * q4
    return y


DECODE["Q6_K"] = q6_k


def dequantize(blocks: np.ndarray, kind: str, block_bytes: int, tables) -> np.ndarray:
    raw = np.asarray(blocks, dtype=np.uint8).reshape(-1, block_bytes)
    return np.array([w for blk in raw for w in DECODE[kind](bytes(blk), tables)], dtype=np.float64)
