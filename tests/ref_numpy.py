"""Independent vectorised numpy decoders (fp64) used to cross-check the
oracle. Written from the ggml block layout description (loop order of
ggml's dequantize_row_* : 128-value chunks, shifts, 16/32-value groups),
not from the oracle's code, so an index or sign slip in either shows up."""
import numpy as np


def f16(a):
    return np.asarray(a, np.uint16).view(np.float16).astype(np.float64)


def _blocks(raw, nbytes):
    raw = np.asarray(raw, np.uint8)
    return raw.reshape(-1, nbytes)


def q2_k(raw):
    b = _blocks(raw, 84)
    sc = b[:, :16].astype(np.int64)
    qs = b[:, 16:80].astype(np.int64)
    d = f16(b[:, 80].astype(np.uint16) | (b[:, 81].astype(np.uint16) << 8))[:, None]
    dm = f16(b[:, 82].astype(np.uint16) | (b[:, 83].astype(np.uint16) << 8))[:, None]
    out = np.zeros((b.shape[0], 256))
    is_ = 0
    for n in range(2):           # 128-value chunks
        q = qs[:, 32 * n: 32 * n + 32]
        for j in range(4):       # shift 2j
            for half in range(2):
                s = sc[:, is_]
                is_ += 1
                vals = (q[:, 16 * half: 16 * half + 16] >> (2 * j)) & 3
                o = 128 * n + 32 * j + 16 * half
                out[:, o:o + 16] = d * (s & 15)[:, None] * vals - dm * (s >> 4)[:, None]
    return out


def q3_scales(sc):
    sc = sc.astype(np.int64)
    s = np.zeros((sc.shape[0], 16), np.int64)
    for j in range(16):
        low = (sc[:, j] & 15) if j < 8 else (sc[:, j - 8] >> 4)
        high = (sc[:, 8 + j % 4] >> (2 * (j // 4))) & 3
        s[:, j] = low | (high << 4)
    return s - 32


def q3_k(raw):
    b = _blocks(raw, 110)
    hm = b[:, :32].astype(np.int64)
    qs = b[:, 32:96].astype(np.int64)
    s = q3_scales(b[:, 96:108])
    d = f16(b[:, 108].astype(np.uint16) | (b[:, 109].astype(np.uint16) << 8))[:, None]
    out = np.zeros((b.shape[0], 256))
    is_ = 0
    m = 1
    for n in range(2):
        q = qs[:, 32 * n: 32 * n + 32]
        for j in range(4):
            for half in range(2):
                sl = slice(16 * half, 16 * half + 16)
                v = ((q[:, sl] >> (2 * j)) & 3) - np.where(hm[:, sl] & m, 0, 4)
                o = 128 * n + 32 * j + 16 * half
                out[:, o:o + 16] = d * s[:, is_][:, None] * v
                is_ += 1
            m <<= 1
    return out


def q4_k(raw):
    b = _blocks(raw, 144)
    d = f16(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))[:, None]
    dm = f16(b[:, 2].astype(np.uint16) | (b[:, 3].astype(np.uint16) << 8))[:, None]
    s = b[:, 4:16].astype(np.int64)
    qs = b[:, 16:].astype(np.int64)
    out = np.zeros((b.shape[0], 256))
    for j in range(8):
        if j < 4:
            sc, mn = s[:, j] & 63, s[:, j + 4] & 63
        else:
            sc = (s[:, j + 4] & 15) | ((s[:, j - 4] >> 6) << 4)
            mn = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
        q = (qs[:, 32 * (j // 2): 32 * (j // 2) + 32] >> (4 * (j % 2))) & 15
        out[:, 32 * j: 32 * j + 32] = d * sc[:, None] * q - dm * mn[:, None]
    return out


def q6_k(raw):
    b = _blocks(raw, 210)
    ql = b[:, :128].astype(np.int64)
    qh = b[:, 128:192].astype(np.int64)
    sc = b[:, 192:208].view(np.int8).astype(np.int64)
    d = f16(b[:, 208].astype(np.uint16) | (b[:, 209].astype(np.uint16) << 8))[:, None]
    out = np.zeros((b.shape[0], 256))
    for n in range(2):
        for l in range(32):
            isc = l // 16
            L, Hh = ql[:, 64 * n:], qh[:, 32 * n:]
            q1 = ((L[:, l] & 15) | (((Hh[:, l] >> 0) & 3) << 4)) - 32
            q2 = ((L[:, l + 32] & 15) | (((Hh[:, l] >> 2) & 3) << 4)) - 32
            q3 = ((L[:, l] >> 4) | (((Hh[:, l] >> 4) & 3) << 4)) - 32
            q4 = ((L[:, l + 32] >> 4) | (((Hh[:, l] >> 6) & 3) << 4)) - 32
            S = sc[:, 8 * n:]
            out[:, 128 * n + l] = d[:, 0] * S[:, isc] * q1
            out[:, 128 * n + l + 32] = d[:, 0] * S[:, isc + 2] * q2
            out[:, 128 * n + l + 64] = d[:, 0] * S[:, isc + 4] * q3
            out[:, 128 * n + l + 96] = d[:, 0] * S[:, isc + 6] * q4
    return out


def q8_0(raw):
    b = _blocks(raw, 34)
    d = f16(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))[:, None]
    return d * b[:, 2:].view(np.int8).astype(np.float64)


DECODERS = {10: q2_k, 11: q3_k, 12: q4_k, 14: q6_k, 8: q8_0}


def dequant_matrix(quant, raw, rows, cols):
    return DECODERS[quant](raw).reshape(rows, cols)


def silu(x):
    return x / (1.0 + np.exp(-x))


def moe_routed_fp64(quant, down_quant, gate, up, down, x, ids, w, E, k, I):
    """Matrix-form fp64 routed MoE: y[t] = sum_r Wd[e] (silu(Wg[e] x) * (Wu[e] x) * w)."""
    T, H = x.shape
    Wg = dequant_matrix(quant, gate, E * I, H).reshape(E, I, H)
    Wu = dequant_matrix(quant, up, E * I, H).reshape(E, I, H)
    Wd = dequant_matrix(down_quant, down, E * H, I).reshape(E, H, I)
    y = np.zeros((T, H))
    x64 = x.astype(np.float64)
    for t in range(T):
        for r in range(k):
            e = int(ids[t * k + r])
            h = silu(Wg[e] @ x64[t]) * (Wu[e] @ x64[t]) * float(w[t * k + r])
            y[t] += Wd[e] @ h
    return y


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
