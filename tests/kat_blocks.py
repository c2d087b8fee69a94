"""Block builders of the reference's own tests, restated in numpy.

q2_k_block / q3_k_block / q4_k_block / q6_k_block / q8_0_block:
    crates/gguf/src/lib.rs:2535-2610
q4_xs_block / q6_xs_block (Laguna XS known-sum tests):
    crates/backend/src/metal/laguna_xs.rs:2513-2560
q2_patterned_block / q3_patterned_block:
    crates/backend/src/metal/gguf_moe.rs:752-880
"""
import numpy as np


def le16(v):
    return [v & 0xFF, (v >> 8) & 0xFF]


def q2_k_block(d, dmin, scale_mins, quant_byte):
    b = [(s & 0x0F) | ((m & 0x0F) << 4) for s, m in scale_mins]
    b += [quant_byte] * 64
    return np.array(b + le16(d) + le16(dmin), np.uint8)


def q8_0_block(d, start):
    return np.array(le16(d) + [((start + i) & 0xFF) for i in range(32)], np.uint8)


def pack_q3_scales(decoded):
    packed = [0] * 12
    for g, s in enumerate(decoded):
        assert s < 64
        if g < 8:
            packed[g] |= s & 0x0F
        else:
            packed[g - 8] |= (s & 0x0F) << 4
        packed[8 + g % 4] |= ((s >> 4) & 3) << (2 * (g // 4))
    return packed


def q3_k_block(d, decoded_scales, quant_byte, high_mask_byte):
    return q3_patterned_block(d, decoded_scales, [quant_byte] * 64, [high_mask_byte] * 32)


def q3_patterned_block(d, decoded_scales, quant, high_mask):
    b = list(high_mask) + list(quant) + pack_q3_scales(decoded_scales) + le16(d)
    return np.array(b, np.uint8)


def q4_k_block(d, dmin, scale, mn, quant_byte):
    s = [0] * 12
    for g in range(8):
        if g < 4:
            s[g] |= scale & 0x3F
            s[g + 4] |= mn & 0x3F
        else:
            s[g + 4] |= scale & 0x0F
            s[g - 4] |= (scale >> 4) << 6
            s[g + 4] |= (mn & 0x0F) << 4
            s[g] |= (mn >> 4) << 6
    return np.array(le16(d) + le16(dmin) + s + [quant_byte] * 128, np.uint8)


def q6_k_block(d, scale, low, high):
    return np.array([low] * 128 + [high] * 64 + [scale & 0xFF] * 16 + le16(d), np.uint8)


def q4_xs_block(quant):
    b = np.zeros(144, np.uint8)
    b[0:2] = le16(0x3C00)
    b[4:16] = 1
    b[16:] = quant | (quant << 4)
    return b


def q6_xs_block(value):
    quant = value + 32
    low, high = quant & 0x0F, quant >> 4
    b = np.zeros(210, np.uint8)
    b[:128] = low | (low << 4)
    b[128:192] = high | (high << 2) | (high << 4) | (high << 6)
    b[192:208] = 1
    b[208:] = le16(0x3C00)
    return b


def q2_patterned_block(d, dmin, seed):
    b = [(seed + i * 13) & 0xFF for i in range(16)]
    b += [(seed * 29 + i * 17) & 0xFF for i in range(64)]
    return np.array(b + le16(d) + le16(dmin), np.uint8)


def q2_patterned_expert_matrix(seed, rows, in_features):
    """Two experts: expert 0 with d=0x1000 dmin=0x0c00, expert 1 zero scales."""
    bpr = in_features // 256
    out = []
    for expert in range(2):
        for row in range(rows):
            for block in range(bpr):
                bs = (seed + row * 17 + block * 7 + expert * 29) & 0xFF
                out.append(q2_patterned_block(0x1000 if expert == 0 else 0,
                                              0x0C00 if expert == 0 else 0, bs))
    return np.concatenate(out)


def q3_patterned_expert_matrix(seed):
    out = []
    for expert in range(2):
        for row in range(256):
            rs = (seed + row * 17 + expert * 29) & 0xFF
            scales = [(rs + g * 7) & 0x3F for g in range(16)]
            quant = [((rs * 13) + i * 19) & 0xFF for i in range(64)]
            hm = [(((rs << (i % 8)) | (rs >> (8 - i % 8))) & 0xFF) ^ ((i * 11) & 0xFF)
                  if i % 8 else rs ^ ((i * 11) & 0xFF) for i in range(32)]
            out.append(q3_patterned_block(0x1000 if expert == 0 else 0, scales, quant, hm))
    return np.concatenate(out)
