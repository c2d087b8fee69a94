"""Pins the CPU oracle: the reference's known-answer tests, exhaustive f16,
independent fp64 numpy decoders, closed forms and brute force."""
import numpy as np
import pytest

import kat_blocks as kb
import oracle_lib as orc
import ref_numpy as rn

Q8_0, Q2_K, Q3_K, Q4_K, Q6_K = 8, 10, 11, 12, 14
rng = np.random.default_rng(1234)


def test_f16_exhaustive_matches_numpy():
    # crates/gguf/src/lib.rs:1501-1528 vs IEEE half (numpy) for all 65536 patterns
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.L().oracle_f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # NaN payload is kept (fraction << 13), as the reference does
    assert got.view(np.uint32)[0x7E01] == 0x7F800000 | (0x201 << 13)


def test_q2_k_reference_kat():
    # crates/gguf/src/lib.rs:2056-2081 with builder tiny_q2_k_values_gguf (:2388-2424)
    sm = [(1, 0), (2, 1), (3, 2), (4, 3), (5, 4), (6, 5), (7, 6), (8, 7), (9, 8), (10, 9),
          (11, 10), (12, 11), (13, 12), (14, 13), (15, 14), (0, 15)]
    v = orc.dequantize(Q2_K, kb.q2_k_block(0x3C00, 0x3800, sm, 0xE4))
    expect = {0: 0.0, 16: -0.5, 32: 2.0, 48: 2.5, 64: 8.0, 80: 9.5, 96: 18.0, 112: 20.5,
              128: -4.0, 144: -4.5, 160: 6.0, 176: 6.5, 192: 20.0, 208: 21.5, 224: 38.0,
              240: -7.5}
    for i, e in expect.items():
        assert v[i] == e, (i, v[i], e)


def test_q3_k_reference_kat():
    # crates/gguf/src/lib.rs:2083-2104
    v = orc.dequantize(Q3_K, kb.q3_k_block(0x3C00, [33] * 16, 0xE4, 0xFF))
    for g, e in enumerate([0, 0, 1, 1, 2, 2, 3, 3, 0, 0, 1, 1, 2, 2, 3, 3]):
        assert v[16 * g] == e and v[16 * g + 15] == e


def test_q4_k_reference_kat():
    # crates/gguf/src/lib.rs:2106-2122
    v = orc.dequantize(Q4_K, kb.q4_k_block(0x3C00, 0x0000, 1, 0, 0x21))
    for g in range(8):
        e = 1.0 if g % 2 == 0 else 2.0
        assert v[32 * g] == e and v[32 * g + 31] == e


def test_q6_k_reference_kat():
    # crates/gguf/src/lib.rs:2124-2139
    v = orc.dequantize(Q6_K, kb.q6_k_block(0x3C00, 1, 0x00, 0x00))
    assert np.all(v == -32.0)


def test_q8_0_reference_kat():
    # crates/gguf/src/lib.rs:2037-2054
    v = orc.dequantize(Q8_0, kb.q8_0_block(0x3800, -8))
    assert v[0] == -4.0 and v[1] == -3.5 and v[16] == 4.0 and v[31] == 11.5


def _random_blocks(quant, n):
    """Random bytes with finite f16 scale fields."""
    bb = {Q2_K: 84, Q3_K: 110, Q4_K: 144, Q6_K: 210, Q8_0: 34}[quant]
    raw = rng.integers(0, 256, size=(n, bb), dtype=np.uint8)
    scale_at = {Q2_K: [80, 82], Q3_K: [108], Q4_K: [0, 2], Q6_K: [208], Q8_0: [0]}[quant]
    for off in scale_at:
        h = rng.standard_normal(n).astype(np.float16).view(np.uint16)
        raw[:, off] = h & 0xFF
        raw[:, off + 1] = h >> 8
    return raw.reshape(-1)


@pytest.mark.parametrize("quant", [Q2_K, Q3_K, Q4_K, Q6_K, Q8_0])
def test_dequant_matches_independent_fp64_decoder(quant):
    raw = _random_blocks(quant, 512)
    got = orc.dequantize(quant, raw).astype(np.float64)
    ref = rn.DECODERS[quant](raw).reshape(-1)
    # fp32 evaluation of a 2-3 term expression: a few ulp of the largest term
    assert np.allclose(got, ref, rtol=2e-6, atol=1e-6 * np.abs(ref).max())


def test_dequant_rejects_non_finite_scale():
    b = kb.q2_k_block(0x7C00, 0, [(1, 1)] * 16, 0)
    with pytest.raises(ValueError):
        orc.dequantize(Q2_K, b)


def test_router_tie_prefers_lower_id():
    # crates/model/src/moe_router.rs:963-972 (tiny_config: k=2, scale 2.5, renorm)
    ids, w = orc.router_topk(np.array([[0.5, 0.5, 0.1, 0.2]], np.float32),
                             np.zeros(4, np.float32), 2, 0, True, 2.5)
    assert list(ids) == [0, 1]
    assert abs(w[0] - 1.25) <= 1e-6 and abs(w[1] - 1.25) <= 1e-6


def _brute_topk(logits, bias, k, score_fn, norm, scale):
    T, E = logits.shape
    ids, ws = [], []
    for t in range(T):
        l64 = logits[t].astype(np.float64)
        if score_fn == 0:
            score = 1.0 / (1.0 + np.exp(-l64))
            sel = score.astype(np.float32) + (bias if bias is not None else 0)
        else:
            score = np.exp(l64 - l64.max())
            sel = logits[t] + (bias if bias is not None else 0)
        order = sorted(range(E), key=lambda e: (-float(sel[e]), e))[:k]
        w = score[order]
        w = w / w.sum() if norm else (w / score.sum() if score_fn == 1 else w)
        ids += order
        ws += list(w * scale)
    return np.array(ids), np.array(ws)


def test_router_specialised_decode_inputs():
    # inputs of specialized_decode_top8_matches_the_reference_router
    # (crates/backend/src/metal/laguna_xs.rs:2269-2316)
    E = 256
    logits = ((np.arange(E, dtype=np.float32) / 64.0) - 2.0)[None]
    bias = np.zeros(E, np.float32)
    bias[3], bias[7], bias[11] = 2.0, 1.9, 1.8
    ids, w = orc.router_topk(logits, bias, 8, 0, True, 1.25)
    bids, bw = _brute_topk(logits, bias, 8, 0, True, 1.25)
    assert list(ids[:3]) == [3, 7, 11]
    assert list(ids) == list(bids)
    assert np.allclose(w, bw, rtol=1e-6)
    assert abs(float(np.sum(w.astype(np.float64))) - 1.25) < 1e-6


@pytest.mark.parametrize("score_fn,norm", [(0, True), (0, False), (1, True), (1, False)])
def test_router_matches_brute_force(score_fn, norm):
    T, E, k = 37, 64, 8
    logits = rng.standard_normal((T, E)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(E)).astype(np.float32) if score_fn == 0 else None
    ids, w = orc.router_topk(logits, bias, k, score_fn, norm, 2.5)
    bids, bw = _brute_topk(logits, bias, k, score_fn, norm, 2.5)
    assert list(ids) == list(bids)
    assert np.allclose(w, bw, rtol=2e-6)


def test_dispatch_reference_kats():
    # crates/moe/src/routing.rs:91-141
    ids = np.array([1, 2, 2, 3], np.uint32)  # token 0 -> [1,2], token 1 -> [2,3]
    off, srt = orc.dispatch(ids, 2, 2, 4)
    e2 = srt[off[2]:off[3]]
    assert list(e2 // 2) == [0, 1] and list(e2 % 2) == [1, 0]
    ids = np.array([0, 1, 0, 2, 0, 3], np.uint32)
    off, srt = orc.dispatch(ids, 3, 2, 4)
    assert list(np.diff(off)) == [3, 1, 1, 1]
    assert list(srt[:3]) == [0, 2, 4]


def test_dispatch_invariants_random():
    T, k, E = 500, 8, 256
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).reshape(-1).astype(np.uint32)
    off, srt = orc.dispatch(ids, T, k, E)
    assert off[-1] == T * k and sorted(srt) == list(range(T * k))
    for e in range(E):
        seg = srt[off[e]:off[e + 1]]
        assert np.all(ids[seg] == e) and np.all(np.diff(seg.astype(np.int64)) > 0)


def test_combine_reference_kat():
    # crates/backend/src/backend.rs:11358-11384
    out = orc.weighted_index_add_combine(np.zeros((4, 2), np.float32), [0, 2, 2],
                                         np.arange(1, 7, dtype=np.float32).reshape(3, 2),
                                         [1.0, 0.5, 2.0])
    assert list(out[0]) == [1.0, 2.0] and list(out[2]) == [11.5, 14.0]


def test_rms_norm_matches_fp64():
    x = rng.standard_normal((5, 4096)).astype(np.float32)
    w = rng.standard_normal(4096).astype(np.float32)
    got = orc.rms_norm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-6) * w
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("quant", [Q2_K, Q3_K, Q4_K, Q6_K, Q8_0])
def test_qmatvec_matches_fp64(quant):
    rows, cols = 48, 1024
    raw = _random_blocks(quant, rows * cols // (256 if quant != Q8_0 else 32))
    x = rng.standard_normal(cols).astype(np.float32)
    got = orc.qmatvec(quant, raw, rows, cols, x)
    ref = rn.dequant_matrix(quant, raw, rows, cols) @ x.astype(np.float64)
    assert rn.rel_l2(got, ref) < 1e-5


def test_q3_known_block_closed_form():
    # q3_selected_expert_matches_known_block_values
    # (crates/backend/src/metal/gguf_moe.rs:468-514): y = silu(d)*d*d, d=384/1024
    sel = kb.q3_k_block(0x1400, [33] * 16, 0xE4, 0xFF)
    unused = kb.q3_k_block(0, [33] * 16, 0xE4, 0xFF)
    w = np.concatenate([np.tile(sel, 256), np.tile(unused, 256)])
    x = np.ones((1, 256), np.float32)
    y = orc.moe_routed(Q3_K, Q3_K, w, w, w, x, np.array([0], np.uint32),
                       np.array([1.0], np.float32), 2, 1, 256)
    d = 384.0 / 1024
    assert np.allclose(y, d / (1 + np.exp(-d)) * d * d, atol=1e-6)


@pytest.mark.parametrize("down", [Q4_K, Q6_K])
def test_xs_top8_known_sum(down):
    # top8_routed_moe_parallel_down_matches_the_known_sum
    # (crates/backend/src/metal/laguna_xs.rs:1905-1974)
    E = k = 8
    H, I = 256, 512
    vals = list(range(1, 9))
    gate = np.concatenate([np.tile(kb.q4_xs_block(v), I * H // 256) for v in vals])
    blk = kb.q4_xs_block(1) if down == Q4_K else kb.q6_xs_block(1)
    dn = np.concatenate([np.tile(blk, H * I // 256) for _ in vals])
    x = np.full((1, H), 1.0 / H, np.float32)
    ids, w = orc.router_topk(np.zeros((1, E), np.float32), np.zeros(E, np.float32), k, 0, True,
                             1.0)
    y = orc.moe_routed(Q4_K, down, gate, gate, dn, x, ids, w, E, k, I)
    expect = sum((I / k) * v * v / (1 + np.exp(-v)) for v in vals)
    assert np.allclose(y, expect, rtol=1e-5)


@pytest.mark.parametrize("quant,down", [(Q2_K, Q2_K), (Q3_K, Q3_K), (Q4_K, Q4_K), (Q4_K, Q6_K)])
def test_moe_routed_matches_fp64(quant, down):
    T, H, I, E, k = 3, 512, 256, 6, 3
    gb = 256 if quant != Q8_0 else 32
    gate = _random_blocks(quant, E * I * H // gb)
    up = _random_blocks(quant, E * I * H // gb)
    dn = _random_blocks(down, E * H * I // 256)
    # scale weights down so activations stay O(1)
    x = (0.05 * rng.standard_normal((T, H))).astype(np.float32)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).reshape(-1).astype(np.uint32)
    w = rng.random(T * k).astype(np.float32)
    got = orc.moe_routed(quant, down, gate, up, dn, x, ids, w, E, k, I)
    ref = rn.moe_routed_fp64(quant, down, gate, up, dn, x, ids, w, E, k, I)
    assert rn.rel_l2(got, ref) < 1e-4


def test_shared_q8_0_matches_fp64():
    T, H, Is = 2, 512, 256
    g = _random_blocks(Q8_0, Is * H // 32)
    u = _random_blocks(Q8_0, Is * H // 32)
    d = _random_blocks(Q8_0, H * Is // 32)
    x = (0.05 * rng.standard_normal((T, H))).astype(np.float32)
    ra = rng.standard_normal((T, H)).astype(np.float32)
    rb = rng.standard_normal((T, H)).astype(np.float32)
    got = orc.shared_q8_0(g, u, d, x, Is, routed=ra, residual=rb)
    Wg = rn.dequant_matrix(Q8_0, g, Is, H)
    Wu = rn.dequant_matrix(Q8_0, u, Is, H)
    Wd = rn.dequant_matrix(Q8_0, d, H, Is)
    x64 = x.astype(np.float64)
    hs = rn.silu(x64 @ Wg.T) * (x64 @ Wu.T)
    ref = ra + rb + hs @ Wd.T
    assert rn.rel_l2(got, ref) < 1e-5


def test_bf16_round_matches_torch_nearest_even():
    # the host-side bf16 rounding the stack tests use, against torch's
    # fp32 -> bf16 conversion (round to nearest even), ties included
    import parity_helpers as ph
    import torch
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(100000) * 10.0 ** rng.integers(-20, 20, 100000)).astype(np.float32)
    ties = (rng.integers(0, 0x7F00, 1000, dtype=np.uint32) << 16) | 0x8000  # finite
    x = np.concatenate([x, ties.view(np.float32), np.float32([0.0, -0.0, 1.0, 65504.0])])
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ph.bf16_round(x).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("sq,sdq", [(Q4_K, Q4_K), (Q4_K, Q6_K), (Q8_0, Q8_0)])
def test_shared_ffn_matches_fp64(sq, sdq):
    # the shared expert in the Laguna XS formats (Q4_K gate/up, Q4_K or Q6_K
    # down) and Q8_0, against fp64 over the independently decoded weights
    T, H, Is = 3, 512, 256
    gb = 32 if sq == Q8_0 else 256
    db = 32 if sdq == Q8_0 else 256
    g = _random_blocks(sq, Is * H // gb)
    u = _random_blocks(sq, Is * H // gb)
    d = _random_blocks(sdq, H * Is // db)
    x = (0.05 * rng.standard_normal((T, H))).astype(np.float32)
    ra = rng.standard_normal((T, H)).astype(np.float32)
    got = orc.shared_ffn(sq, sdq, g, u, d, x, Is, routed=ra)
    x64 = x.astype(np.float64)
    hs = rn.silu(x64 @ rn.dequant_matrix(sq, g, Is, H).T) * (x64 @ rn.dequant_matrix(sq, u, Is, H).T)
    ref = ra + hs @ rn.dequant_matrix(sdq, d, H, Is).T
    assert rn.rel_l2(got, ref) < 1e-5
    if sq == Q8_0:  # the Q8_0 entry point is the same computation
        assert np.array_equal(got, orc.shared_q8_0(g, u, d, x, Is, routed=ra))


def test_oracle_batched_rows_match_per_token_calls():
    # the oracle dequantises each expert row once and dots it with all the
    # expert's tokens, four summation chains at a time; every token's result
    # must equal the same token computed on its own (one row per call, the
    # single-chain path), bit for bit
    T, H, I, E, k = 9, 512, 256, 4, 3
    gate = _random_blocks(Q2_K, E * I * H // 256)
    up = _random_blocks(Q2_K, E * I * H // 256)
    dn = _random_blocks(Q2_K, E * H * I // 256)
    x = (0.05 * rng.standard_normal((T, H))).astype(np.float32)
    ids = rng.integers(0, E, T * k).astype(np.uint32)  # repeats inside a token allowed
    w = rng.random(T * k).astype(np.float32)
    batch = orc.moe_routed(Q2_K, Q2_K, gate, up, dn, x, ids, w, E, k, I)
    for t in range(T):
        one = orc.moe_routed(Q2_K, Q2_K, gate, up, dn, x[t:t + 1], ids[t * k:(t + 1) * k],
                             w[t * k:(t + 1) * k], E, k, I)
        assert np.array_equal(one.view(np.uint32), batch[t:t + 1].view(np.uint32))
    sg = _random_blocks(Q8_0, 256 * H // 32)
    su = _random_blocks(Q8_0, 256 * H // 32)
    sd = _random_blocks(Q8_0, H * 256 // 32)
    sb = orc.shared_q8_0(sg, su, sd, x, 256, routed=batch)
    for t in range(T):
        one = orc.shared_q8_0(sg, su, sd, x[t:t + 1], 256, routed=batch[t:t + 1])
        assert np.array_equal(one.view(np.uint32), sb[t:t + 1].view(np.uint32))
