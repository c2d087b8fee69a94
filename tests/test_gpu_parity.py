"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Bars: dequantised weights bit-exact; selected
expert ids exact except near-ties within 1e-6 of the k-th selection value
(counted and reported); MoE outputs within relative L2 2e-3.
"""
import dataclasses
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import kat_blocks as kb
import oracle_lib as orc
import parity_helpers as ph
import ref_numpy as rn
from inferno_amd import configs as cf
from inferno_amd import ops
from inferno_amd._lib import Q2_K, Q3_K, Q4_K, Q6_K, Q8_0, SCORE_SIGMOID, SCORE_SOFTMAX

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(7)
BB = {Q2_K: 84, Q3_K: 110, Q4_K: 144, Q6_K: 210, Q8_0: 34}


def random_blocks(quant, n):
    raw = rng.integers(0, 256, size=(n, BB[quant]), dtype=np.uint8)
    scale_at = {Q2_K: [80, 82], Q3_K: [108], Q4_K: [0, 2], Q6_K: [208], Q8_0: [0]}[quant]
    for off in scale_at:
        h = (0.01 * rng.standard_normal(n)).astype(np.float16).view(np.uint16)
        raw[:, off] = h & 0xFF
        raw[:, off + 1] = h >> 8
    return raw.reshape(-1)


def dev(a, cuda):
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


@pytest.mark.parametrize("quant", [Q2_K, Q3_K, Q4_K, Q6_K, Q8_0])
def test_dequant_bit_exact(cuda, quant):
    raw = random_blocks(quant, 4096)
    # include subnormal and zero scales
    raw[BB[quant] * 0: BB[quant] * 1] = 0
    got = ph.to_np(ops.dequantize(quant, dev(raw, cuda)))
    ref = orc.dequantize(quant, raw)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_reference_kats(cuda):
    sm = [(i + 1 if i < 15 else 0, i) for i in range(16)]
    v = ph.to_np(ops.dequantize(Q2_K, dev(kb.q2_k_block(0x3C00, 0x3800, sm, 0xE4), cuda)))
    assert v[16] == -0.5 and v[224] == 38.0 and v[240] == -7.5
    v = ph.to_np(ops.dequantize(Q4_K, dev(kb.q4_k_block(0x3C00, 0, 1, 0, 0x21), cuda)))
    assert v[0] == 1.0 and v[32] == 2.0
    v = ph.to_np(ops.dequantize(Q8_0, dev(kb.q8_0_block(0x3800, -8), cuda)))
    assert v[0] == -4.0 and v[31] == 11.5


@pytest.mark.parametrize("T,H,E,bf16", [(1, 6144, 256, True), (16, 2048, 64, False),
                                        (77, 4096, 128, True), (100, 2048, 100, False),
                                        (2100, 1024, 256, True), (2050, 512, 72, False),
                                        (40, 800, 64, True)])
def test_router_logits(cuda, T, H, E, bf16):
    x = torch.randn(T, H, device=cuda)
    if bf16:
        x = x.bfloat16()
    w = 0.02 * torch.randn(E, H, device=cuda)
    got = ph.to_np(ops.router_logits(x, w)).astype(np.float64)
    xs, ws = ph.x_f32(x).astype(np.float64), ph.to_np(w).astype(np.float64)
    ref64 = xs @ ws.T
    cond = np.abs(xs) @ np.abs(ws).T  # fp32 summation error scales with sum |x*w|
    orc_err = np.abs(orc.linear(ph.x_f32(x), ph.to_np(w)) - ref64)
    assert np.all(np.abs(got - ref64) <= 2e-6 * cond)
    assert np.all(orc_err <= 2e-5 * cond)


@pytest.mark.parametrize("score_fn,norm,E,k", [(SCORE_SIGMOID, True, 256, 8),
                                               (SCORE_SOFTMAX, True, 64, 8),
                                               (SCORE_SOFTMAX, True, 128, 10),
                                               (SCORE_SOFTMAX, False, 128, 10),
                                               (SCORE_SIGMOID, False, 100, 16)])
def test_router_topk_matches_oracle(cuda, score_fn, norm, E, k):
    T = 333
    logits = (1.5 * rng.standard_normal((T, E))).astype(np.float32)
    bias = (0.1 * rng.standard_normal(E)).astype(np.float32) if score_fn == SCORE_SIGMOID else None
    ids, w, tok = ops.router_topk(dev(logits, cuda), None if bias is None else dev(bias, cuda),
                                  k, score_fn, norm, 2.5)
    oid, ow = orc.router_topk(logits, bias, k, score_fn, norm, 2.5)
    spec = SimpleNamespace(score_fn=score_fn, top_k=k)
    sel = ph.selection_values(spec, logits, bias)
    _, flips = ph.compare_routing(spec, ph.to_np(ids).view(np.uint32), oid, sel)
    print(f"near-tie tokens: {flips}")
    same = (ph.to_np(ids).view(np.uint32).reshape(T, k) == oid.reshape(T, k)).all(1)
    assert np.allclose(ph.to_np(w).reshape(T, k)[same], ow.reshape(T, k)[same], rtol=2e-6,
                       atol=1e-7)
    assert np.array_equal(ph.to_np(tok), np.repeat(np.arange(T), k))


def test_router_tie_kat(cuda):
    # crates/model/src/moe_router.rs:963-972
    ids, w, _ = ops.router_topk(dev(np.array([[0.5, 0.5, 0.1, 0.2]], np.float32), cuda),
                                dev(np.zeros(4, np.float32), cuda), 2, SCORE_SIGMOID, True, 2.5)
    assert list(ph.to_np(ids)) == [0, 1]
    assert np.allclose(ph.to_np(w), [1.25, 1.25], atol=1e-6)


@pytest.mark.parametrize("E", [8, 64, 65, 128, 256])
def test_router_topk_tiers(cuda, E):
    """Router top-k over widths on both sides of the one-candidate-per-lane
    selection (E <= 64) with tied logits in three tiers and a tie-breaking
    bias on some experts: ids (rank order) and weights as the oracle's."""
    T, k = 6, min(8, E)
    rng = np.random.default_rng(E)
    tiers = np.array([-1.0, 0.0, 0.75], np.float32)
    logits = tiers[rng.integers(0, 3, size=(T, E))].astype(np.float32)
    bias = np.zeros(E, np.float32)
    bias[rng.choice(E, size=max(1, E // 8), replace=False)] = 0.125
    for score_fn in (SCORE_SIGMOID, SCORE_SOFTMAX):
        b = bias if score_fn == SCORE_SIGMOID else None
        ids, w, _ = ops.router_topk(dev(logits, cuda), None if b is None else dev(b, cuda), k,
                                    score_fn, True, 1.5)
        oid, ow = orc.router_topk(logits, b, k, score_fn, True, 1.5)
        assert np.array_equal(ph.to_np(ids).view(np.uint32), oid), (E, score_fn)
        np.testing.assert_allclose(ph.to_np(w), ow, rtol=2e-6, atol=0)


def test_router_specialised_decode_case(cuda):
    # laguna_xs.rs:2269-2316 inputs; expected ids from the oracle
    E = 256
    logits = ((np.arange(E, dtype=np.float32) / 64.0) - 2.0)[None]
    bias = np.zeros(E, np.float32)
    bias[3], bias[7], bias[11] = 2.0, 1.9, 1.8
    ids, w, _ = ops.router_topk(dev(logits, cuda), dev(bias, cuda), 8, SCORE_SIGMOID, True, 1.25)
    oid, ow = orc.router_topk(logits, bias, 8, 0, True, 1.25)
    assert list(ph.to_np(ids)) == list(oid)
    assert np.allclose(ph.to_np(w), ow, rtol=2e-6)


@pytest.mark.parametrize("T,k,E", [(1, 8, 256), (16, 8, 64), (512, 8, 256), (4096, 8, 256),
                                   (37, 10, 128), (3, 1, 1), (1111, 7, 200)])
def test_dispatch_matches_oracle(cuda, T, k, E):
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).reshape(-1).astype(np.uint32)
    if T == 4096:  # heavy skew: half the tokens share experts 0..7
        ids.reshape(T, k)[: T // 2] = np.arange(8)
    off, srt, act = ops.dispatch(dev(ids.view(np.int32), cuda), T, k, E)
    ooff, osrt = orc.dispatch(ids, T, k, E)
    assert np.array_equal(ph.to_np(off).view(np.uint32), ooff)
    assert np.array_equal(ph.to_np(srt).view(np.uint32), osrt)
    a = ph.to_np(act)
    used = np.nonzero(np.diff(ooff))[0]
    assert a[0] == len(used) and np.array_equal(a[1: 1 + len(used)], used)


def test_dispatch_empty(cuda):
    off, srt, act = ops.dispatch(torch.zeros(1, dtype=torch.int32, device=cuda), 0, 8, 16)
    assert ph.to_np(off).sum() == 0 and ph.to_np(act)[0] == 0


def _moe_case(cuda, quant, down, T, H, I, E, k, x_bf16):
    gb = 256
    gate = random_blocks(quant, E * I * H // gb)
    up = random_blocks(quant, E * I * H // gb)
    dn = random_blocks(down, E * H * I // 256)
    x = torch.randn(T, H, device=cuda)
    if x_bf16:
        x = x.bfloat16()
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).reshape(-1).astype(np.uint32)
    w = rng.random(T * k).astype(np.float32)
    out = ops.gguf_moe(quant, down, dev(gate, cuda), dev(up, cuda), dev(dn, cuda), x,
                       dev(ids.view(np.int32), cuda), dev(w, cuda), k, E, I)
    ref = orc.moe_routed(quant, down, gate, up, dn, ph.x_f32(x), ids, w, E, k, I)
    return ph.to_np(out), ref


@pytest.mark.parametrize("quant,down", [(Q2_K, Q2_K), (Q3_K, Q3_K), (Q4_K, Q4_K), (Q4_K, Q6_K)])
@pytest.mark.parametrize("T,H,I,E,k,bf16", [(1, 512, 256, 16, 4, True), (4, 256, 256, 16, 4, False),
                                            (9, 768, 512, 8, 3, True), (33, 1536, 768, 12, 5, False)])
def test_gguf_moe_matches_oracle(cuda, switches, quant, down, T, H, I, E, k, bf16):
    # the GEMV kernels at every T: random Q4_K bytes give gate/up products
    # past the f16 range of the grouped GEMM's h (that path is tested on
    # synthesised weights in test_gguf_moe_mfma_prefill)
    switches(INFERNO_PREFILL_MIN_ASSIGNMENTS="100000")
    got, ref = _moe_case(cuda, quant, down, T, H, I, E, k, bf16)
    err = rn.rel_l2(got, ref)
    print(f"rel_l2={err:.3e}")
    assert err < ph.TOL_REL_L2


def _skewed_ids(T, E, k, hot=(0, 1), share=(1.0, 0.8)):
    """Routing where expert hot[i] takes a `share[i]` fraction of the tokens
    (ranks 0, 1, ...) and the other ranks are random distinct experts."""
    rows = []
    for _ in range(T):
        first = [h for h, p in zip(hot, share) if rng.random() < p]
        rest = [e for e in rng.permutation(E) if e not in first][: k - len(first)]
        rows.append(first + rest)
    return np.array(rows, np.uint32).reshape(-1)


@pytest.mark.parametrize("quant,down", [(Q2_K, Q2_K), (Q3_K, Q3_K), (Q4_K, Q4_K), (Q4_K, Q6_K)])
@pytest.mark.parametrize("T,H,I,E,k,bf16,skew", [(64, 512, 256, 16, 4, True, False),
                                                 (96, 768, 512, 8, 4, False, True),
                                                 (40, 512, 256, 8, 4, True, "dup")])
def test_gguf_moe_mfma_prefill(cuda, quant, down, T, H, I, E, k, bf16, skew):
    # T * k >= 48 assignments: the MFMA grouped GEMM (f16 operands, fp32
    # accumulation). The skewed case gives two experts >= 64 rows (128-row
    # tiles) next to small experts (32-row tiles). "dup": caller ids that
    # name expert 0 twice in every token (the entry point takes any ids),
    # so one expert holds 2 T = 80 rows although T = 40: the 128-row tile
    # launch must run (the layer's own top-k never repeats an id, and there
    # T <= 64 skips it).
    # weights of realistic size (N(0, 0.02) quantised): the f16 operands and
    # the f16 intermediate, as in the reference's prefill kernels
    # (gguf_moe_prefill_kernels.metal:50-59, :263), cover |h| < 65504 only
    seed = 77 + quant
    gate = ph.to_np(ops.synth_quantized(quant, seed, 0.02, E * I, H, cuda))
    up = ph.to_np(ops.synth_quantized(quant, seed + 1, 0.02, E * I, H, cuda))
    dn = ph.to_np(ops.synth_quantized(down, seed + 2, 0.02, E * H, I, cuda))
    x = torch.randn(T, H, device=cuda)
    if bf16:
        x = x.bfloat16()
    if skew == "dup":
        ids = np.stack([np.concatenate([[0, 0], 1 + rng.permutation(E - 1)[:k - 2]])
                        for _ in range(T)]).reshape(-1).astype(np.uint32)
    else:
        ids = (_skewed_ids(T, E, k) if skew else
               np.stack([rng.permutation(E)[:k] for _ in range(T)]).reshape(-1).astype(np.uint32))
    w = rng.random(T * k).astype(np.float32)
    args = (quant, down, dev(gate, cuda), dev(up, cuda), dev(dn, cuda), x,
            dev(ids.view(np.int32), cuda), dev(w, cuda), k, E, I)
    out = ops.gguf_moe(*args)
    out2 = ops.gguf_moe(*args)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "MFMA prefill output is not bitwise reproducible"
    ref = orc.moe_routed(quant, down, gate, up, dn, ph.x_f32(x), ids, w, E, k, I)
    err = rn.rel_l2(ph.to_np(out), ref)
    print(f"rel_l2={err:.3e}")
    ops.kernel_timing(True)
    try:
        ops.gguf_moe(*args)
        torch.cuda.synchronize()
        assert ops.kernel_timing_label(ops.TIMER_DOWN).startswith("prefill:")
    finally:
        ops.kernel_timing(False)
    assert err < ph.TOL_REL_L2


def test_q3_known_block(cuda):
    # gguf_moe.rs:468-514: silu(d)*d*d with d = 384/1024
    sel = kb.q3_k_block(0x1400, [33] * 16, 0xE4, 0xFF)
    unused = kb.q3_k_block(0, [33] * 16, 0xE4, 0xFF)
    wb = dev(np.concatenate([np.tile(sel, 256), np.tile(unused, 256)]), cuda)
    x = torch.ones(1, 256, device=cuda)
    ids, w, _ = ops.router_topk(dev(np.array([[10.0, -10.0]], np.float32), cuda),
                                dev(np.zeros(2, np.float32), cuda), 1, SCORE_SIGMOID, True, 1.0)
    out = ph.to_np(ops.gguf_moe(Q3_K, Q3_K, wb, wb, wb, x, ids, w, 1, 2, 256))
    d = 384.0 / 1024
    assert np.allclose(out, d / (1 + np.exp(-d)) * d * d, atol=1e-4)


@pytest.mark.parametrize("down", [Q4_K, Q6_K])
def test_xs_top8_known_sum(cuda, down):
    # laguna_xs.rs:1905-1974 closed form sum_v (I/k) v^2 sigmoid(v)
    E = k = 8
    H, I = 256, 512
    vals = list(range(1, 9))
    gate = np.concatenate([np.tile(kb.q4_xs_block(v), I * H // 256) for v in vals])
    blk = kb.q4_xs_block(1) if down == Q4_K else kb.q6_xs_block(1)
    dn = np.concatenate([np.tile(blk, H * I // 256) for _ in vals])
    x = torch.full((1, H), 1.0 / H, device=cuda)
    ids, w, _ = ops.router_topk(torch.zeros(1, E, device=cuda), torch.zeros(E, device=cuda), k,
                                SCORE_SIGMOID, True, 1.0)
    g = dev(gate, cuda)
    out = ph.to_np(ops.gguf_moe(Q4_K, down, g, g, dev(dn, cuda), x, ids, w, k, E, I))
    expect = sum((I / k) * v * v / (1 + np.exp(-v)) for v in vals)
    assert np.allclose(out, expect, rtol=1e-5)


@pytest.mark.parametrize("T,H,Is", [(1, 6144, 2048), (5, 1024, 512)])
def test_shared_q8_0(cuda, T, H, Is):
    g = random_blocks(Q8_0, Is * H // 32)
    u = random_blocks(Q8_0, Is * H // 32)
    d = random_blocks(Q8_0, H * Is // 32)
    x = torch.randn(T, H, device=cuda).bfloat16()
    ra = torch.randn(T, H, device=cuda)
    rb = torch.randn(T, H, device=cuda)
    hs = ops.q8_0_gate_up_swiglu(dev(g, cuda), dev(u, cuda), x, Is)
    out = ops.q8_0_matvec_add2(dev(d, cuda), hs, ra, rb, H)
    ref = orc.shared_q8_0(g, u, d, ph.x_f32(x), Is, routed=ph.to_np(ra), residual=ph.to_np(rb))
    assert rn.rel_l2(ph.to_np(out), ref) < ph.TOL_REL_L2


def test_combine_and_gather_kats(cuda):
    # backend.rs:11336-11384
    acc = torch.zeros(4, 2, device=cuda)
    tok = torch.tensor([0, 2, 2], dtype=torch.int32, device=cuda)
    y = torch.arange(1, 7, dtype=torch.float32, device=cuda).view(3, 2)
    w = torch.tensor([1.0, 0.5, 2.0], device=cuda)
    out = ph.to_np(ops.weighted_index_add_combine(acc, tok, y, w))
    assert list(out[0]) == [1.0, 2.0] and list(out[2]) == [11.5, 14.0]
    x = torch.tensor([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], device=cuda)
    g = ph.to_np(ops.gather_tokens(x, torch.tensor([2, 0, 2], dtype=torch.int32, device=cuda)))
    assert g.tolist() == [[5.0, 6.0], [1.0, 2.0], [5.0, 6.0]]
    yk = torch.randn(6, 8, device=cuda)
    wk = torch.rand(6, device=cuda)
    sh, res = torch.randn(3, 8, device=cuda), torch.randn(3, 8, device=cuda)
    c = ph.to_np(ops.topk_combine_residual(sh, res, yk, wk, 2))
    ref = ph.to_np(sh + res + (yk * wk[:, None]).view(3, 2, 8).sum(1))
    assert np.allclose(c, ref, rtol=1e-6, atol=1e-6)
    # the four-column kernel (k up to 8 and up to 16) and the scalar one
    # (H not a multiple of 4): rank order, against fp64 sums
    for T, k, H in ((5, 10, 64), (4, 7, 256), (3, 3, 6)):
        yk = torch.randn(T * k, H, device=cuda)
        wk = torch.rand(T * k, device=cuda)
        sh, res = torch.randn(T, H, device=cuda), torch.randn(T, H, device=cuda)
        c = ph.to_np(ops.topk_combine_residual(sh, res, yk, wk, k))
        y64 = ph.to_np(yk).astype(np.float64) * ph.to_np(wk).astype(np.float64)[:, None]
        ref = ph.to_np(sh).astype(np.float64) + ph.to_np(res) + y64.reshape(T, k, H).sum(1)
        assert np.allclose(c, ref, rtol=1e-5, atol=1e-5), (T, k, H)


def test_rms_norm(cuda):
    x = torch.randn(7, 4096, device=cuda)
    w = torch.randn(4096, device=cuda)
    got = ph.to_np(ops.rms_norm(x, w, 1e-6))
    ref = orc.rms_norm(ph.to_np(x), ph.to_np(w), 1e-6)
    assert np.allclose(got, ref, rtol=2e-6, atol=1e-6)


def _layer_parity(cuda, key, T, tokens=None, variants=1, tol=None):
    """Layer output against the oracle on `variants` seeded inputs of T tokens
    (rows `tokens` of each; all rows by default). The MoE part's relative L2
    error is taken over all checked rows together and must stay below `tol`
    (default); returns it."""
    cfg = cf.CONFIGS[key] if isinstance(key, str) else key
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=T)
    tokens = np.arange(T) if tokens is None else np.asarray(tokens)
    got_all, ref_all, flips = [], [], 0
    for v in range(variants):
        x = cf.make_input(cfg, T, variant=v, device=cuda)
        if cfg.balanced and v == 0:  # the near-uniform load the benchmark runs (bias fitted as it does)
            logits = ops.router_logits(x, lt.router)
            lt.bias.copy_(torch.from_numpy(cf.zipf_bias(cfg, ph.to_np(logits))).to(cuda))
        residual = torch.randn(T, cfg.hidden, device=cuda)
        ids = torch.empty(T * cfg.top_k, dtype=torch.int32, device=cuda)
        w = torch.empty(T * cfg.top_k, dtype=torch.float32, device=cuda)
        out = lt.layer.forward(x, residual, ids=ids, weights=w)
        out2 = lt.layer.forward(x, residual)
        torch.cuda.synchronize()
        assert torch.equal(out, out2), (
            f"layer output is not bitwise reproducible: {(out != out2).sum().item()} of "
            f"{out.numel()} differ, NaNs {torch.isnan(out).sum().item()}/"
            f"{torch.isnan(out2).sum().item()}, first at {(out != out2).nonzero()[:4].tolist()}")
        ref, _, _, f = ph.oracle_layer_tokens(cfg, lt, x, residual, tokens,
                                              ph.to_np(ids).view(np.uint32), ph.to_np(w))
        flips += f
        res = ph.to_np(residual)[tokens]
        got_all.append(ph.to_np(out)[tokens] - res)
        ref_all.append(ref - res)
    err = rn.rel_l2(np.concatenate(got_all), np.concatenate(ref_all))
    print(f"{cfg.name} T={T} x{variants} inputs, {len(tokens)} rows each: "
          f"rel_l2(moe part)={err:.3e} near-tie tokens={flips}")
    assert err < (ph.TOL_REL_L2 if tol is None else tol)
    return err


@pytest.mark.parametrize("quant", [Q2_K, Q3_K, Q4_K])
@pytest.mark.parametrize("T", [1, 300])
def test_layer_from_gguf_file(cuda, tmp_path, T, quant):
    # a layer written to a GGUF file (packed experts [H, I, E] / [I, H, E],
    # f32 router [H, E], bias, Q8_0 shared expert), loaded through the reader
    # and run on the GPU (decode at T = 1, prefill at T = 300), against the
    # oracle run on the tensors the reader hands out (host views of the file)
    from inferno_amd import gguf as G
    cfg = cf.Config("gguf_file", 10, 1024, 16, 512, 4, (quant,), SCORE_SIGMOID, True, 2.5, 0.1,
                    512, torch.bfloat16, (T,))
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=T)
    H, E, I, Is = cfg.hidden, cfg.experts, cfg.intermediate, cfg.shared_intermediate
    sg, su, sd = lt.shared
    ts = [("blk.5.ffn_gate_inp.weight", (H, E), G.GGML_F32, ph.to_np(lt.router).tobytes()),
          ("blk.5.exp_probs_b.bias", (E,), G.GGML_F32, ph.to_np(lt.bias).tobytes()),
          ("blk.5.ffn_gate_exps.weight", (H, I, E), quant, ph.to_np(lt.gate).tobytes()),
          ("blk.5.ffn_up_exps.weight", (H, I, E), quant, ph.to_np(lt.up).tobytes()),
          ("blk.5.ffn_down_exps.weight", (I, H, E), quant, ph.to_np(lt.down).tobytes()),
          ("blk.5.ffn_gate_shexp.weight", (H, Is), Q8_0, ph.to_np(sg).tobytes()),
          ("blk.5.ffn_up_shexp.weight", (H, Is), Q8_0, ph.to_np(su).tobytes()),
          ("blk.5.ffn_down_shexp.weight", (Is, H), Q8_0, ph.to_np(sd).tobytes())]
    path = tmp_path / "layer.gguf"
    G.write_gguf(path, [("general.architecture", G.MT_STRING, "glm")], ts)
    x = cf.make_input(cfg, T, device=cuda)
    residual = torch.randn(T, H, device=cuda)
    ids = torch.empty(T * cfg.top_k, dtype=torch.int32, device=cuda)
    w = torch.empty(T * cfg.top_k, device=cuda)
    with G.GGUFFile(path) as g:
        layer = G.moe_layer_from_gguf(g, 5, top_k=cfg.top_k, score_fn=cfg.score_fn,
                                      norm_topk_prob=cfg.norm, routed_scaling_factor=cfg.scale,
                                      device=cuda, max_tokens=T)
        got = layer.forward(x, residual, ids=ids, weights=w)
        torch.cuda.synchronize()

        def host(name, dtype=torch.uint8):
            return torch.from_numpy(np.array(g.tensor_bytes(name))).view(dtype)
        from_file = SimpleNamespace(
            quant=quant, router=host("blk.5.ffn_gate_inp.weight", torch.float32).view(E, H),
            bias=host("blk.5.exp_probs_b.bias", torch.float32),
            gate=host("blk.5.ffn_gate_exps.weight"), up=host("blk.5.ffn_up_exps.weight"),
            down=host("blk.5.ffn_down_exps.weight"),
            shared=tuple(host(f"blk.5.ffn_{m}_shexp.weight") for m in ("gate", "up", "down")))
        tokens = np.arange(T) if T < 64 else np.r_[0:32, T - 32:T]
        ref, _, _, flips = ph.oracle_layer_tokens(cfg, from_file, x, residual, tokens,
                                                  ph.to_np(ids).view(np.uint32), ph.to_np(w))
    res = ph.to_np(residual)[tokens]
    err = rn.rel_l2(ph.to_np(got)[tokens] - res, ref - res)
    print(f"GGUF file layer quant={quant} T={T}: rel_l2={err:.3e} near-tie tokens={flips}")
    assert err < ph.TOL_REL_L2


@pytest.mark.parametrize("T", [100, 2085])
def test_layer_prefill_shared_ragged_tiles(cuda, T):
    # the dense Q8_0 shared-expert GEMM over T rows: 32-row tiles below 2048
    # tokens, 128-row tiles from 2048, the last tile partly filled (4 and 37
    # rows); checked on the first and the last tokens
    cfg = cf.Config("shared_ragged", 9, 1024, 16, 512, 2, (Q2_K,), SCORE_SIGMOID, True, 1.0, 0.1,
                    512, torch.bfloat16, (T,))
    _layer_parity(cuda, cfg, T, tokens=np.r_[0:24, T - 48:T])


@pytest.mark.parametrize("key,T", [("c2", 4), ("c2", 8), ("c4", 6)])
def test_layer_decode_several_tokens_shared(cuda, key, T):
    # below the grouped GEMM's 66 assignments with a Q8_0 shared expert: the
    # several-token decode launches (select, packed-f16 tiles), full size
    _layer_parity(cuda, key, T)


@pytest.mark.parametrize("T", [1, 16])
def test_layer_c1_q4k_softmax(cuda, T):
    # T = 1: 16 seeded tokens; T = 16: every token of two batches
    _layer_parity(cuda, "c1", T, variants=16 if T == 1 else 2)


def test_layer_c2_glm_q2k_decode_full_size(cuda):
    # 16 seeded tokens, one layer call each (16 routing patterns)
    _layer_parity(cuda, "c2", 1, variants=16)


# Exact ties in the one-token decode selection: a zero router makes every
# logit 0, so the selection keys are the bias tiers (sigmoid) or all equal
# (softmax, no bias); the k winners must be the oracle's (key desc, id asc),
# in rank order, with the oracle's weights. Q2_K / Q3_K take the fp8 x fp4
# gate/up (four router slots per lane; two at H = 4096 for E <= 128), Q4_K
# the run gate/up (one slot per lane for E <= 64, else four).
@pytest.mark.parametrize("score_fn", [SCORE_SIGMOID, SCORE_SOFTMAX])
@pytest.mark.parametrize("E,k,quant,H", [(64, 8, Q2_K, 1024), (256, 8, Q2_K, 1024),
                                         (256, 16, Q4_K, 1024), (64, 8, Q4_K, 1024),
                                         (128, 10, Q2_K, 4096), (128, 10, Q3_K, 4096)])
def test_layer_decode_selection_ties(cuda, score_fn, E, k, quant, H):
    cfg = cf.Config(f"ties_e{E}_k{k}_h{H}", 90 + E // 64, H, E, 512, k, (quant,), score_fn, True,
                    2.5, 0.0, 256, torch.bfloat16, (1,))
    bias = None
    if score_fn == SCORE_SIGMOID:
        tiers = np.array([0.0, 0.25, 0.5], np.float32)
        bias = torch.from_numpy(tiers[np.arange(E) % 3].copy()).to(cuda)
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=1, bias=bias)
    lt.router.zero_()
    x = cf.make_input(cfg, 1, device=cuda)
    ids = torch.empty(k, dtype=torch.int32, device=cuda)
    w = torch.empty(k, device=cuda)
    out = lt.layer.forward(x, None, ids=ids, weights=w)
    torch.cuda.synchronize()
    oid, ow = orc.router_topk(np.zeros((1, E), np.float32),
                              None if bias is None else ph.to_np(bias), k, score_fn, True, 2.5)
    got = ph.to_np(ids).view(np.uint32)
    assert np.array_equal(got, oid), (got, oid)
    np.testing.assert_allclose(ph.to_np(w), ow, rtol=2e-6, atol=0)
    assert torch.isfinite(out).all()


# One-token Q2_K bf16 layers of other shapes: the MFMA gate/up at 4, 8 and 12
# super-block columns, the MFMA down (I = 2048) with 4 ranks, the tile-kernel
# down after the MFMA gate/up (I != 2048), with and without a shared expert.
@pytest.mark.parametrize("H,E,I,k,Is", [(1024, 16, 2048, 4, 256), (2048, 32, 512, 8, 0),
                                        (3072, 16, 1024, 6, 512)])
def test_layer_q2k_decode_mfma_shapes(cuda, H, E, I, k, Is):
    cfg = cf.Config(f"q2k_decode_h{H}_e{E}_i{I}_k{k}_s{Is}", 20 + H // 1024, H, E, I, k,
                    (cf.Q2_K,), cf.SCORE_SIGMOID, True, 2.5, 0.1, Is, torch.bfloat16, (1,))
    _layer_parity(cuda, cfg, 1)


# One-token layers on the f16-run matrix-core kernels (gate/up and down) for
# every routed format: bf16 tokens, 3 to 8 down columns, 4 to 16 ranks, with
# and without a shared expert. Q2_K keeps the fp8 x fp4 gate/up and takes the
# run down, as does Q3_K when its rows are whole 16-byte chunks (H a multiple
# of 2048); fp32 tokens take the grouped run gate/up with two f16 terms.
@pytest.mark.parametrize("quant", [Q2_K, Q3_K, Q4_K])
@pytest.mark.parametrize("H,E,I,k,Is,dt", [(2048, 64, 768, 8, 0, torch.float32),
                                           (4096, 128, 1536, 10, 1536, torch.bfloat16),
                                           (1024, 32, 1024, 16, 256, torch.bfloat16),
                                           (3072, 16, 2048, 4, 512, torch.bfloat16),
                                           (2048, 64, 768, 8, 0, torch.bfloat16),
                                           (3072, 16, 2048, 4, 512, torch.float32)])
def test_layer_runs_decode_shapes(cuda, quant, H, E, I, k, Is, dt):
    cfg = cf.Config(f"runs_decode_q{quant}_h{H}_i{I}_k{k}_s{Is}", 40 + H // 1024 + quant, H, E, I,
                    k, (quant,), cf.SCORE_SOFTMAX if k == 10 else cf.SCORE_SIGMOID, True, 2.5,
                    0.0 if k == 10 else 0.1, Is, dt, (1,))
    _layer_parity(cuda, cfg, 1, variants=4)
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=1)
    ops.kernel_timing(True)
    try:
        lt.layer.forward(cf.make_input(cfg, 1, device=cuda), None)
        torch.cuda.synchronize()
        gu = ops.kernel_timing_label(ops.TIMER_GATE_UP)
        dn = ops.kernel_timing_label(ops.TIMER_DOWN)
    finally:
        ops.kernel_timing(False)
    if dt == torch.float32:  # two f16 terms per run on the grouped run gate/up
        # which selects itself when no shared expert needs the select launch
        assert gu.startswith("runs32+select:" if Is == 0 else "runs32:"), gu
        assert dn.startswith("runs-down:"), dn
        return
    if quant == Q2_K or (quant == Q3_K and (H // 256) % 8 == 0):
        assert gu.startswith("mfma"), gu  # the fp8 x fp4 gate/up (with or without the selection)
    else:
        assert gu.startswith("runs:"), gu
    assert dn.startswith("runs-down:") or dn.startswith("mfma-down:"), dn


# Several-token decode layers (T > 1, below the grouped GEMM's threshold, no shared
# expert) on the f16-run matrix-core kernels grouped by expert: every routed
# format, bf16 and fp32 tokens (the two-term f16 runs), and loads from ~2 to
# ~30 tokens per expert (the latter past the kernels' per-pass token count, so
# an expert's tiles run in several token chunks).
@pytest.mark.parametrize("quant,H,E,I,k,T,dt", [
    (Q4_K, 2048, 64, 768, 8, 16, torch.float32),     # c1 at T = 16
    (Q2_K, 4096, 128, 1536, 10, 16, torch.bfloat16),  # Laguna-S shape, 160 assignments
    (Q3_K, 3072, 16, 2048, 4, 32, torch.bfloat16),    # ~8 tokens per expert
    (Q4_K, 1024, 4, 768, 2, 60, torch.float32),       # ~30 tokens per expert
    (Q2_K, 1024, 4, 1024, 2, 60, torch.bfloat16),
    (Q3_K, 2048, 8, 768, 3, 40, torch.float32),
    (Q2_K, 6144, 256, 2048, 8, 16, torch.bfloat16)])  # GLM shape without the shared expert
def test_layer_runs_multi_decode(cuda, switches, quant, H, E, I, k, T, dt):
    # the grouped GEMM takes these loads by default; the threshold raised
    # keeps them on the several-token decode kernels under test
    switches(INFERNO_PREFILL_MIN_ASSIGNMENTS="100000")
    cfg = cf.Config(f"runs_multi_q{quant}_h{H}_e{E}_i{I}_k{k}_t{T}", 70 + H // 1024 + quant, H, E,
                    I, k, (quant,), cf.SCORE_SOFTMAX if k == 10 else cf.SCORE_SIGMOID, True, 2.5,
                    0.0 if k == 10 else 0.1, 0, dt, (T,))
    _layer_parity(cuda, cfg, T, variants=2)
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=T)
    ops.kernel_timing(True)
    try:
        lt.layer.forward(cf.make_input(cfg, T, device=cuda), None)
        torch.cuda.synchronize()
        gu = ops.kernel_timing_label(ops.TIMER_GATE_UP)
        dn = ops.kernel_timing_label(ops.TIMER_DOWN)
    finally:
        ops.kernel_timing(False)
    assert gu.startswith("runs-multi:"), gu
    assert dn.startswith("runs-multi-down:"), dn


# Laguna XS layer formats (crates/model/src/laguna/gguf_model.rs:808-860,
# laguna_xs_gguf_moe_shared_device backend.rs:1754): routed Q4_K gate/up with
# Q4_K or Q6_K down, shared expert Q4_K gate/up with the routed down format,
# at c1's shape (H 2048, 64 experts, I 768, top-8 softmax, fp32 tokens),
# one token (16 seeded inputs), 16 tokens, and 64 tokens (512 assignments:
# the grouped GEMM path). Shared width 768 is the XS layer's own (the shared
# expert as the token's ninth assignment, laguna_xs.rs:1001-1144): one token
# runs it as assignment k of the run kernels, asserted below; 1024 (another
# width) keeps the shared expert on its own kernels.
@pytest.mark.parametrize("Is", [768, 1024])
@pytest.mark.parametrize("down", [Q4_K, Q6_K])
@pytest.mark.parametrize("T", [1, 16, 64])
def test_layer_laguna_xs_q4k_shared(cuda, down, T, Is):
    c1 = cf.CONFIGS["c1"]
    cfg = cf.Config(f"xs_q4k_down{down}_s{Is}", 60 + down, c1.hidden, c1.experts,
                    c1.intermediate, c1.top_k, (Q4_K,), c1.score_fn, True, 1.0, 0.0, Is,
                    torch.float32, (T,), down_quant=down, shared_quant=Q4_K)
    _layer_parity(cuda, cfg, T, variants=16 if T == 1 else 1)
    if T == 64:  # the grouped GEMMs, Q6_K down included, and the dense shared GEMMs
        lt = cf.build_layer(cfg, 0, cuda, max_tokens=T)
        ops.kernel_timing(True)
        try:
            lt.layer.forward(cf.make_input(cfg, T, device=cuda), None)
            torch.cuda.synchronize()
            assert ops.kernel_timing_label(ops.TIMER_GATE_UP).startswith("prefill:")
            assert ops.kernel_timing_label(ops.TIMER_DOWN).startswith("prefill:")
        finally:
            ops.kernel_timing(False)
    if T != 1:
        return
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=1)
    ops.kernel_timing(True)
    try:
        lt.layer.forward(cf.make_input(cfg, 1, device=cuda), None)
        torch.cuda.synchronize()
        gu = ops.kernel_timing_label(ops.TIMER_GATE_UP)
        dn = ops.kernel_timing_label(ops.TIMER_DOWN)
    finally:
        ops.kernel_timing(False)
    if Is == c1.intermediate:
        assert gu.startswith("runs+shared+select:"), gu
        assert dn.startswith("runs-down+shared:"), dn
    else:
        assert gu.startswith("stage:"), gu


# The shared expert as assignment k of the one-token run kernels for every
# routed gate/up format and every down format, bf16 and fp32 tokens, k up to
# 16 (the slot table's last entry), against the oracle.
@pytest.mark.parametrize("quant,down,H,E,I,k,dt", [
    (Q4_K, Q6_K, 2048, 256, 512, 8, torch.bfloat16),
    (Q2_K, Q2_K, 4096, 128, 1536, 10, torch.bfloat16),
    (Q3_K, Q6_K, 2048, 64, 1024, 16, torch.float32),
    (Q4_K, Q4_K, 3072, 32, 2048, 4, torch.float32)])
def test_layer_decode_shared_slot_shapes(cuda, quant, down, H, E, I, k, dt):
    cfg = cf.Config(f"shared_slot_q{quant}_d{down}_h{H}_i{I}_k{k}", 80 + quant + down, H, E, I, k,
                    (quant,), cf.SCORE_SIGMOID, True, 2.5, 0.1, I, dt, (1,), down_quant=down,
                    shared_quant=quant)
    _layer_parity(cuda, cfg, 1, variants=4)
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=1)
    ops.kernel_timing(True)
    try:
        lt.layer.forward(cf.make_input(cfg, 1, device=cuda), None)
        torch.cuda.synchronize()
        gu = ops.kernel_timing_label(ops.TIMER_GATE_UP)
        dn = ops.kernel_timing_label(ops.TIMER_DOWN)
    finally:
        ops.kernel_timing(False)
    assert gu.startswith("runs+shared+select:"), gu
    assert dn.startswith("runs-down+shared:"), dn


def test_layer_c3_glm_q3k_prefill_all_tokens(cuda):
    # every one of the 512 tokens, near-uniform expert load (~16 per expert)
    _layer_parity(cuda, "c3", 512)


def c5_check_tokens(ids, T, k, E):
    """Tokens whose rows the c5 test checks: every token of the hottest
    expert (its full 128-row tiles), every token of one expert per partial
    tile class (last tile of 97-128, 65-96, 33-64 and 1-32 rows), the first
    and the last tokens, topped up with evenly spaced ones to 256 or more."""
    ids = np.asarray(ids).reshape(T, k)
    load = np.bincount(ids.reshape(-1).astype(np.int64), minlength=E)
    chosen = {int(np.argmax(load))}
    classes = {}
    for e in np.argsort(-load, kind="stable"):
        n = int(load[e])
        if n == 0 or int(e) in chosen:
            continue
        rem = n % 128 or 128
        cls = (rem - 1) // 32
        if cls not in classes and n < 128 * 4:
            classes[cls] = int(e)
    chosen |= set(classes.values())
    rows = set(np.nonzero(np.isin(ids, list(chosen)).any(axis=1))[0].tolist())
    rows |= {0, T - 1}
    step = max(1, T // 256)
    for t in range(0, T, step):
        if len(rows) >= 256:
            break
        rows.add(t)
    return np.array(sorted(rows)), load, sorted(classes)


@pytest.mark.parametrize("variant", ["default", "wide"])
def test_layer_c5_glm_q2k_prefill_zipf(cuda, switches, variant):
    # full-size skewed prefill: router bias fitted so the load follows
    # Zipf(1.1) over 216 experts (hottest capped at one slot per token,
    # 12.5%), 40 experts without a token. "wide": the Q2_K GEMMs on their
    # larger-workgroup kernels (INFERNO_PREFILL_Q2_SMALL_WG=0,
    # INFERNO_PREFILL_G128_WIDE=1), against the same oracle bound
    if variant == "wide":
        switches(INFERNO_PREFILL_Q2_SMALL_WG="0", INFERNO_PREFILL_G128_WIDE="1")
    cfg = cf.CONFIGS["c5"]
    T, k, E = 4096, cfg.top_k, cfg.experts
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=T)
    x = cf.make_input(cfg, T, device=cuda)
    logits = ops.router_logits(x, lt.router)
    lt.bias.copy_(torch.from_numpy(cf.zipf_bias(cfg, ph.to_np(logits))).to(cuda))
    residual = torch.randn(T, cfg.hidden, device=cuda)
    ids = torch.empty(T * k, dtype=torch.int32, device=cuda)
    w = torch.empty(T * k, dtype=torch.float32, device=cuda)
    out = lt.layer.forward(x, residual, ids=ids, weights=w)
    out2 = lt.layer.forward(x, residual)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "layer output is not bitwise reproducible"
    ids_np = ph.to_np(ids).view(np.uint32)
    tokens, load, classes = c5_check_tokens(ids_np, T, k, E)
    share = load.max() / (T * k)
    print(f"c5 load: hottest share {share:.4f}, empty experts {(load == 0).sum()}, "
          f"partial tile classes covered {classes}, rows checked {len(tokens)}")
    assert share >= 0.12 and 36 <= (load == 0).sum() <= 44
    assert len(tokens) >= 256 and len(classes) == 4
    ref, _, _, flips = ph.oracle_layer_tokens(cfg, lt, x, residual, tokens, ids_np, ph.to_np(w))
    res = ph.to_np(residual)[tokens]
    err = rn.rel_l2(ph.to_np(out)[tokens] - res, ref - res)
    print(f"c5 T={T}: rel_l2(moe part)={err:.3e} near-tie tokens={flips}")
    assert err < ph.TOL_REL_L2


@pytest.mark.parametrize("T", [1, 32])
def test_stack_c4_laguna_q2k_q3k_rmsnorm_chain(cuda, T):
    """c4 end to end: layers 0-1 Q2_K, 2-3 Q3_K (top-10 softmax, Q8_0 shared
    expert), RMSNorm (eps 1e-6) before every layer, bf16 activations, one
    residual stream, against the oracle chain run from the same input.
    T = 1: 16 seeded tokens, one stack call each; T = 32: every token.
    Tokens whose expert set differs from the oracle chain's within the drift
    bound of the k-th selection value (sum_h |W_r| |a_gpu - a_oracle|, from
    the GPU's own stream entering the layer: the chain's inputs drift apart
    by rounding) are counted and left out of the error; any other set
    difference fails.

    Tolerance: each layer is held to the north_star's 2e-3 by
    test_stack_c4_each_layer_on_gpu_stream (same input on both sides). Along
    a chain the two sides' residual streams drift apart, and each RMSNorm
    re-rounds them to bf16, so per-layer errors compound: the chain is held
    to n_layers * 2e-3 (measured 2.5e-3 over 16 tokens)."""
    cfg = cf.CONFIGS["c4"]
    k = cfg.top_k
    lts, stack = cf.build_stack(cfg, cuda, max_tokens=T)
    prefixes = [ops.MoEStack([lt.layer for lt in lts[:l]], [lt.norm_w for lt in lts[:l]],
                             eps=cfg.rms_eps, act_dtype=cfg.x_dtype, max_tokens=T)
                for l in range(1, cfg.layers)]
    variants = range(16) if T == 1 else [0]
    got_all, ref_all, r0_all = [], [], []
    n_tie = [0] * cfg.layers
    for v in variants:
        hidden = cf.make_hidden(cfg, T, variant=v, device=cuda)
        ids = torch.empty(cfg.layers * T * k, dtype=torch.int32, device=cuda)
        out = stack.forward(hidden, ids=ids)
        out2 = stack.forward(hidden)
        streams = [hidden] + [pre.forward(hidden) for pre in prefixes]
        torch.cuda.synchronize()
        assert torch.equal(out, out2), "stack output is not bitwise reproducible"
        tokens = np.arange(T)
        ref, ties = ph.oracle_stack_tokens(cfg, lts, hidden, tokens, ph.to_np(ids).view(np.uint32),
                                           gpu_streams=streams)
        drop = set(t for tl in ties for t in tl)
        keep = np.array([t for t in tokens if t not in drop], dtype=np.int64)
        n_tie = [a + len(b) for a, b in zip(n_tie, ties)]
        r0 = ph.to_np(hidden)
        got_all.append(ph.to_np(out)[keep])
        ref_all.append(ref[keep])
        r0_all.append(r0[keep])
    got, ref, r0 = (np.concatenate(a) for a in (got_all, ref_all, r0_all))
    checked = got.shape[0]
    # the stack's own contribution (four MoE blocks), input stream removed
    err = rn.rel_l2(got - r0, ref - r0)
    print(f"c4 stack chain T={T} x{len(variants)}: rel_l2={err:.3e} over {checked} tokens; "
          f"chain near-tie tokens (expert set changed) per layer={n_tie}")
    assert checked >= (12 if T == 1 else 24)
    assert err < cfg.layers * ph.TOL_REL_L2


@pytest.mark.parametrize("T", [1, 32])
def test_stack_c4_fused_norm_router_variant(cuda, monkeypatch, T):
    """Each c4 layer as a one-layer stack with INFERNO_STACK_FUSED_ROUTER=1
    (RMSNorm and router logits in one launch before a decode layer) against
    the default: the normalised rows are bit-identical and the logits are
    summed in another order, so the same experts except near-ties, and the
    same output within 1e-5 rel-L2 on tokens whose routing agrees (measured
    5.9e-6 over 16 tokens: an f16 rounding of h or a bf16 rounding flipped
    here and there). Along a whole stack the bf16 re-rounding of every RMSNorm
    amplifies such last-bit differences, as it does between the GPU and the
    oracle chain, so the layers are compared one at a time. T = 32 takes the
    prefill path, where the variant does not apply: identical bits."""
    cfg = cf.CONFIGS["c4"]
    k = cfg.top_k
    lts, _ = cf.build_stack(cfg, cuda, max_tokens=T)
    got, ref, same, total = [], [], 0, 0
    for l, lt in enumerate(lts):
        stack = ops.MoEStack([lt.layer], [lt.norm_w], eps=cfg.rms_eps, act_dtype=cfg.x_dtype,
                             max_tokens=T)
        for v in range(4 if T == 1 else 1):
            hidden = cf.make_hidden(cfg, T, variant=10 * l + v, device=cuda)
            ids0 = torch.empty(T * k, dtype=torch.int32, device=cuda)
            ids1 = torch.empty_like(ids0)
            out0 = stack.forward(hidden, ids=ids0)
            monkeypatch.setenv("INFERNO_STACK_FUSED_ROUTER", "1")
            out1 = stack.forward(hidden, ids=ids1)
            out1b = stack.forward(hidden)
            monkeypatch.delenv("INFERNO_STACK_FUSED_ROUTER")
            torch.cuda.synchronize()
            assert torch.equal(out1, out1b), "fused variant not bitwise reproducible"
            if T > 1:
                assert torch.equal(out0, out1) and torch.equal(ids0, ids1)
                continue
            total += 1
            if np.array_equal(np.sort(ph.to_np(ids0)), np.sort(ph.to_np(ids1))):
                same += 1
                got.append(ph.to_np(out1)[0] - ph.to_np(hidden)[0])
                ref.append(ph.to_np(out0)[0] - ph.to_np(hidden)[0])
    if T == 1:
        assert same >= total - 2
        err = rn.rel_l2(np.stack(got), np.stack(ref))
        print(f"c4 fused norm+router, layer by layer: {same}/{total} tokens same routing, "
              f"rel_l2={err:.2e}")
        assert err < 1e-5


@pytest.mark.parametrize("T", [1, 32])
def test_stack_c4_each_layer_on_gpu_stream(cuda, T):
    """c4 layer by layer: the GPU stream entering layer l (output of the
    stack's first l layers) is normalised by the library's RMSNorm (the fp32
    kernel the stack runs, rounded to bf16 on the host: the same nearest-even
    rounding, so bit-identical activations), then run through the oracle's
    layer l; the result must match the GPU's first l+1 layers within the
    north_star's 2e-3, routing exact up to 1e-6 near-ties. (The oracle's
    own RMSNorm sums in another order, so a bf16 activation can round the
    other way; it is checked on its own and in the chain test.)"""
    cfg = cf.CONFIGS["c4"]
    k = cfg.top_k
    lts, _ = cf.build_stack(cfg, cuda, max_tokens=T)
    prefixes = [ops.MoEStack([lt.layer for lt in lts[:l + 1]], [lt.norm_w for lt in lts[:l + 1]],
                             eps=cfg.rms_eps, act_dtype=cfg.x_dtype, max_tokens=T)
                for l in range(cfg.layers)]
    variants = range(16) if T == 1 else [1]
    for v in variants:
        hidden = cf.make_hidden(cfg, T, variant=v, device=cuda)
        r = hidden
        for l, (lt, pre) in enumerate(zip(lts, prefixes)):
            ids = torch.empty((l + 1) * T * k, dtype=torch.int32, device=cuda)
            nxt = pre.forward(hidden, ids=ids)
            torch.cuda.synchronize()
            rows = np.arange(T)
            r_np = ph.to_np(r)
            a = ph.to_np(ops.rms_norm(r, lt.norm_w, cfg.rms_eps))
            if cfg.x_dtype == torch.bfloat16:
                a = ph.bf16_round(a)
            g_ids = ph.to_np(ids).view(np.uint32)[l * T * k:]
            ref, _, _, flips = ph.oracle_layer_rows(cfg, lt, a, r_np, g_ids)
            err = rn.rel_l2(ph.to_np(nxt)[rows] - r_np, ref - r_np)
            print(f"c4 layer {l} ({'Q2_K' if lt.quant == Q2_K else 'Q3_K'}) T={T} v{v}: "
                  f"rel_l2={err:.3e} near-tie tokens={flips}")
            assert err < ph.TOL_REL_L2
            r = nxt


@pytest.fixture
def switches(monkeypatch):
    """Sets kernel-variant switches for one test (the library reads them on
    every call); monkeypatch restores the environment afterwards."""
    def set_(**kv):
        for k, v in kv.items():
            monkeypatch.setenv(k, v)
    return set_


def test_layer_prefill_fragment_kernel_variant(cuda, switches):
    """The prefill GEMMs all on the fragment-load kernel and the fp32 router
    logits (INFERNO_PREFILL_GEMM2=0, INFERNO_ROUTER_BF16X3=0): c3, every
    token, against the oracle."""
    switches(INFERNO_PREFILL_GEMM2="0", INFERNO_ROUTER_BF16X3="0")
    _layer_parity(cuda, "c3", 512)


@pytest.mark.parametrize("key", ["c2", "c4"])
def test_layer_decode_tile_kernel_variant(cuda, switches, key):
    """One-token Q2_K decode on the packed-f16 tile kernels
    (INFERNO_DECODE_MFMA=0) instead of the matrix-core kernels: c2 and c4
    layer 0, eight seeded tokens, against the oracle; the launch label
    confirms which gate/up kernel ran."""
    switches(INFERNO_DECODE_MFMA="0")
    _layer_parity(cuda, key, 1, variants=8)
    cfg = cf.CONFIGS[key]
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=1)
    ops.kernel_timing(True)
    try:
        lt.layer.forward(cf.make_input(cfg, 1, device=cuda), None)
        torch.cuda.synchronize()
        label = ops.kernel_timing_label(ops.TIMER_GATE_UP)
        ops.kernel_timing_read(ops.TIMER_GATE_UP)
    finally:
        ops.kernel_timing(False)
    assert label.startswith("tiles:"), label


def _labels_of_one_step(cfg, cuda, T=1):
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=T)
    ops.kernel_timing(True)
    try:
        lt.layer.forward(cf.make_input(cfg, T, device=cuda), None)
        torch.cuda.synchronize()
        timers = (ops.TIMER_ROUTE, ops.TIMER_SELECT, ops.TIMER_GATE_UP, ops.TIMER_DOWN)
        labels = {tm: ops.kernel_timing_label(tm) for tm in timers}
        counts = {tm: ops.kernel_timing_read(tm)[1] for tm in timers}
    finally:
        ops.kernel_timing(False)
    return labels, counts


_E128_FP32 = cf.Config("q4k_h2048_e128_fp32_q8shared", 91, 2048, 128, 768, 8, (Q4_K,),
                       cf.SCORE_SIGMOID, True, 2.5, 0.1, 1024, torch.float32, (24,))


@pytest.mark.parametrize("key,T", [("c1", 16), ("xs", 64), ("c1", 300), (_E128_FP32, 24),
                                   ("c2", 16), ("c4", 32)])
def test_layer_prefill_router_x16_variant(cuda, switches, key, T):
    """fp32 and bf16 tokens on the grouped GEMMs with the router logits over K chunks:
    the logits launch also writes x in f16 for the GEMMs (no conversion
    launch); INFERNO_ROUTER_X16=0 keeps the conversion launch. Same f16
    rounding of the same values: outputs bit-identical; the default agrees
    with the oracle."""
    cfg = cf.CONFIGS[key] if isinstance(key, str) else key  # E 128: two expert groups
    _layer_parity(cuda, cfg, T, tokens=None if T <= 64 else np.arange(0, T, 7))
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=T)
    x = cf.make_input(cfg, T, variant=2, device=cuda)
    residual = torch.randn(T, cfg.hidden, device=cuda)
    outs = []
    for flag in ("1", "0"):
        switches(INFERNO_ROUTER_X16=flag)
        outs.append(lt.layer.forward(x, residual))
        torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


# The router caps (256 experts, top-16, the reference's limits,
# metal/moe.rs:618-623, moe_kernels.metal:131) on a small layer: one token,
# a few tokens (the decode launches) and 64 tokens (1024 assignments: the
# grouped GEMM, ~4 rows per expert), Q2_K with a Q8_0 shared expert, bf16
# and fp32 tokens, against the oracle.
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T", [1, 4, 64])
def test_layer_router_caps(cuda, T, dt):
    cfg = cf.Config(f"caps_e256_k16_t{T}", 95, 512, 256, 256, 16, (Q2_K,), cf.SCORE_SIGMOID, True,
                    2.5, 0.1, 256, dt, (T,))
    _layer_parity(cuda, cfg, T, variants=2)


@pytest.mark.parametrize("runs", [True, False])
def test_layer_c1_fp32_token_kernels(cuda, switches, runs):
    """One fp32 token (c1): the f16 run kernels with two f16 terms per run
    (default) or the packed-f16 tile kernels (INFERNO_DECODE_RUNS_F32=0); 16
    seeded tokens against the oracle; the launch labels confirm which ran."""
    if not runs:
        switches(INFERNO_DECODE_RUNS_F32="0")
    _layer_parity(cuda, "c1", 1, variants=16)
    labels, counts = _labels_of_one_step(cf.CONFIGS["c1"], cuda)
    # the grouped run gate/up selects itself (no select launch)
    assert counts == {ops.TIMER_ROUTE: 1, ops.TIMER_SELECT: 0 if runs else 1,
                      ops.TIMER_GATE_UP: 1, ops.TIMER_DOWN: 1}, counts
    want = ("runs32+select:", "runs-down:") if runs else ("tiles:", "down8:")
    assert labels[ops.TIMER_GATE_UP].startswith(want[0]), labels[ops.TIMER_GATE_UP]
    assert labels[ops.TIMER_DOWN].startswith(want[1]), labels[ops.TIMER_DOWN]


@pytest.mark.parametrize("key", ["c2", "c4", "c1"])
def test_layer_decode_select_launch_variant(cuda, switches, key):
    """INFERNO_DECODE_SEL=0 keeps the separate select launch (top-k, dispatch
    and the shared down in their own launch) on the one-token fp8 x fp4 path
    (c2, c4 layer 2) and the one-fp32-token grouped run path (c1): same
    oracle bound, and the same ids and weights as the default path, whose
    gate/up launch selects; the launch labels say which ran."""
    cfg = cf.CONFIGS[key]
    lt = cf.build_layer(cfg, 2 if key == "c4" else 0, cuda, max_tokens=1)
    x = cf.make_input(cfg, 1, device=cuda)
    got = {}
    for sel in ("1", "0"):
        switches(INFERNO_DECODE_SEL=sel)
        ids = torch.empty(cfg.top_k, dtype=torch.int32, device=cuda)
        w = torch.empty(cfg.top_k, device=cuda)
        out = lt.layer.forward(x, None, ids=ids, weights=w)
        torch.cuda.synchronize()
        got[sel] = (ph.to_np(ids).copy(), ph.to_np(w).copy(), ph.to_np(out).copy())
        labels, counts = _labels_of_one_step(cfg, cuda)
        kind = "runs32" if key == "c1" else "mfma"
        assert labels[ops.TIMER_GATE_UP].startswith(kind + ("+select:" if sel == "1" else ":"))
        assert counts[ops.TIMER_SELECT] == (0 if sel == "1" else 1), counts
    assert np.array_equal(got["1"][0], got["0"][0])
    assert np.array_equal(got["1"][1], got["0"][1])
    err = rn.rel_l2(got["1"][2], got["0"][2])
    print(f"{key}: select in gate/up vs select launch rel_l2={err:.3e}")
    assert err < 1e-5  # only the shared down's summation order differs
    switches(INFERNO_DECODE_SEL="0")
    _layer_parity(cuda, cfg, 1, variants=4)


@pytest.mark.parametrize("sel", ["1", "0"])
def test_layer_decode_shared_expert_alone(cuda, switches, sel):
    """c2's shape with the routed part scaled to zero (routing scale 0): the
    output is the residual plus the Q8_0 shared expert alone, so its decode
    path is checked without the routed experts' error. Its gate/up runs in
    the route launch (K parts); its down in the selecting gate/up launch
    (default) or the select launch (INFERNO_DECODE_SEL=0), both against h
    staged as f16 runs with a power-of-two scale per 16 values: ~2^-12
    relative per value, measured ~4e-4 rel-L2 on this part, bound 1e-3."""
    switches(INFERNO_DECODE_SEL=sel)
    cfg = dataclasses.replace(cf.CONFIGS["c2"], name="c2_shared_alone", scale=0.0)
    labels, _ = _labels_of_one_step(cfg, cuda)
    want = "mfma+select:" if sel == "1" else "mfma:"
    assert labels[ops.TIMER_GATE_UP].startswith(want), labels[ops.TIMER_GATE_UP]
    _layer_parity(cuda, cfg, 1, variants=4, tol=1e-3)


@pytest.mark.parametrize("key,T", [("c3", 512), ("c3", 2048), ("c5", 4096)])
def test_layer_prefill_router_blas(cuda, switches, key, T):
    """bf16 tokens of a large batch (512 and up): router logits as one bf16
    library GEMM over the exact three-term split of the fp32 router (fp32
    accumulation; the three terms' results added in order), against the
    matrix-core logits kernel
    (INFERNO_ROUTER_BLAS=0): the selected ids agree except on near-ties of
    the fp64 scores (gap below 1e-5 of the k-th score), the routing weights
    within 1e-5, and the layer agrees with the oracle."""
    cfg = cf.CONFIGS[key]
    _layer_parity(cuda, cfg, T, tokens=np.arange(0, T, 32))
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=T)
    x = cf.make_input(cfg, T, variant=1, device=cuda)
    k = cfg.top_k
    res = []
    for flag in ("1", "0"):
        switches(INFERNO_ROUTER_BLAS=flag)
        ids = torch.empty(T * k, dtype=torch.int32, device=cuda)
        w = torch.empty(T * k, dtype=torch.float32, device=cuda)
        lt.layer.forward(x, None, ids=ids, weights=w)
        torch.cuda.synchronize()
        res.append((ph.to_np(ids).reshape(T, k), ph.to_np(w).reshape(T, k)))
    (ia, wa), (ib, wb) = res
    bad = np.nonzero((ia != ib).any(axis=1))[0]
    if len(bad):
        lg = ph.x_f32(x)[bad].astype(np.float64) @ ph.to_np(lt.router).astype(np.float64).T
        sc = 1.0 / (1.0 + np.exp(-lg)) + ph.to_np(lt.bias).astype(np.float64)[None, :]
        srt = np.sort(sc, axis=1)
        gaps = srt[:, -k] - srt[:, -k - 1]
        assert np.all(gaps < 1e-5 * np.abs(srt[:, -k])), gaps
    good = np.setdiff1d(np.arange(T), bad)
    np.testing.assert_allclose(wa[good], wb[good], rtol=1e-5, atol=1e-7)
    print(f"{key} T={T}: tokens with other ids {len(bad)}")


@pytest.mark.parametrize("blas", ["1", "0"])
@pytest.mark.parametrize("key,T", [("c3", 512), ("c4", 300), ("e128_fp32", 300), ("c4", 32),
                                   ("c2", 12)])
def test_layer_prefill_shared_expert_alone(cuda, switches, blas, key, T):
    """The Q8_0 shared expert of a grouped-GEMM batch alone (routing scale
    0): on the library GEMMs (default: the blocks expanded to f16, fp32
    accumulation, h in f16) or on the grouped kernels' dense
    path (INFERNO_SHARED_BLAS=0); every 4th token against the oracle. Both
    round x and h to f16 as the reference prefill does: bound 2e-3."""
    switches(INFERNO_SHARED_BLAS=blas)
    base = _E128_FP32 if key == "e128_fp32" else cf.CONFIGS[key]  # fp32 tokens: x16 from the router
    cfg = dataclasses.replace(base, name=f"{key}_shared_alone", scale=0.0, balanced=False, zipf=0.0)
    _layer_parity(cuda, cfg, T, tokens=np.arange(0, T, 4))


@pytest.mark.parametrize("key", ["c2", "c4", "c1", "xs", "small", "small_noshared"])
def test_layer_decode_warm_down_has_no_effect_on_results(cuda, switches, key):
    """The selecting gate/up launch warms L2 with the down launch's first
    tiles under its last routed tile (loads into its free tile registers,
    never used): the outputs must be bitwise those of
    INFERNO_DECODE_WARM_DOWN=0, on c2 (Q2_K MFMA down), c4 layer 2 (Q3_K run
    down), c1 (Q4_K run gate/up and down), XS (the shared expert as rank k
    of the Q6_K run down) and a 1024-wide layer with and without a shared
    expert."""
    if key.startswith("small"):
        cfg = cf.Config("warm_" + key, 27, 1024, 16, 2048, 4, (cf.Q2_K,), cf.SCORE_SIGMOID,
                        True, 2.5, 0.1, 0 if key.endswith("noshared") else 256, torch.bfloat16, (1,))
    else:
        cfg = cf.CONFIGS[key]
    lt = cf.build_layer(cfg, 2 if key == "c4" else 0, cuda, max_tokens=1)
    inputs = [(cf.make_input(cfg, 1, variant=v, device=cuda), torch.randn(1, cfg.hidden, device=cuda))
              for v in range(3)]
    got = {}
    for warm in ("1", "0"):
        switches(INFERNO_DECODE_WARM_DOWN=warm)
        outs = []
        for x, residual in inputs:
            outs.append(ph.to_np(lt.layer.forward(x, residual)).copy())
        torch.cuda.synchronize()
        got[warm] = outs
    for a, b in zip(got["1"], got["0"]):
        assert np.isfinite(a).all()
        assert np.array_equal(a, b)
    if key not in ("c4", "c1", "xs"):  # the fp8 x fp4 kernels (c4's layer 2: its label tests)
        labels, _ = _labels_of_one_step(cfg, cuda)
        assert labels[ops.TIMER_GATE_UP].startswith("mfma+select:")


def test_kernel_timing_hook_counts_decode_launches(cuda):
    """The measurement hook: events recorded around each timed launch without
    waiting, summed when read; two decode steps give two launches per timer,
    positive times and a label naming the kernel."""
    cfg = cf.CONFIGS["c2"]
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=1)
    x = cf.make_input(cfg, 1, device=cuda)
    timers = [ops.TIMER_GATE_UP, ops.TIMER_DOWN, ops.TIMER_ROUTE, ops.TIMER_SELECT]
    ops.kernel_timing(True)
    try:
        for tm in timers:
            ops.kernel_timing_read(tm)
        lt.layer.forward(x, None)
        lt.layer.forward(x, None)
        got = {tm: ops.kernel_timing_read(tm) for tm in timers}
        labels = {tm: ops.kernel_timing_label(tm) for tm in timers}
    finally:
        ops.kernel_timing(False)
    # one token on the fp8 x fp4 gate/up: the selection runs in the gate/up
    # launch and the select launch is skipped
    assert labels[ops.TIMER_GATE_UP].startswith("mfma+select:"), labels[ops.TIMER_GATE_UP]
    for tm in timers:
        ms, n = got[tm]
        if tm == ops.TIMER_SELECT:
            assert n == 0, (tm, ms, n)
            continue
        assert n == 2 and ms > 0, (tm, ms, n)
        assert ":" in labels[tm]
    assert ops.kernel_timing_read(ops.TIMER_GATE_UP)[1] == 0  # read resets
