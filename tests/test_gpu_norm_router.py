"""GPU parity of the fused RMSNorm -> router logits -> top-k launch
(inferno_rms_norm_router_topk) against the RMSNorm launch and the CPU oracle.

Bars: the normalised row is bit-identical to inferno_rms_norm's (the same
device code, rounded to the activation type afterwards); logits within
2e-6 * sum|x w| of fp64 on the oracle's normalised row; the top-k is the
oracle's top-k of the GPU's own logits exactly (ids and rank order;
weights rtol 2e-6), so routing is checked apart from logit rounding; and
the ids of the oracle's own logits agree except near-ties within 1e-6 of
the k-th selection value (counted). Repeated calls reuse the ticket
workspace, so every case runs three times (the second and third with other
token counts) and must give identical bits each time.
"""
import numpy as np
import pytest
import torch

import oracle_lib as orc
import parity_helpers as ph
from inferno_amd import ops
from inferno_amd._lib import SCORE_SIGMOID, SCORE_SOFTMAX

pytestmark = pytest.mark.gpu


def _logit_bound(xn, router):
    return 2e-6 * (np.abs(xn.astype(np.float64)) @ np.abs(router.astype(np.float64)).T) + 1e-30


def test_reference_fused_norm_router_case(cuda):
    # fused_decode_rms_norm_router_matches_separate_kernels
    # (crates/backend/src/metal/laguna_xs.rs:2357-2420): H 2048, E 256, eps
    # 1e-6, input (i % 37 - 18) / 23, norm weight 0.5 + (i % 29) / 31, router
    # ((i % 43) - 21) / 1024; fused normalised row and logits against the
    # separate RMSNorm and router launches
    H, E, eps = 2048, 256, 1e-6
    i = np.arange(H)
    x = ((i % 37) - 18.0) / 23.0
    nw = 0.5 + (i % 29) / 31.0
    r = ((np.arange(E * H) % 43) - 21.0) / 1024.0
    x, nw, r = (torch.tensor(a, dtype=torch.float32, device=cuda) for a in (x, nw, r))
    x = x.view(1, H)
    router = r.view(E, H)
    nr = ops.NormRouter(1, cuda)
    normed, logits, _, _ = nr(x, nw, eps, router, topk=False)
    sep = ops.rms_norm(x, nw, eps)
    sep_logits = ops.router_logits(sep, router)
    torch.cuda.synchronize()
    assert torch.equal(normed, sep)
    xn = ph.to_np(sep)
    ref = xn.astype(np.float64) @ ph.to_np(router).astype(np.float64).T
    assert np.all(np.abs(ph.to_np(logits) - ref) <= _logit_bound(xn, ph.to_np(router)))
    assert np.all(np.abs(ph.to_np(sep_logits) - ref) <= _logit_bound(xn, ph.to_np(router)))
    # the oracle's RMSNorm (another summation order of the squares) agrees
    # to a few fp32 roundings of the scale
    np.testing.assert_allclose(xn, orc.rms_norm(ph.to_np(x), ph.to_np(nw), eps), rtol=1e-5, atol=1e-7)


CASES = [
    # H, E, k, score_fn, bias sd, scale, act dtype (the c1, c4 and c2 routers)
    (2048, 64, 8, SCORE_SOFTMAX, 0.0, 1.0, torch.float32),
    (4096, 128, 10, SCORE_SOFTMAX, 0.0, 1.0, torch.bfloat16),
    (6144, 256, 8, SCORE_SIGMOID, 0.1, 2.5, torch.bfloat16),
]


@pytest.mark.parametrize("H,E,k,score_fn,bias_sd,scale,act", CASES)
def test_norm_router_topk(cuda, H, E, k, score_fn, bias_sd, scale, act):
    g = torch.Generator(device="cpu").manual_seed(H + E + k)
    router = (0.02 * torch.randn(E, H, generator=g)).to(cuda)
    nw = (1.0 + 0.1 * torch.randn(H, generator=g)).to(cuda)
    bias = (bias_sd * torch.randn(E, generator=g)).to(cuda) if bias_sd else None
    nr = ops.NormRouter(1, cuda)
    near = 0
    for T in (1, 4, 16, 1):
        x = (3.0 * torch.randn(T, H, generator=g)).to(cuda)
        out = nr(x, nw, 1e-6, router, bias, k, score_fn, True, scale, act)
        out2 = nr(x, nw, 1e-6, router, bias, k, score_fn, True, scale, act)
        torch.cuda.synchronize()
        for a, b in zip(out, out2):
            assert torch.equal(a, b), "not bitwise reproducible across calls"
        normed, logits, ids, w = out
        sep = ops.rms_norm(x, nw, 1e-6)
        sep = sep.to(act) if act == torch.bfloat16 else sep
        torch.cuda.synchronize()
        assert torch.equal(normed, sep), "normalised row differs from the RMSNorm launch"
        xn = ph.to_np(normed.float())
        rt = ph.to_np(router)
        ref = xn.astype(np.float64) @ rt.astype(np.float64).T
        lg = ph.to_np(logits)
        assert np.all(np.abs(lg - ref) <= _logit_bound(xn, rt))
        bnp = None if bias is None else ph.to_np(bias)
        oid, ow = orc.router_topk(lg, bnp, k, score_fn, True, scale)
        assert np.array_equal(ph.to_np(ids).view(np.uint32), oid)
        np.testing.assert_allclose(ph.to_np(w), ow, rtol=2e-6, atol=0)
        # against the oracle's own logits: exact except near-ties
        olg = orc.linear(xn, rt)
        oid2, _ = orc.router_topk(olg, bnp, k, score_fn, True, scale)
        score = olg.astype(np.float64) if score_fn == SCORE_SOFTMAX else \
            1 / (1 + np.exp(-olg.astype(np.float64)))
        sel = np.sort(score + (0 if bnp is None else bnp), axis=1)
        for t in range(T):
            if not np.array_equal(np.sort(oid[t * k:(t + 1) * k]), np.sort(oid2[t * k:(t + 1) * k])):
                gap = sel[t, -k] - sel[t, -k - 1]
                assert gap < 1e-6, (t, gap)
                near += 1
    # the ticket workspace is back to zero after every call
    torch.cuda.synchronize()
    assert int(nr._ws.view(torch.int32)[:16].abs().sum()) == 0
    print(f"H={H} E={E} k={k}: near-tie tokens {near}")
