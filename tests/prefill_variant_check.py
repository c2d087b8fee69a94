"""Parity of the non-default prefill variants.

The prefill switches (INFERNO_PREFILL_GEMM2, INFERNO_ROUTER_BF16X3) are read
once per process, so tests/test_gpu_parity.py runs this file in a child
process with both set to 0: every routed GEMM on the fragment-load kernel
(gemm_kernel, also for the 32- and 64-token tiles) and the router logits of
bf16 tokens on the fp32 matrix-core kernel. It runs c3 (Q3_K, T = 512,
near-uniform load) and checks bitwise reproducibility and sampled tokens
against the oracle (same tolerance as the other layer tests).
"""
import os
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

import parity_helpers as ph  # noqa: E402
import ref_numpy as rn  # noqa: E402
from inferno_amd import configs as cf  # noqa: E402
from inferno_amd import ops  # noqa: E402


def main():
    assert os.environ.get("INFERNO_PREFILL_GEMM2") == "0"
    assert os.environ.get("INFERNO_ROUTER_BF16X3") == "0"
    cuda = torch.device("cuda:0")
    cfg = cf.CONFIGS["c3"]
    T = 512
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=T)
    x = cf.make_input(cfg, T, device=cuda)
    logits = ops.router_logits(x, lt.router)
    lt.bias.copy_(torch.from_numpy(cf.zipf_bias(cfg, ph.to_np(logits))).to(cuda))
    residual = torch.randn(T, cfg.hidden, device=cuda)
    ids = torch.empty(T * cfg.top_k, dtype=torch.int32, device=cuda)
    w = torch.empty(T * cfg.top_k, dtype=torch.float32, device=cuda)
    out = lt.layer.forward(x, residual, ids=ids, weights=w)
    out2 = lt.layer.forward(x, residual)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "prefill variant is not bitwise reproducible"
    tokens = np.array([0, 1, 255, 511])
    ref, _, _, flips = ph.oracle_layer_tokens(cfg, lt, x, residual, tokens,
                                              ph.to_np(ids).view(np.uint32), ph.to_np(w))
    res = ph.to_np(residual)[tokens]
    err = rn.rel_l2(ph.to_np(out)[tokens] - res, ref - res)
    print(f"gemm1 c3: rel_l2(moe part)={err:.3e} near-tie tokens={flips}", flush=True)
    assert err < ph.TOL_REL_L2, f"rel_l2 {err}"
    print("gemm1 ok")


if __name__ == "__main__":
    main()
