"""Parity of the non-default one-token decode variants.

The decode path switches (INFERNO_DECODE_MFMA, INFERNO_DECODE_RING) are read
once per process, so tests/test_gpu_parity.py runs this file in a child
process per variant:
  tiles  INFERNO_DECODE_MFMA=0: the packed-f16 tile kernels for gate/up and
         down (the default for layers the MFMA kernels do not cover);
  ring   INFERNO_DECODE_MFMA=0 INFERNO_DECODE_RING=1: the opt-in LDS-ring
         gate/up.
Each runs c2 (Q2_K routed + Q8_0 shared, H 6144) and c4 layer 0 (Q2_K, H
4096, top-10, 1536-row shared expert), checked for bitwise reproducibility
over three calls and against the oracle (same tolerance as the other layer
tests).
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


def check(key):
    cuda = torch.device("cuda:0")
    cfg = cf.CONFIGS[key]
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=1)
    x = cf.make_input(cfg, 1, device=cuda)
    residual = torch.randn(1, cfg.hidden, device=cuda)
    ids = torch.empty(cfg.top_k, dtype=torch.int32, device=cuda)
    w = torch.empty(cfg.top_k, dtype=torch.float32, device=cuda)
    outs = [lt.layer.forward(x, residual, ids=ids, weights=w) for _ in range(3)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(outs[0], o), f"{key}: {VARIANT} decode is not bitwise reproducible"
    ref, _, _, flips = ph.oracle_layer_tokens(cfg, lt, x, residual, np.arange(1),
                                              ph.to_np(ids).view(np.uint32), ph.to_np(w))
    res = ph.to_np(residual)
    err = rn.rel_l2(ph.to_np(outs[0]) - res, ref - res)
    print(f"{VARIANT} {key}: rel_l2(moe part)={err:.3e} near-tie tokens={flips}", flush=True)
    assert err < ph.TOL_REL_L2, f"{key}: rel_l2 {err}"


VARIANT = sys.argv[1] if len(sys.argv) > 1 else "tiles"

if __name__ == "__main__":
    assert os.environ.get("INFERNO_DECODE_MFMA") == "0"
    assert (os.environ.get("INFERNO_DECODE_RING") == "1") == (VARIANT == "ring")
    for key in ("c2", "c4"):
        check(key)
    print(f"{VARIANT} ok")
