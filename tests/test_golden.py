"""Golden fixtures (tests/golden/, written by make_golden.py from the oracle).

CPU: the oracle and the deterministic host quantiser still reproduce the
fixtures exactly. GPU: the HIP path matches them — dequantisation bit-exact,
routing ids exact and weights to 1e-6, MoE outputs within relative L2 2e-3.
"""
import json
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "golden"))

import make_golden as mg  # noqa: E402
import oracle_lib as orc  # noqa: E402
import parity_helpers as ph  # noqa: E402
import ref_numpy as rn  # noqa: E402
from inferno_amd import ops  # noqa: E402

G = np.load(HERE / "golden" / "golden.npz", allow_pickle=False)
META = json.loads((HERE / "golden" / "golden.json").read_text())
S = META["moe_shape"]


@pytest.mark.parametrize("quant", list(mg.NAMES))
def test_golden_block_oracle(quant):
    name = mg.NAMES[quant]
    b = mg.quantized(quant, 4000 + quant, 1, 256)
    assert np.array_equal(b, G[f"block_{name}_bytes"]), "host quantiser drifted"
    got = orc.dequantize(quant, G[f"block_{name}_bytes"])
    assert np.array_equal(got.view(np.uint32), G[f"block_{name}_values"].view(np.uint32))


@pytest.mark.parametrize("i", range(4))
def test_golden_router_oracle(i):
    key, m = f"router_{i}", META[f"router_{i}"]
    bias = G[f"{key}_bias"] if f"{key}_bias" in G else None
    ids, w = orc.router_topk(G[f"{key}_logits"], bias, m["k"], m["score_fn"], m["norm"],
                             m["scale"])
    assert np.array_equal(ids, G[f"{key}_ids"])
    assert np.array_equal(w.view(np.uint32), G[f"{key}_weights"].view(np.uint32))


@pytest.mark.parametrize("key", sorted(META["moe"]))
def test_golden_moe_oracle(key):
    m = META["moe"][key]
    case = [f"moe_{mg.NAMES[q]}_{mg.NAMES[d]}" for q, d in mg.MOE_CASES].index(key)
    base, g, u, d = mg.moe_weights(m["quant"], m["down_quant"], case)
    assert base == m["seed_base"] and mg.sha(g, u, d) == m["weights_sha256"]
    y = orc.moe_routed(m["quant"], m["down_quant"], g, u, d, G[f"{key}_x"], G[f"{key}_ids"],
                       G[f"{key}_weights"], S["E"], S["k"], S["I"])
    assert np.array_equal(y.view(np.uint32), G[f"{key}_y"].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("quant", list(mg.NAMES))
def test_golden_block_gpu(cuda, quant):
    name = mg.NAMES[quant]
    got = ph.to_np(ops.dequantize(quant, torch.from_numpy(G[f"block_{name}_bytes"]).to(cuda)))
    assert np.array_equal(got.reshape(-1).view(np.uint32),
                          G[f"block_{name}_values"].reshape(-1).view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(4))
def test_golden_router_gpu(cuda, i):
    key, m = f"router_{i}", META[f"router_{i}"]
    bias = torch.from_numpy(G[f"{key}_bias"]).to(cuda) if f"{key}_bias" in G else None
    ids, w, _ = ops.router_topk(torch.from_numpy(G[f"{key}_logits"]).to(cuda), bias, m["k"],
                                m["score_fn"], m["norm"], m["scale"])
    assert np.array_equal(ph.to_np(ids).view(np.uint32), G[f"{key}_ids"])
    assert np.allclose(ph.to_np(w), G[f"{key}_weights"], rtol=1e-6, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("key", sorted(META["moe"]))
def test_golden_moe_gpu(cuda, key):
    m = META["moe"][key]
    case = [f"moe_{mg.NAMES[q]}_{mg.NAMES[d]}" for q, d in mg.MOE_CASES].index(key)
    _, g, u, d = mg.moe_weights(m["quant"], m["down_quant"], case)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)  # noqa: E731
    y = ops.gguf_moe(m["quant"], m["down_quant"], dev(g), dev(u), dev(d), dev(G[f"{key}_x"]),
                     dev(G[f"{key}_ids"].view(np.int32)), dev(G[f"{key}_weights"]), S["k"],
                     S["E"], S["I"])
    err = rn.rel_l2(ph.to_np(y), G[f"{key}_y"])
    assert err < ph.TOL_REL_L2, err
