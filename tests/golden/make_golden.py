"""Writes tests/golden/golden.npz and golden.json from the CPU oracle.

Test infrastructure: the fixtures pin the oracle and the HIP path against
fixed vectors.
- One super-block per quant kind (bytes + dequantised values).
- One router case per (score function, renormalisation).
- One end-to-end routed-MoE case per (gate/up, down) kind pair.

The MoE weights are regenerated from their seeds by the library's
deterministic host quantiser (inferno_synth_quantized_host). A SHA-256 of
those bytes is stored, so generator drift is caught.

Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parent.parent))

import oracle_lib as orc  # noqa: E402
from inferno_amd import ops  # noqa: E402
from inferno_amd._lib import Q2_K, Q3_K, Q4_K, Q6_K, Q8_0, SCORE_SIGMOID, SCORE_SOFTMAX  # noqa: E402

NAMES = {Q2_K: "q2_k", Q3_K: "q3_k", Q4_K: "q4_k", Q6_K: "q6_k", Q8_0: "q8_0"}
MOE_CASES = [(Q2_K, Q2_K), (Q3_K, Q3_K), (Q4_K, Q4_K), (Q4_K, Q6_K)]
MOE_SHAPE = dict(T=4, E=4, k=2, H=256, I=256)


def normal(seed, n, std=1.0):
    return ops.synth_normal_host(seed, std, n).numpy()


def quantized(quant, seed, rows, cols):
    return ops.synth_quantized_host(quant, seed, 0.02, rows, cols).numpy()


def moe_weights(quant, down, case):
    s = MOE_SHAPE
    base = 5000 + 10 * case
    g = quantized(quant, base + 1, s["E"] * s["I"], s["H"])
    u = quantized(quant, base + 2, s["E"] * s["I"], s["H"])
    d = quantized(down, base + 3, s["E"] * s["H"], s["I"])
    return base, g, u, d


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def build():
    arrays, meta = {}, {"moe_shape": MOE_SHAPE, "moe": {}}
    for q, name in NAMES.items():
        b = quantized(q, 4000 + q, 1, 256)
        arrays[f"block_{name}_bytes"] = b
        arrays[f"block_{name}_values"] = orc.dequantize(q, b)
    for i, (score_fn, norm) in enumerate([(SCORE_SIGMOID, True), (SCORE_SIGMOID, False),
                                          (SCORE_SOFTMAX, True), (SCORE_SOFTMAX, False)]):
        T, E, k = 5, 16, 4
        logits = (1.5 * normal(4100 + i, T * E)).reshape(T, E).astype(np.float32)
        bias = (0.1 * normal(4200 + i, E)).astype(np.float32) if score_fn == SCORE_SIGMOID else None
        ids, w = orc.router_topk(logits, bias, k, score_fn, norm, 2.5)
        key = f"router_{i}"
        arrays[f"{key}_logits"] = logits
        if bias is not None:
            arrays[f"{key}_bias"] = bias
        arrays[f"{key}_ids"] = ids
        arrays[f"{key}_weights"] = w
        meta[key] = {"score_fn": score_fn, "norm": norm, "k": k, "scale": 2.5}
    s = MOE_SHAPE
    for case, (q, dq) in enumerate(MOE_CASES):
        base, g, u, d = moe_weights(q, dq, case)
        x = normal(base + 4, s["T"] * s["H"]).reshape(s["T"], s["H"]).astype(np.float32)
        ids = np.array([[0, 1], [2, 3], [1, 2], [3, 0]], np.uint32).reshape(-1)
        w = np.abs(normal(base + 5, s["T"] * s["k"])).astype(np.float32)
        y = orc.moe_routed(q, dq, g, u, d, x, ids, w, s["E"], s["k"], s["I"])
        key = f"moe_{NAMES[q]}_{NAMES[dq]}"
        arrays[f"{key}_x"] = x
        arrays[f"{key}_ids"] = ids
        arrays[f"{key}_weights"] = w
        arrays[f"{key}_y"] = y
        meta["moe"][key] = {"quant": q, "down_quant": dq, "seed_base": base,
                            "weights_sha256": sha(g, u, d)}
    return arrays, meta


if __name__ == "__main__":
    arrays, meta = build()
    np.savez(HERE / "golden.npz", **arrays)
    (HERE / "golden.json").write_text(json.dumps(meta, indent=1, sort_keys=True) + "\n")
    print(f"wrote {len(arrays)} arrays")
