"""The five BASELINE.json workloads as seeded synthetic GPU-resident layers.

Seeds: 1000 + config index; sub-streams per tensor (x, router, bias, gate,
up, down, shared gate/up/down) and per layer. Weights are N(0, 0.02)
quantised on the device (inferno_synth_quantized); activations N(0, 1).
"""
from dataclasses import dataclass, field

import numpy as np
import torch

from ._lib import BF16, F32, Q2_K, Q3_K, Q4_K, Q6_K, Q8_0, SCORE_SIGMOID, SCORE_SOFTMAX
from . import ops


@dataclass
class Config:
    name: str
    index: int
    hidden: int
    experts: int
    intermediate: int
    top_k: int
    quants: tuple              # routed kind per layer
    score_fn: int
    norm: bool
    scale: float
    bias_std: float            # 0 = no correction bias
    shared_intermediate: int   # 0 = no shared expert
    x_dtype: torch.dtype
    tokens: tuple
    zipf: float = 0.0          # >0: bias calibrated so expert load follows Zipf(s)
    balanced: bool = False     # bias calibrated so expert load is near-uniform (Zipf(0))
    zipf_empty: int = 0        # experts given no slot by the calibrated bias
    down_quant: int = 0        # routed down format (0: the gate/up format)
    shared_quant: int = Q8_0   # shared expert gate/up format
    shared_down_quant: int = 0  # shared down format (0: the routed down format for a
                                # non-Q8_0 shared expert, as Laguna XS; Q8_0 otherwise)
    rms_eps: float = 1e-6
    notes: str = ""
    weight_std: float = 0.02

    @property
    def seed(self):
        return 1000 + self.index

    @property
    def layers(self):
        return len(self.quants)


CONFIGS = {
    "c1": Config("c1_q4k_h2048_e64_top8_softmax", 0, 2048, 64, 768, 8, (Q4_K,), SCORE_SOFTMAX,
                 True, 1.0, 0.0, 0, torch.float32, (1, 16)),
    "c2": Config("c2_glm_q2k_h6144_e256_top8_sigmoid_decode", 1, 6144, 256, 2048, 8, (Q2_K,),
                 SCORE_SIGMOID, True, 2.5, 0.1, 2048, torch.bfloat16, (1,)),
    "c3": Config("c3_glm_q3k_prefill_t512", 2, 6144, 256, 2048, 8, (Q3_K,), SCORE_SIGMOID, True,
                 2.5, 0.1, 2048, torch.bfloat16, (512,), balanced=True),
    "c4": Config("c4_laguna_s_4layer_q2k_q3k_top10_softmax", 3, 4096, 128, 1536, 10,
                 (Q2_K, Q2_K, Q3_K, Q3_K), SCORE_SOFTMAX, True, 1.0, 0.0, 1536, torch.bfloat16,
                 (1, 32)),
    "c5": Config("c5_glm_q2k_prefill_t4096_zipf", 4, 6144, 256, 2048, 8, (Q2_K,), SCORE_SIGMOID,
                 True, 2.5, 0.1, 2048, torch.bfloat16, (4096,), zipf=1.1, zipf_empty=40),
    # not a BASELINE workload: the Laguna XS layer formats (routed Q4_K gate/up
    # with Q6_K down, a Q4_K/Q6_K shared expert of the routed width) at c1's
    # shape, one token and 64 tokens
    "xs": Config("xs_c1shape_q4k_q6kdown_q4k_shared", 5, 2048, 64, 768, 8, (Q4_K,),
                 SCORE_SOFTMAX, True, 1.0, 0.0, 768, torch.float32, (1, 64), down_quant=Q6_K,
                 shared_quant=Q4_K),
}

# sub-stream ids
_X, _ROUTER, _BIAS, _GATE, _UP, _DOWN, _SG, _SU, _SD, _NORM = range(10)


def stream_seed(cfg, layer, which, variant=0):
    return (cfg.seed << 20) | (layer << 12) | (variant << 4) | which


@dataclass
class LayerTensors:
    quant: int
    router: torch.Tensor
    bias: torch.Tensor
    gate: torch.Tensor
    up: torch.Tensor
    down: torch.Tensor
    shared: tuple = None
    norm_w: torch.Tensor = None
    down_quant: int = 0
    shared_quant: int = Q8_0
    shared_down_quant: int = Q8_0
    layer: ops.MoELayer = field(default=None, repr=False)


def make_input(cfg, T, variant=0, device="cuda"):
    return ops.synth_normal(stream_seed(cfg, 0, _X, variant), 1.0, T * cfg.hidden,
                            dtype=cfg.x_dtype, device=device).view(T, cfg.hidden)


def build_layer(cfg, layer=0, device="cuda", max_tokens=1, bias=None):
    H, E, I = cfg.hidden, cfg.experts, cfg.intermediate
    q = cfg.quants[layer]
    ws = cfg.weight_std
    router = ops.synth_normal(stream_seed(cfg, layer, _ROUTER), ws, E * H, device=device).view(E, H)
    if bias is None and cfg.bias_std > 0:
        bias = ops.synth_normal(stream_seed(cfg, layer, _BIAS), cfg.bias_std, E, device=device)
    dq = cfg.down_quant or q
    sq = cfg.shared_quant
    sdq = cfg.shared_down_quant or (Q8_0 if sq == Q8_0 else dq)
    gate = ops.synth_quantized(q, stream_seed(cfg, layer, _GATE), ws, E * I, H, device)
    up = ops.synth_quantized(q, stream_seed(cfg, layer, _UP), ws, E * I, H, device)
    down = ops.synth_quantized(dq, stream_seed(cfg, layer, _DOWN), ws, E * H, I, device)
    shared = None
    Is = cfg.shared_intermediate
    if Is:
        shared = (ops.synth_quantized(sq, stream_seed(cfg, layer, _SG), ws, Is, H, device),
                  ops.synth_quantized(sq, stream_seed(cfg, layer, _SU), ws, Is, H, device),
                  ops.synth_quantized(sdq, stream_seed(cfg, layer, _SD), ws, H, Is, device))
    norm_w = 1.0 + ops.synth_normal(stream_seed(cfg, layer, _NORM), 0.1, H, device=device)
    lt = LayerTensors(q, router, bias, gate, up, down, shared, norm_w, down_quant=dq,
                      shared_quant=sq, shared_down_quant=sdq)
    lt.layer = ops.MoELayer(
        hidden=H, experts=E, intermediate=I, top_k=cfg.top_k, quant=q, down_quant=dq,
        score_fn=cfg.score_fn, norm_topk_prob=cfg.norm, routed_scaling_factor=cfg.scale,
        router=router, router_bias=bias, gate=gate, up=up, down=down,
        shared_intermediate=Is,
        shared_gate=shared[0] if shared else None, shared_up=shared[1] if shared else None,
        shared_down=shared[2] if shared else None, shared_quant=sq, shared_down_quant=sdq,
        max_tokens=max_tokens)
    return lt


def load_targets(cfg, T):
    """Integer slot counts per expert rank for a T-token batch: Zipf(cfg.zipf)
    over the first E - cfg.zipf_empty ranks (cfg.zipf = 0: equal load), none
    for the last cfg.zipf_empty. An expert takes at most one slot per token,
    so a share above T slots is capped at T (for top-8: 12.5% of the slots)
    and the excess spread over the other active ranks in proportion."""
    E, k = cfg.experts, cfg.top_k
    A = T * k
    active = E - cfg.zipf_empty
    p = np.zeros(E)
    p[:active] = np.arange(1, active + 1, dtype=np.float64) ** (-cfg.zipf)
    target = A * p / p.sum()
    for _ in range(64):
        over = target > T
        if not over.any():
            break
        excess = (target[over] - T).sum()
        target[over] = T
        rest = (~over) & (p > 0)
        target[rest] += excess * target[rest] / target[rest].sum()
    counts = np.floor(target).astype(np.int64)
    counts[np.argsort(-(target - counts), kind="stable")[:A - counts.sum()]] += 1
    return counts


def zipf_bias(cfg, logits, iters=60):
    """Correction bias that gives expert e exactly load_targets(cfg, T)[e]
    top-k slots on these router logits (sigmoid scores), to within a slot.

    Damped best response: with the other experts' biases fixed, expert e is
    selected by token t exactly when score[t, e] + b_e exceeds the k-th
    largest selection value among the other experts of t; the bias that gives
    e its target count c is the midpoint between the c-th and (c+1)-th
    smallest of those margins. Every expert moves halfway to its best
    response per iteration (numpy, on the host, from the device logits).
    """
    T, E = logits.shape
    k = cfg.top_k
    target = load_targets(cfg, T)
    score = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    b = np.zeros(E)
    for _ in range(iters):
        sel = score + b
        top = -np.partition(-sel, k, axis=1)[:, :k + 1]
        top.sort(axis=1)  # ascending: (k+1)-th largest first
        kth, k1th = top[:, 1], top[:, 0]
        thr = np.where(sel >= kth[:, None], k1th[:, None], kth[:, None])
        need = np.sort(thr - score, axis=0)
        nb = np.empty(E)
        for e in range(E):
            c = target[e]
            if c == 0:
                nb[e] = need[0, e] - 1.0
            elif c >= T:
                nb[e] = need[T - 1, e] + 1.0
            else:
                nb[e] = 0.5 * (need[c - 1, e] + need[c, e])
        b = 0.5 * b + 0.5 * nb
    return b.astype(np.float32)


def build_stack(cfg, device="cuda", max_tokens=1):
    """The config's consecutive layers (one per entry of cfg.quants), each
    with its own seeded tensors and RMSNorm weight, as an ops.MoEStack."""
    lts = [build_layer(cfg, l, device, max_tokens=max_tokens) for l in range(cfg.layers)]
    stack = ops.MoEStack([lt.layer for lt in lts], [lt.norm_w for lt in lts], eps=cfg.rms_eps,
                         act_dtype=cfg.x_dtype, max_tokens=max_tokens)
    return lts, stack


def make_hidden(cfg, T, variant=0, device="cuda"):
    """fp32 residual stream entering the stack: the config's N(0, 1)
    activations (bf16 values for bf16 configs) held as fp32."""
    return make_input(cfg, T, variant, device).float()
