"""Helpers that run the CPU oracle on a GPU-resident layer (tests only)."""
import numpy as np
import torch

import oracle_lib as orc
import ref_numpy as rn
from inferno_amd import ops

TOL_REL_L2 = 2e-3   # MoE output within relative L2 2e-3
NEAR_TIE = 1e-6     # routing near-ties within 1e-6 of the k-th selection value


def to_np(t):
    return t.detach().cpu().numpy()


def x_f32(x):
    return to_np(x.float())


def compact_experts(lt, cfg, experts):
    """Host copies of the packed gate/up/down bytes of `experts` only."""
    E, H, I = cfg.experts, cfg.hidden, cfg.intermediate
    g = lt.gate.view(E, -1)[experts]
    u = lt.up.view(E, -1)[experts]
    d = lt.down.view(E, -1)[experts]
    return to_np(g).reshape(-1), to_np(u).reshape(-1), to_np(d).reshape(-1)


def selection_values(cfg, logits, bias):
    l64 = logits.astype(np.float32)
    if cfg.score_fn == 0:
        s = (1.0 / (1.0 + np.exp(-l64.astype(np.float64)))).astype(np.float32)
    else:
        s = l64
    return s + (bias if bias is not None else 0)


def compare_routing(cfg, ids_gpu, ids_orc, sel_orc, tie=NEAR_TIE, tokens_out=None):
    """Counts tokens whose GPU selection differs from the oracle's only by
    near-ties: at every rank the two chosen experts' selection values (the
    oracle's fp32 values) differ by at most `tie`. Any other difference
    raises. Returns (all_exact, n_near_tie_tokens); the near-tie token rows
    are appended to tokens_out when given."""
    T = sel_orc.shape[0]
    k = cfg.top_k
    a = np.asarray(ids_gpu).reshape(T, k)
    b = np.asarray(ids_orc).reshape(T, k)
    flips = 0
    for t in range(T):
        if np.array_equal(a[t], b[t]):
            continue
        gap = np.abs(sel_orc[t, a[t]].astype(np.float64) - sel_orc[t, b[t]].astype(np.float64))
        if np.all(gap <= tie):
            flips += 1
            if tokens_out is not None:
                tokens_out.append(t)
            continue
        raise AssertionError(f"token {t}: gpu ids {a[t]} vs oracle {b[t]} (not a near-tie: "
                             f"largest gap {gap.max():.3e} > {tie:.1e})")
    return flips == 0, flips


def oracle_layer_tokens(cfg, lt, x, residual, tokens, ids_gpu, w_gpu, bias_np=None):
    """Oracle forward of layer `lt` for the given token rows.

    Routing is recomputed by the oracle from x and the router; the routed
    output uses the oracle's routing. Returns (out, ids_orc, w_orc, flips).
    """
    xs = x_f32(x)[tokens]
    res = None if residual is None else to_np(residual)[tokens]
    g_ids = np.asarray(ids_gpu).reshape(-1, cfg.top_k)[tokens].reshape(-1)
    g_w = None if w_gpu is None else np.asarray(w_gpu).reshape(-1, cfg.top_k)[tokens].reshape(-1)
    return oracle_layer_rows(cfg, lt, xs, res, g_ids, bias_np, w_gpu_rows=g_w)


def oracle_layer_rows(cfg, lt, xs, res, ids_gpu_rows, bias_np=None, tie=NEAR_TIE,
                      tie_tokens=None, w_gpu_rows=None):
    """Oracle forward of layer `lt` on activation rows xs (fp32 numpy) with
    residual rows res (or None); ids_gpu_rows = the GPU's routing of the same
    rows, compared with the oracle's (near-ties within `tie` counted, their
    rows appended to tie_tokens). When the GPU's weights w_gpu_rows are given,
    the experts of a near-tie row are computed with the GPU's selection (ids
    and weights), so that row's expert arithmetic is still compared."""
    router = to_np(lt.router)
    bias = bias_np if bias_np is not None else (None if lt.bias is None else to_np(lt.bias))
    logits = orc.linear(xs, router)
    ids_o, w_o = orc.router_topk(logits, bias, cfg.top_k, cfg.score_fn, cfg.norm, cfg.scale)
    sel = selection_values(cfg, logits, bias)
    k = cfg.top_k
    rows_tied = []
    _, flips = compare_routing(cfg, ids_gpu_rows, ids_o, sel, tie, rows_tied)
    if tie_tokens is not None:
        tie_tokens.extend(rows_tied)
    if w_gpu_rows is not None and rows_tied:
        ids_o = ids_o.reshape(-1, k).copy()
        w_o = w_o.reshape(-1, k).copy()
        gi = np.asarray(ids_gpu_rows).reshape(-1, k)
        gw = np.asarray(w_gpu_rows).reshape(-1, k)
        for t in rows_tied:
            ids_o[t], w_o[t] = gi[t], gw[t]
        ids_o, w_o = ids_o.reshape(-1), w_o.reshape(-1)
    experts = np.unique(ids_o)
    remap = {int(e): i for i, e in enumerate(experts)}
    g, u, d = compact_experts(lt, cfg, torch.as_tensor(experts.astype(np.int64), device=lt.gate.device))
    ids_c = np.array([remap[int(e)] for e in ids_o], np.uint32)
    dq = getattr(lt, "down_quant", 0) or lt.quant
    routed = orc.moe_routed(lt.quant, dq, g, u, d, xs, ids_c, w_o, len(experts), k,
                            cfg.intermediate)
    if lt.shared is not None:
        sg, su, sd = (to_np(s) for s in lt.shared)
        out = orc.shared_ffn(getattr(lt, "shared_quant", 8), getattr(lt, "shared_down_quant", 8),
                             sg, su, sd, xs, cfg.shared_intermediate, routed=routed,
                             residual=res)
    else:
        out = routed + (0 if res is None else res)
    return out, ids_o, w_o, flips


def bf16_round(a):
    """fp32 -> nearest-even bf16 -> fp32 (finite inputs)."""
    b = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16 << 16
    return b.astype(np.uint32).view(np.float32)


# Routing tolerance inside an oracle chain of several layers. From the second
# layer on, the GPU and the oracle feed the layer residual streams that
# already differ by the earlier layers' rounding, so their activations differ
# by some delta and every logit by at most sum_h |W_r[e, h]| |delta_h|: experts
# whose selection values lie that close to the k-th may trade places. The
# bound is computed per token and layer from the GPU's own stream entering
# the layer (oracle_stack_tokens gpu_streams); CHAIN_TIE is the fallback when
# those are not given.
CHAIN_TIE = 2e-2


def compare_routing_sets(cfg, ids_gpu, ids_orc, sel_orc, tie):
    """Chain routing check: rank order inside the same expert set only
    changes the order of the rank sum and passes; a different set passes
    when every expert in one set and not the other is within `tie` (a scalar
    or one bound per token) of the k-th selection value (its token row is
    returned), else raises."""
    T = sel_orc.shape[0]
    k = cfg.top_k
    a = np.asarray(ids_gpu).reshape(T, k)
    b = np.asarray(ids_orc).reshape(T, k)
    ties = np.broadcast_to(np.asarray(tie, np.float64), (T,))
    diff_rows = []
    for t in range(T):
        sa, sb = set(a[t].tolist()), set(b[t].tolist())
        if sa == sb:
            continue
        kth = float(np.sort(sel_orc[t, b[t]])[0])
        gap = max(abs(float(sel_orc[t, e]) - kth) for e in sa ^ sb)
        if gap > ties[t]:
            raise AssertionError(f"token {t}: gpu experts {sorted(sa)} vs oracle {sorted(sb)} "
                                 f"(selection gap {gap:.3e} to the k-th > {ties[t]:.3e})")
        diff_rows.append(t)
    return diff_rows


def stack_layer_input(cfg, lt, r):
    """The oracle's activations for a stack layer: RMSNorm of the residual
    rows r, rounded to bf16 for bf16 configs."""
    a = orc.rms_norm(r, to_np(lt.norm_w), cfg.rms_eps)
    return bf16_round(a) if cfg.x_dtype == torch.bfloat16 else a


def oracle_stack_tokens(cfg, lts, hidden, tokens, ids_gpu_all, gpu_streams=None):
    """Oracle chain of a layer stack on the given token rows: for each layer,
    a = rms_norm(r) rounded to the activation type, r = layer(a, residual=r).
    gpu_streams[l] (optional): the GPU's residual stream entering layer l
    (all T rows); it bounds how far the two chains' logits can have drifted.
    Returns (final rows, per layer the token rows whose expert set differs
    from the GPU's within that bound)."""
    r = to_np(hidden)[tokens].astype(np.float32)
    T = hidden.shape[0]
    k = cfg.top_k
    differs = []
    off = 0
    for l, lt in enumerate(lts):
        a = stack_layer_input(cfg, lt, r)
        g_ids = np.asarray(ids_gpu_all[off:off + T * k]).reshape(T, k)[tokens].reshape(-1)
        off += T * k
        router = to_np(lt.router)
        logits = orc.linear(a, router)
        bias = None if lt.bias is None else to_np(lt.bias)
        ids_o, _ = orc.router_topk(logits, bias, k, cfg.score_fn, cfg.norm, cfg.scale)
        tie = CHAIN_TIE
        if gpu_streams is not None and l > 0:
            a_gpu = stack_layer_input(cfg, lt, to_np(gpu_streams[l])[tokens].astype(np.float32))
            delta = np.abs(a_gpu.astype(np.float64) - a.astype(np.float64))
            tie = 2.0 * (delta @ np.abs(router.astype(np.float64)).T).max(axis=1) + 1e-6
        differs.append(compare_routing_sets(cfg, g_ids, ids_o,
                                            selection_values(cfg, logits, bias), tie))
        # the layer itself, with the oracle's own routing (rank order checks off)
        r, _, _, _ = oracle_layer_rows(cfg, lt, a, r, ids_o, tie=0.0)
    return r, differs
