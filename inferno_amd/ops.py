"""Torch-tensor wrappers over the C ABI (device memory and streams only).

Every function here calls straight into libinferno_moe.so; tensors must live
on the GPU. uint32 outputs of the ABI are held in torch.int32 tensors.
"""
import ctypes as C

import torch

from ._lib import BF16, F32, Q8_0, LayerDesc, check, lib

_DT = {torch.float32: F32, torch.bfloat16: BF16}


def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _s():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dev(t):
    if not t.is_cuda:
        raise ValueError("inferno_amd ops need GPU tensors")
    return t


def block_bytes(quant):
    return lib().inferno_block_bytes(quant)


def block_values(quant):
    return lib().inferno_block_values(quant)


def matrix_bytes(quant, rows, cols):
    return rows * (cols // block_values(quant)) * block_bytes(quant)


def dequantize(quant, blocks):
    n_blocks = blocks.numel() // block_bytes(quant)
    out = torch.empty(n_blocks * block_values(quant), dtype=torch.float32, device=blocks.device)
    check(lib().inferno_gguf_dequantize(_s(), quant, _p(_dev(blocks)), n_blocks, _p(out)))
    return out


def router_logits(x, w_router):
    T, H = x.shape
    E = w_router.shape[0]
    out = torch.empty(T, E, dtype=torch.float32, device=x.device)
    check(lib().inferno_router_logits(_s(), _p(_dev(x)), _DT[x.dtype], _p(w_router), T, H, E,
                                      _p(out)))
    return out


def router_topk(logits, bias, k, score_fn, norm, scale):
    T, E = logits.shape
    ids = torch.empty(T * k, dtype=torch.int32, device=logits.device)
    w = torch.empty(T * k, dtype=torch.float32, device=logits.device)
    tok = torch.empty(T * k, dtype=torch.int32, device=logits.device)
    check(lib().inferno_moe_router_topk(_s(), _p(_dev(logits)), _p(bias), T, E, k, score_fn,
                                        int(norm), float(scale), _p(ids), _p(w), _p(tok)))
    return ids, w, tok


def dispatch(ids, T, k, E):
    dev = ids.device
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    sorted_ = torch.empty(max(T * k, 1), dtype=torch.int32, device=dev)
    active = torch.empty(E + 1, dtype=torch.int32, device=dev)
    check(lib().inferno_moe_dispatch(_s(), _p(_dev(ids)), T, k, E, _p(offsets), _p(sorted_),
                                     _p(active)))
    return offsets, sorted_[: T * k], active


def gguf_moe(quant, down_quant, gate, up, down, x, ids, weights, k, E, I):
    T, H = x.shape
    ws_bytes = lib().inferno_gguf_moe_workspace_bytes(T, k, E, H, I)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    out = torch.empty(T, H, dtype=torch.float32, device=x.device)
    check(lib().inferno_gguf_moe(_s(), quant, down_quant, _p(gate), gate.numel(), _p(up),
                                 up.numel(), _p(down), down.numel(), _p(_dev(x)), _DT[x.dtype],
                                 _p(ids), _p(weights), T, k, E, H, I, _p(out), _p(ws), ws_bytes))
    return out


def gemv_workspace(rows, K, device):
    n = lib().inferno_gemv_workspace_bytes(rows, K)
    return torch.empty(max(n, 1), dtype=torch.uint8, device=device)


def expert_gate_up_swiglu(quant, gate, up, x, offsets, sorted_, active, weights, k, E, I,
                          out=None, ws=None):
    T, H = x.shape
    if out is None:
        out = torch.empty(T * k, I, dtype=torch.float32, device=x.device)
    if ws is None:
        ws = gemv_workspace(T, H, x.device)
    check(lib().inferno_moe_expert_gate_up_swiglu(
        _s(), quant, _p(gate), gate.numel(), _p(up), up.numel(), _p(_dev(x)), _DT[x.dtype],
        _p(offsets), _p(sorted_), _p(active), _p(weights), T, k, E, H, I, _p(out), _p(ws),
        ws.numel()))
    return out


def expert_down(down_quant, down, h, offsets, sorted_, active, T, k, E, H, out=None, ws=None):
    I = h.shape[1]
    if out is None:
        out = torch.empty(T * k, H, dtype=torch.float32, device=h.device)
    if ws is None:
        ws = gemv_workspace(T * k, I, h.device)
    check(lib().inferno_moe_expert_down(_s(), down_quant, _p(down), down.numel(), _p(_dev(h)),
                                        _p(offsets), _p(sorted_), _p(active), T, k, E, H, I,
                                        _p(out), _p(ws), ws.numel()))
    return out


def q8_0_gate_up_swiglu(gate, up, x, Is):
    T, H = x.shape
    out = torch.empty(T, Is, dtype=torch.float32, device=x.device)
    ws = gemv_workspace(T, H, x.device)
    check(lib().inferno_q8_0_gate_up_swiglu(_s(), _p(gate), gate.numel(), _p(up), up.numel(),
                                            _p(_dev(x)), _DT[x.dtype], T, H, Is, _p(out), _p(ws),
                                            ws.numel()))
    return out


def q8_0_matvec_add2(w, inp, residual_a, residual_b, O):
    T, In = inp.shape
    out = torch.empty(T, O, dtype=torch.float32, device=inp.device)
    ws = gemv_workspace(T, In, inp.device)
    check(lib().inferno_q8_0_matvec_add2(_s(), _p(w), w.numel(), _p(_dev(inp)), _p(residual_a),
                                         _p(residual_b), T, In, O, _p(out), _p(ws), ws.numel()))
    return out


def topk_combine_residual(shared, residual, expert_outputs, expert_weights, k):
    A, H = expert_outputs.shape
    T = A // k
    out = torch.empty(T, H, dtype=torch.float32, device=expert_outputs.device)
    check(lib().inferno_moe_topk_combine_residual(_s(), _p(shared), _p(residual),
                                                  _p(_dev(expert_outputs)), _p(expert_weights),
                                                  T, H, k, _p(out)))
    return out


def weighted_index_add_combine(acc, token_indices, expert_outputs, expert_weights):
    T, H = acc.shape
    A = token_indices.numel()
    out = torch.empty_like(acc)
    check(lib().inferno_moe_weighted_index_add_combine(_s(), _p(_dev(acc)), _p(token_indices),
                                                       _p(expert_outputs), _p(expert_weights),
                                                       T, H, A, _p(out)))
    return out


def gather_tokens(x, token_indices):
    T, H = x.shape
    A = token_indices.numel()
    out = torch.empty(A, H, dtype=torch.float32, device=x.device)
    check(lib().inferno_moe_gather_tokens(_s(), _p(_dev(x)), _p(token_indices), T, H, A, _p(out)))
    return out


def rms_norm(x, w, eps):
    rows, H = x.shape
    out = torch.empty_like(x)
    check(lib().inferno_rms_norm(_s(), _p(_dev(x)), _p(w), rows, H, float(eps), _p(out)))
    return out


class NormRouter:
    """RMSNorm -> router logits (-> top-k) of decode tokens in one launch
    (inferno_rms_norm_router_topk; Backend::laguna_xs_rms_norm_router_device
    followed by the decode top-k). Holds the zero-filled ticket workspace the
    top-k needs; calls through one instance must not overlap."""

    def __init__(self, max_tokens=1, device="cuda"):
        self._ws = torch.zeros(lib().inferno_rms_norm_router_topk_workspace_bytes(max_tokens),
                               dtype=torch.uint8, device=device)
        self.max_tokens = max_tokens

    def __call__(self, x, norm_weight, eps, router, bias=None, k=0, score_fn=0, norm=True,
                 scale=1.0, act_dtype=torch.float32, topk=True):
        T, H = x.shape
        E = router.shape[0]
        if T > self.max_tokens:
            self.__init__(T, x.device)
        normed = torch.empty(T, H, dtype=act_dtype, device=x.device)
        logits = torch.empty(T, E, dtype=torch.float32, device=x.device)
        ids = torch.empty(T * k, dtype=torch.int32, device=x.device) if topk else None
        w = torch.empty(T * k, dtype=torch.float32, device=x.device) if topk else None
        check(lib().inferno_rms_norm_router_topk(
            _s(), _p(_dev(x)), _p(norm_weight), float(eps), _p(router), _p(bias), T, H, E, k,
            score_fn, int(norm), float(scale), _DT[act_dtype], _p(normed), _p(logits), _p(ids),
            _p(w), _p(self._ws), self._ws.numel()))
        return normed, logits, ids, w


TIMER_GATE_UP, TIMER_DOWN, TIMER_ROUTE, TIMER_SELECT = 0, 1, 2, 3


def kernel_timing(enable):
    """Turns the event timing of the layer's launches (route, select, gate/up,
    down) on or off. Events are recorded around each launch without a wait;
    ``kernel_timing_read`` settles and sums them (measurement only)."""
    check(lib().inferno_kernel_timing_enable(1 if enable else 0))


def kernel_timing_read(which):
    """(total ms, launches) accumulated by one timer since the last read."""
    ms, n = C.c_double(0.0), C.c_uint64(0)
    check(lib().inferno_kernel_timing_read(which, C.byref(ms), C.byref(n)))
    return ms.value, n.value


def kernel_timing_label(which):
    """Label of the last launch a timer measured: "<kind>: <kernel> (...)"."""
    buf = C.create_string_buffer(256)
    check(lib().inferno_kernel_timing_label(which, buf, len(buf)))
    return buf.value.decode()


def synth_normal(seed, stddev, n, dtype=torch.float32, device="cuda"):
    out = torch.empty(n, dtype=dtype, device=device)
    check(lib().inferno_synth_normal(_s(), seed, float(stddev), n, _DT[dtype], _p(out)))
    return out


def synth_quantized(quant, seed, stddev, rows, cols, device="cuda"):
    out = torch.empty(matrix_bytes(quant, rows, cols), dtype=torch.uint8, device=device)
    check(lib().inferno_synth_quantized(_s(), quant, seed, float(stddev), rows, cols, _p(out)))
    return out


def synth_normal_host(seed, stddev, n):
    out = torch.empty(n, dtype=torch.float32)
    check(lib().inferno_synth_normal_host(seed, float(stddev), n, _p(out)))
    return out


def synth_quantized_host(quant, seed, stddev, rows, cols):
    out = torch.empty(matrix_bytes(quant, rows, cols), dtype=torch.uint8)
    check(lib().inferno_synth_quantized_host(quant, seed, float(stddev), rows, cols, _p(out)))
    return out


def quantize_rows_host(quant, x):
    rows, cols = x.shape
    x = x.contiguous().float()
    out = torch.empty(matrix_bytes(quant, rows, cols), dtype=torch.uint8)
    check(lib().inferno_quantize_rows_host(quant, _p(x), rows, cols, _p(out)))
    return out


class MoELayer:
    """One MoE FFN layer resident on the GPU (inferno_moe_layer_forward).

    Holds device tensors for the router, routed experts and optional Q8_0
    shared expert, and a reusable workspace sized for `max_tokens`.
    """

    def __init__(self, *, hidden, experts, intermediate, top_k, quant, down_quant, score_fn,
                 norm_topk_prob, routed_scaling_factor, router, router_bias, gate, up, down,
                 shared_intermediate=0, shared_gate=None, shared_up=None, shared_down=None,
                 shared_quant=Q8_0, shared_down_quant=Q8_0, max_tokens=1):
        self.tensors = [router, router_bias, gate, up, down, shared_gate, shared_up, shared_down]
        d = LayerDesc()
        d.hidden, d.experts, d.intermediate, d.top_k = hidden, experts, intermediate, top_k
        d.quant, d.down_quant, d.score_fn = quant, down_quant, score_fn
        d.norm_topk_prob, d.routed_scaling_factor = int(norm_topk_prob), routed_scaling_factor
        d.router, d.router_bias = _p(router), _p(router_bias)
        d.gate, d.up, d.down = _p(gate), _p(up), _p(down)
        d.gate_bytes, d.up_bytes, d.down_bytes = gate.numel(), up.numel(), down.numel()
        d.shared_intermediate = shared_intermediate
        if shared_intermediate:
            d.shared_gate, d.shared_up, d.shared_down = _p(shared_gate), _p(shared_up), _p(shared_down)
            d.shared_gate_bytes = shared_gate.numel()
            d.shared_up_bytes = shared_up.numel()
            d.shared_down_bytes = shared_down.numel()
            d.shared_quant, d.shared_down_quant = shared_quant, shared_down_quant
        self.desc = d
        self.hidden, self.top_k = hidden, top_k
        self.device = gate.device
        self._ws = None
        self.reserve(max_tokens)

    def reserve(self, T):
        need = lib().inferno_moe_layer_workspace_bytes(C.byref(self.desc), T)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)

    def forward(self, x, residual=None, out=None, ids=None, weights=None):
        T = x.shape[0]
        self.reserve(T)
        if out is None:
            out = torch.empty(T, self.hidden, dtype=torch.float32, device=x.device)
        check(lib().inferno_moe_layer_forward(
            _s(), C.byref(self.desc), _p(_dev(x)), _DT[x.dtype], _p(residual), T, _p(out),
            _p(ids), _p(weights), _p(self._ws), self._ws.numel()))
        return out


class MoEStack:
    """Consecutive MoE layers on one residual stream (inferno_moe_stack_forward):
    for each layer, RMSNorm of the stream (rounded to ``act_dtype``), then
    stream += routed + shared expert outputs of the normalised activations."""

    def __init__(self, layers, norm_weights, eps=1e-6, act_dtype=torch.bfloat16, max_tokens=1):
        if len(layers) != len(norm_weights) or not layers:
            raise ValueError("one RMSNorm weight per layer is needed")
        self.layers = list(layers)
        self.norm_weights = list(norm_weights)
        self.eps, self.act_dtype = float(eps), act_dtype
        n = len(layers)
        self.descs = (LayerDesc * n)(*[l.desc for l in layers])
        self.norm_ptrs = (C.c_void_p * n)(*[w.data_ptr() for w in norm_weights])
        self.hidden = layers[0].hidden
        self.device = layers[0].device
        self._ws = None
        self.reserve(max_tokens)

    def reserve(self, T):
        need = lib().inferno_moe_stack_workspace_bytes(self.descs, len(self.layers), T)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)

    def forward(self, hidden, out=None, ids=None):
        """hidden: fp32 [T, H] residual stream. ids (optional int32 tensor of
        sum_l T*k_l) receives every layer's routing, layer after layer."""
        T = hidden.shape[0]
        self.reserve(T)
        if out is None:
            out = torch.empty(T, self.hidden, dtype=torch.float32, device=hidden.device)
        check(lib().inferno_moe_stack_forward(
            _s(), self.descs, len(self.layers), self.norm_ptrs, self.eps, _DT[self.act_dtype],
            _p(_dev(hidden)), T, _p(out), _p(ids), _p(self._ws), self._ws.numel()))
        return out


def layer_forward_noalloc(layer, x, residual=None, out=None, ids=None, weights=None):
    """``layer``'s forward through inferno_moe_layer_forward_noalloc: the
    library's fixed device scratch instead of a workspace (no allocation in
    the library; ``out`` is allocated here when not given)."""
    T = x.shape[0]
    if out is None:
        out = torch.empty(T, layer.hidden, dtype=torch.float32, device=x.device)
    check(lib().inferno_moe_layer_forward_noalloc(
        _s(), C.byref(layer.desc), _p(_dev(x)), _DT[x.dtype], _p(residual), T, _p(out), _p(ids),
        _p(weights)))
    return out
