"""ctypes binding of the C ABI in include/inferno_moe.h."""
import ctypes as C
from pathlib import Path

lib_path = Path(__file__).resolve().parent / "libinferno_moe.so"

F32, BF16 = 0, 1
Q8_0, Q2_K, Q3_K, Q4_K, Q6_K = 8, 10, 11, 12, 14
SCORE_SIGMOID, SCORE_SOFTMAX = 0, 1

_vp, _sz, _i, _f, _u64 = C.c_void_p, C.c_size_t, C.c_int, C.c_float, C.c_uint64


class InfernoError(RuntimeError):
    pass


class LayerDesc(C.Structure):
    """Mirror of `struct inferno_moe_layer`."""
    _fields_ = [
        ("hidden", _sz), ("experts", _sz), ("intermediate", _sz), ("top_k", _sz),
        ("quant", _i), ("down_quant", _i), ("score_fn", _i), ("norm_topk_prob", _i),
        ("routed_scaling_factor", _f),
        ("router", _vp), ("router_bias", _vp),
        ("gate", _vp), ("up", _vp), ("down", _vp),
        ("gate_bytes", _sz), ("up_bytes", _sz), ("down_bytes", _sz),
        ("shared_intermediate", _sz),
        ("shared_gate", _vp), ("shared_up", _vp), ("shared_down", _vp),
        ("shared_gate_bytes", _sz), ("shared_up_bytes", _sz), ("shared_down_bytes", _sz),
        ("shared_quant", _i), ("shared_down_quant", _i),
    ]


# name -> (restype, argtypes); every symbol the header declares.
SIGNATURES = {
    "inferno_last_error": (C.c_char_p, []),
    "inferno_block_bytes": (_i, [_i]),
    "inferno_block_values": (_i, [_i]),
    "inferno_stream_synchronize": (_i, [_vp]),
    "inferno_kernel_timing_enable": (_i, [_i]),
    "inferno_kernel_timing_read": (_i, [_i, C.POINTER(C.c_double), C.POINTER(C.c_uint64)]),
    "inferno_kernel_timing_label": (_i, [_i, C.c_char_p, C.c_size_t]),
    "inferno_gguf_dequantize": (_i, [_vp, _i, _vp, _sz, _vp]),
    "inferno_router_logits": (_i, [_vp, _vp, _i, _vp, _sz, _sz, _sz, _vp]),
    "inferno_moe_router_topk": (_i, [_vp, _vp, _vp, _sz, _sz, _sz, _i, _i, _f, _vp, _vp, _vp]),
    "inferno_moe_dispatch": (_i, [_vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp]),
    "inferno_gguf_moe_workspace_bytes": (_sz, [_sz, _sz, _sz, _sz, _sz]),
    "inferno_gguf_moe": (_i, [_vp, _i, _i, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _i, _vp, _vp,
                              _sz, _sz, _sz, _sz, _sz, _vp, _vp, _sz]),
    "inferno_gemv_workspace_bytes": (_sz, [_sz, _sz]),
    "inferno_moe_expert_gate_up_swiglu": (_i, [_vp, _i, _vp, _sz, _vp, _sz, _vp, _i, _vp, _vp,
                                               _vp, _vp, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _sz]),
    "inferno_moe_expert_down": (_i, [_vp, _i, _vp, _sz, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz,
                                     _sz, _vp, _vp, _sz]),
    "inferno_q8_0_gate_up_swiglu": (_i, [_vp, _vp, _sz, _vp, _sz, _vp, _i, _sz, _sz, _sz, _vp,
                                         _vp, _sz]),
    "inferno_q8_0_matvec_add2": (_i, [_vp, _vp, _sz, _vp, _vp, _vp, _sz, _sz, _sz, _vp, _vp,
                                      _sz]),
    "inferno_moe_topk_combine_residual": (_i, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "inferno_moe_weighted_index_add_combine": (_i, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "inferno_moe_gather_tokens": (_i, [_vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "inferno_rms_norm": (_i, [_vp, _vp, _vp, _sz, _sz, _f, _vp]),
    "inferno_rms_norm_router_topk_workspace_bytes": (_sz, [_sz]),
    "inferno_rms_norm_router_topk": (_i, [_vp, _vp, _vp, _f, _vp, _vp, _sz, _sz, _sz, _sz, _i, _i,
                                          _f, _i, _vp, _vp, _vp, _vp, _vp, _sz]),
    "inferno_moe_layer_workspace_bytes": (_sz, [C.POINTER(LayerDesc), _sz]),
    "inferno_moe_layer_forward": (_i, [_vp, C.POINTER(LayerDesc), _vp, _i, _vp, _sz, _vp, _vp,
                                       _vp, _vp, _sz]),
    "inferno_moe_layer_noalloc_max_bytes": (_sz, []),
    "inferno_moe_layer_forward_noalloc": (_i, [_vp, C.POINTER(LayerDesc), _vp, _i, _vp, _sz,
                                               _vp, _vp, _vp]),
    "inferno_moe_stack_workspace_bytes": (_sz, [C.POINTER(LayerDesc), _sz, _sz]),
    "inferno_moe_stack_forward": (_i, [_vp, C.POINTER(LayerDesc), _sz, C.POINTER(_vp), _f, _i,
                                       _vp, _sz, _vp, _vp, _vp, _sz]),
    "inferno_synth_normal": (_i, [_vp, _u64, _f, _sz, _i, _vp]),
    "inferno_synth_normal_host": (_i, [_u64, _f, _sz, _vp]),
    "inferno_quantize_rows_host": (_i, [_i, _vp, _sz, _sz, _vp]),
    "inferno_synth_quantized": (_i, [_vp, _i, _u64, _f, _sz, _sz, _vp]),
    "inferno_synth_quantized_host": (_i, [_i, _u64, _f, _sz, _sz, _vp]),
}
EXPORTED_SYMBOLS = tuple(SIGNATURES)

_LIB = None


def lib():
    """Loads the HIP library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not lib_path.exists():
            raise InfernoError(
                f"{lib_path} is missing: build it with `python -m inferno_amd._build` "
                "(there is no CPU fallback)")
        L = C.CDLL(str(lib_path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _LIB = L
    return _LIB


def check(status):
    if status != 0:
        msg = lib().inferno_last_error().decode()
        raise InfernoError(f"inferno status {status}: {msg}")
    return status
