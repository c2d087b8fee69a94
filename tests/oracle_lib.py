"""ctypes binding of the CPU oracle (oracle/liboracle.so) — test-only checker."""
import ctypes as C
from pathlib import Path

import numpy as np

_PATH = Path(__file__).resolve().parent.parent / "oracle" / "liboracle.so"
_L = None
_vp, _sz, _i, _f = C.c_void_p, C.c_size_t, C.c_int, C.c_float

_SIG = {
    "oracle_f16_to_f32": (_f, [C.c_uint16]),
    "oracle_block_bytes": (_i, [_i]),
    "oracle_block_values": (_i, [_i]),
    "oracle_dequantize": (_i, [_i, _vp, _sz, _vp]),
    "oracle_linear": (_i, [_vp, _vp, _sz, _sz, _sz, _vp, _i]),
    "oracle_router_topk": (_i, [_vp, _vp, _sz, _sz, _sz, _i, _i, _f, _vp, _vp]),
    "oracle_dispatch": (_i, [_vp, _sz, _sz, _sz, _vp, _vp]),
    "oracle_qmatvec": (_i, [_i, _vp, _sz, _sz, _vp, _vp]),
    "oracle_moe_routed": (_i, [_i, _i, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _vp, _vp,
                               _vp, _i]),
    "oracle_shared_q8_0": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp, _i]),
    "oracle_shared_ffn": (_i, [_i, _i, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp, _i]),
    "oracle_weighted_index_add_combine": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "oracle_rms_norm": (_i, [_vp, _vp, _sz, _sz, _f, _vp]),
}

import os as _os

try:
    THREADS = max(1, min(16, len(_os.sched_getaffinity(0))))
except AttributeError:
    THREADS = 8


def L():
    global _L
    if _L is None:
        lib = C.CDLL(str(_PATH))
        for n, (r, a) in _SIG.items():
            getattr(lib, n).restype = r
            getattr(lib, n).argtypes = a
        _L = lib
    return _L


def _p(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _ok(st, what):
    if st != 0:
        raise ValueError(f"oracle {what} failed: {st}")


def dequantize(quant, blocks):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    n = blocks.size // L().oracle_block_bytes(quant)
    out = np.empty(n * L().oracle_block_values(quant), np.float32)
    _ok(L().oracle_dequantize(quant, _p(blocks), n, _p(out)), "dequantize")
    return out


def linear(x, w):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty((x.shape[0], w.shape[0]), np.float32)
    _ok(L().oracle_linear(_p(x), _p(w), x.shape[0], x.shape[1], w.shape[0], _p(out), THREADS),
        "linear")
    return out


def router_topk(logits, bias, k, score_fn, norm, scale):
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    ids = np.empty(T * k, np.uint32)
    w = np.empty(T * k, np.float32)
    _ok(L().oracle_router_topk(_p(logits), _p(b), T, E, k, score_fn, int(norm), scale, _p(ids),
                               _p(w)), "router_topk")
    return ids, w


def dispatch(ids, T, k, E):
    ids = np.ascontiguousarray(ids, np.uint32)
    off = np.empty(E + 1, np.uint32)
    srt = np.empty(max(T * k, 1), np.uint32)
    _ok(L().oracle_dispatch(_p(ids), T, k, E, _p(off), _p(srt)), "dispatch")
    return off, srt[: T * k]


def qmatvec(quant, w, rows, cols, x):
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    _ok(L().oracle_qmatvec(quant, _p(w), rows, cols, _p(x), _p(y)), "qmatvec")
    return y


def moe_routed(quant, down_quant, gate, up, down, x, ids, w, E, k, I):
    x = np.ascontiguousarray(x, np.float32)
    T, H = x.shape
    y = np.empty((T, H), np.float32)
    gate, up, down = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
    ids = np.ascontiguousarray(ids, np.uint32)
    w = np.ascontiguousarray(w, np.float32)
    _ok(L().oracle_moe_routed(quant, down_quant, _p(gate), _p(up), _p(down), _p(x), T, H, I, E, k,
                              _p(ids), _p(w), _p(y), THREADS), "moe_routed")
    return y


def shared_q8_0(gate, up, down, x, Is, routed=None, residual=None):
    x = np.ascontiguousarray(x, np.float32)
    T, H = x.shape
    out = np.empty((T, H), np.float32)
    r = None if routed is None else np.ascontiguousarray(routed, np.float32)
    s = None if residual is None else np.ascontiguousarray(residual, np.float32)
    gate, up, down = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
    _ok(L().oracle_shared_q8_0(_p(gate), _p(up), _p(down), _p(x), T, H, Is, _p(r), _p(s),
                               _p(out), THREADS), "shared_q8_0")
    return out


def shared_ffn(quant, down_quant, gate, up, down, x, Is, routed=None, residual=None):
    """Shared expert of any format (Q8_0 GLM / Laguna S; Q4_K + Q4_K/Q6_K XS)."""
    x = np.ascontiguousarray(x, np.float32)
    T, H = x.shape
    out = np.empty((T, H), np.float32)
    r = None if routed is None else np.ascontiguousarray(routed, np.float32)
    s = None if residual is None else np.ascontiguousarray(residual, np.float32)
    gate, up, down = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
    _ok(L().oracle_shared_ffn(quant, down_quant, _p(gate), _p(up), _p(down), _p(x), T, H, Is,
                              _p(r), _p(s), _p(out), THREADS), "shared_ffn")
    return out


def weighted_index_add_combine(acc, tok, y, w):
    acc = np.ascontiguousarray(acc, np.float32)
    T, H = acc.shape
    out = np.empty_like(acc)
    tok = np.ascontiguousarray(tok, np.uint32)
    y = np.ascontiguousarray(y, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    _ok(L().oracle_weighted_index_add_combine(_p(acc), _p(tok), _p(y), _p(w), T, H, len(tok),
                                              _p(out)), "combine")
    return out


def rms_norm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    w = np.ascontiguousarray(w, np.float32)
    _ok(L().oracle_rms_norm(_p(x), _p(w), x.shape[0], x.shape[1], eps, _p(out)), "rms_norm")
    return out


def moe_layer(cfg_quant, cfg_down, router, bias, gate, up, down, x, k, E, I, score_fn, norm,
              scale, shared=None, Is=0, residual=None):
    """Whole layer on the CPU: logits -> top-k -> routed -> (+shared) + residual."""
    logits = linear(x, router)
    ids, w = router_topk(logits, bias, k, score_fn, norm, scale)
    routed = moe_routed(cfg_quant, cfg_down, gate, up, down, x, ids, w, E, k, I)
    if shared is not None:
        out = shared_q8_0(*shared, x, Is, routed=routed, residual=residual)
    else:
        out = routed + (0 if residual is None else residual)
    return out, ids, w, logits
