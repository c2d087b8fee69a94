"""CPU-side checks of the product library: it loads without a GPU, exports
every symbol include/inferno_moe.h declares, and its host-side helpers
(block geometry, generator, quantiser) behave."""
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle_lib as orc
from inferno_amd import EXPORTED_SYMBOLS, lib, ops
from inferno_amd._lib import Q2_K, Q3_K, Q4_K, Q6_K, Q8_0

HEADER = Path(__file__).resolve().parent.parent / "include" / "inferno_moe.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(inferno_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = lib()
    names = declared_symbols()
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), n
    assert sorted(EXPORTED_SYMBOLS) == names


def test_block_geometry():
    L = lib()
    assert [L.inferno_block_bytes(q) for q in (Q2_K, Q3_K, Q4_K, Q6_K, Q8_0)] == [84, 110, 144, 210, 34]
    assert L.inferno_block_values(Q8_0) == 32 and L.inferno_block_values(Q2_K) == 256
    assert L.inferno_block_bytes(99) == -1


def test_error_paths_without_gpu():
    # argument validation happens before any device work (crates/backend/src/metal/moe.rs:582-623)
    L = lib()
    st = L.inferno_moe_router_topk(None, None, None, 1, 8, 0, 0, 1, 1.0, None, None, None)
    assert st < 0 and b"1..=16" in L.inferno_last_error()
    st = L.inferno_moe_router_topk(None, None, None, 1, 300, 8, 0, 1, 1.0, None, None, None)
    assert st < 0 and b"256" in L.inferno_last_error()
    st = L.inferno_gguf_moe(None, Q2_K, Q2_K, None, 84, None, 84, None, 84, None, 0, None, None,
                            1, 1, 1, 250, 256, None, None, 0)
    assert st < 0 and b"256-wide" in L.inferno_last_error()
    st = L.inferno_gguf_moe(None, Q2_K, Q2_K, None, 83, None, 84, None, 84, None, 0, None, None,
                            1, 1, 1, 256, 256, None, None, 0)
    assert st == -2 and b"gate expert payload" in L.inferno_last_error()
    st = L.inferno_gguf_moe(None, Q8_0, Q2_K, None, 0, None, 0, None, 0, None, 0, None, None,
                            1, 1, 1, 256, 256, None, None, 0)
    assert st < 0


def test_valid_call_without_a_device_is_unsupported():
    # the reference's Ok(None) when no native device backs the backend
    # (crates/backend/src/backend.rs:6688-6692): INFERNO_UNSUPPORTED (1), after
    # argument validation; nothing is launched
    if torch.cuda.is_available():
        pytest.skip("a GPU is present: the call would run")
    import ctypes as C
    L = lib()
    x = C.c_void_p(16)  # never dereferenced: no device to launch on
    st = L.inferno_rms_norm(None, x, x, 1, 64, 1e-6, x)
    assert st == 1 and b"no HIP device" in L.inferno_last_error()
    st = L.inferno_rms_norm(None, x, x, 1, 0, 1e-6, x)  # invalid arguments still come first
    assert st == -1


def test_synth_normal_host_statistics_and_determinism():
    a = ops.synth_normal_host(5, 1.0, 200000).numpy()
    b = ops.synth_normal_host(5, 1.0, 200000).numpy()
    assert np.array_equal(a, b)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    c = ops.synth_normal_host(6, 1.0, 1000).numpy()
    assert not np.array_equal(a[:1000], c)


@pytest.mark.parametrize("quant,tol", [(Q2_K, 0.45), (Q3_K, 0.30), (Q4_K, 0.12), (Q6_K, 0.03),
                                       (Q8_0, 0.01)])
def test_host_quantiser_roundtrip(quant, tol):
    rows, cols = 16, 1024
    x = torch.randn(rows, cols) * 0.02
    q = ops.quantize_rows_host(quant, x).numpy()
    back = orc.dequantize(quant, q).reshape(rows, cols)
    err = np.linalg.norm(back - x.numpy()) / np.linalg.norm(x.numpy())
    assert err < tol, err


def test_synth_quantized_host_is_quantised_normal():
    q = ops.synth_quantized_host(Q4_K, 9, 0.02, 4, 512).numpy()
    x = ops.synth_normal_host(9, 0.02, 4 * 512).numpy()
    back = orc.dequantize(Q4_K, q)
    assert np.linalg.norm(back - x) / np.linalg.norm(x) < 0.12


def test_norm_router_argument_errors_without_gpu():
    # the fused RMSNorm -> router -> top-k entry point validates before any
    # device work: unsupported widths are Ok(None)-style (1), a missing
    # workspace with the top-k an error, a valid call without a device 1
    import ctypes as C
    L = lib()
    x = C.c_void_p(16)
    ids = C.c_void_p(32)
    st = L.inferno_rms_norm_router_topk(None, x, x, 1e-6, x, None, 1, 24, 64, 8, 0, 1, 1.0, 0,
                                        None, x, None, None, None, 0)
    assert st == 1 and b"multiple of 64" in L.inferno_last_error()
    st = L.inferno_rms_norm_router_topk(None, x, x, 1e-6, x, None, 1, 2048, 64, 8, 0, 1, 1.0, 0,
                                        None, x, ids, ids, x, 0)
    assert st == -2 and b"workspace too small" in L.inferno_last_error()
    st = L.inferno_rms_norm_router_topk(None, x, x, 1e-6, x, None, 1, 2048, 64, 8, 7, 1, 1.0, 0,
                                        None, x, None, None, None, 0)
    assert st == -1
    assert L.inferno_rms_norm_router_topk_workspace_bytes(3) == 256
    if not torch.cuda.is_available():
        st = L.inferno_rms_norm_router_topk(None, x, x, 1e-6, x, None, 1, 2048, 64, 8, 0, 1, 1.0,
                                            0, None, x, None, None, None, 0)
        assert st == 1 and b"no HIP device" in L.inferno_last_error()
