"""The no-allocation layer entry point (inferno_moe_layer_forward_noalloc,
fixed device scratch) against inferno_moe_layer_forward with a caller
workspace: bit-identical outputs and routing, on two calls in a row, the
second with fewer tokens (the scratch keeps the first call's contents).
The no-alloc entry point keeps the shared expert and the router on the
grouped kernels (the library GEMMs allocate), so the workspace entry point
is run with INFERNO_SHARED_BLAS=0 for the bitwise comparison."""
import pytest
import torch

from inferno_amd import configs as cf
from inferno_amd import ops
from inferno_amd._lib import InfernoError, lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,T1,T2", [("c2", 16, 1), ("c4", 32, 1), ("c1", 16, 3)])
def test_noalloc_matches_workspace_entry_point(cuda, monkeypatch, name, T1, T2):
    monkeypatch.setenv("INFERNO_SHARED_BLAS", "0")
    cfg = cf.CONFIGS[name]
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=T1)
    k = cfg.top_k
    for v, T in enumerate((T1, T2)):
        x = cf.make_input(cfg, T, variant=v, device=cuda)
        residual = torch.randn(T, cfg.hidden, device=cuda)
        ids_a = torch.empty(T * k, dtype=torch.int32, device=cuda)
        w_a = torch.empty(T * k, device=cuda)
        ids_b = torch.empty_like(ids_a)
        w_b = torch.empty_like(w_a)
        want = lt.layer.forward(x, residual, ids=ids_a, weights=w_a)
        got = ops.layer_forward_noalloc(lt.layer, x, residual, ids=ids_b, weights=w_b)
        torch.cuda.synchronize()
        assert torch.equal(ids_a, ids_b) and torch.equal(w_a, w_b), (name, T)
        assert torch.equal(got, want), (name, T)
        print(f"{name} T={T}: no-alloc output identical to the workspace entry point")


def test_noalloc_rejects_shapes_beyond_its_scratch(cuda):
    cfg = cf.CONFIGS["c2"]
    lt = cf.build_layer(cfg, 0, cuda, max_tokens=1)
    T = 512
    assert lib().inferno_moe_layer_workspace_bytes(lt.layer.desc, T) > \
        lib().inferno_moe_layer_noalloc_max_bytes()
    x = cf.make_input(cfg, T, device=cuda)
    with pytest.raises(InfernoError, match="fixed maximum"):
        ops.layer_forward_noalloc(lt.layer, x)
