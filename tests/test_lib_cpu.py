"""The C-ABI library loads on a CPU-only host and exports exactly what include/pmoe.h declares.

No compute is launched here: only workspace-size queries and argument
rejections, which return before any HIP call.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "pmoe.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"PMOE_API\s+[\w\s\*]+?\b(pmoe_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from pluggy_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.fail("libpmoe.so is not built (run python -m pluggy_amd.build / __graft_entry__.build())")
    return _lib.load()


def test_header_declares_the_entry_points():
    syms = declared_symbols()
    assert len(syms) >= 20
    for name in ("pmoe_router_forward", "pmoe_router_backward", "pmoe_permute", "pmoe_dispatch",
                 "pmoe_gate_up_swiglu", "pmoe_down_proj", "pmoe_combine", "pmoe_expert_ffn_forward",
                 "pmoe_expert_ffn_backward"):
        assert name in syms


def test_library_exports_every_declared_symbol(lib):
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_table_matches_header():
    from pluggy_amd import _lib

    assert sorted(_lib.SIGNATURES) == declared_symbols()


def test_version_and_workspace_queries(lib):
    assert lib.pmoe_version().startswith(b"pmoe")
    from pluggy_amd import _lib

    # backward workspace holds grad_y (P*H) and grad_gate_up_out (P*2I) in bf16
    P, H, I = 8192 * 8, 2048, 768
    assert _lib.size("pmoe_expert_ffn_backward_workspace_size", 8192, 8, H, I, 1) >= P * H * 2 + P * 2 * I * 2
    assert _lib.size("pmoe_permute_workspace_size", 8192, 8, 128) >= 32 * 128 * 4
    assert _lib.size("pmoe_router_forward_workspace_size", 0, 2048, 128) >= 3 * 128 * 2048 * 2


@pytest.mark.parametrize("args,needle", [
    ((None, 10, 9, 8), b"exceeds num_experts"),       # K > E
    ((None, 10, 2, 2000), b"> 1024"),                  # too many experts
    ((None, 10, 70, 100), b"top_k=70 > 64"),
])
def test_permute_rejects_bad_arguments(lib, args, needle):
    rc = lib.pmoe_permute(*args, None, None, None, None, None, 0, None)
    assert rc == -1
    assert needle in lib.pmoe_last_error_string()


def test_gemm_rejects_unaligned_hidden(lib):
    from pluggy_amd import _lib

    rc = lib.pmoe_down_proj(None, None, None, _lib.PMOE_BF16, 64, 8, 100, 64, None, None)
    assert rc == -1 and b"multiple of 8" in lib.pmoe_last_error_string()


def test_workspace_too_small_is_rejected(lib):
    rc = lib.pmoe_permute(ctypes.c_void_p(16), 100, 2, 8, ctypes.c_void_p(16), ctypes.c_void_p(16),
                          ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), 4, None)
    assert rc == -3 and b"workspace" in lib.pmoe_last_error_string()


def test_product_path_has_no_cpu_fallback():
    import torch

    import pluggy_amd

    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pluggy_amd.moe_expert_ffn(torch.zeros(4, 8), torch.zeros(4, 1, dtype=torch.int64), torch.ones(4, 1),
                                  torch.zeros(2, 16, 8), torch.zeros(2, 8, 8))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pluggy_amd.router_topk(torch.zeros(4, 8), torch.zeros(2, 8), 1)


def test_product_package_does_not_import_the_oracle():
    for path in (ROOT / "pluggy_amd").rglob("*.py"):
        src = path.read_text()
        assert "import oracle" not in src and "from oracle" not in src, path


@pytest.mark.parametrize("entry", ["pmoe_down_proj_backward", "pmoe_gate_up_backward"])
def test_weight_gradient_dtype_is_checked(lib, entry):
    """fp32 operands cannot write bf16 weight gradients; bf16 operands may write fp32 ones."""
    from pluggy_amd import _lib

    P, E, H, I = 64, 4, 64, 32
    if entry == "pmoe_down_proj_backward":  # grad, row_index, row_weight, grad_rows, mid, gate_up_out, down, offs
        lead = (None, None, None, P, None, None, None, None)
        tail = (None, None, _lib.PMOE_BF16, None, 0, None)
    else:  # grad_gate_up_out, x, row_index, x_rows, gate_up_proj, offs
        lead = (None, None, None, P, None, None)
        tail = (None, None, _lib.PMOE_BF16, None)
    rc = getattr(lib, entry)(*lead, _lib.PMOE_F32, P, E, H, I, *tail)
    assert rc == -1 and b"dtype must be the operands' or fp32" in lib.pmoe_last_error_string()



def test_noalloc_forward_rejects_sizes_beyond_its_static_scratch(lib):
    """The allocation-free forward refuses, before any HIP call, a pair count
    whose permutation histograms exceed its 256 KiB static scratch."""
    from pluggy_amd import _lib

    T, K, E, H, I = 131073, 8, 128, 64, 32  # 513 chunks x 128 experts x 4 bytes > 256 KiB
    dev = ctypes.c_void_p(256)  # the routing weights must be given; never dereferenced here
    outs = [None] * 10
    outs[6] = dev  # sorted_w
    with pytest.raises(RuntimeError, match="static maximum"):
        _lib.call("pmoe_expert_ffn_forward_noalloc", None, None, dev, _lib.PMOE_F32, None, None, _lib.PMOE_BF16,
                  T, K, E, H, I, *outs, None)


def test_expert_ffn_requires_the_routing_weights(lib):
    """The routing weights reach the output only through sorted_w (the SwiGLU
    epilogue scales each sorted row; the combine is unweighted), so the C-ABI
    forward and backward refuse NULL top_weights / sorted_w before any launch
    instead of returning the unweighted sum or its gradients."""
    from pluggy_amd import _lib

    T, K, E, H, I = 64, 2, 8, 64, 32
    dev = ctypes.c_void_p(256)  # never dereferenced: the argument check returns first
    fwd = lambda top_w, sorted_w: lib.pmoe_expert_ffn_forward(  # noqa: E731
        dev, dev, top_w, _lib.PMOE_F32, dev, dev, _lib.PMOE_BF16, T, K, E, H, I, dev, dev, dev, dev, dev, dev,
        sorted_w, dev, dev, dev, dev, 1 << 20, None)
    for top_w, sorted_w in ((None, dev), (dev, None), (None, None)):
        assert fwd(top_w, sorted_w) == -1
        assert b"top_weights and sorted_w are required" in lib.pmoe_last_error_string()
    rc = lib.pmoe_expert_ffn_forward_noalloc(dev, dev, dev, _lib.PMOE_F32, dev, dev, _lib.PMOE_BF16, T, K, E, H, I,
                                            dev, dev, dev, dev, dev, dev, None, dev, dev, dev, None)
    assert rc == -1 and b"top_weights and sorted_w are required" in lib.pmoe_last_error_string()
    rc = lib.pmoe_expert_ffn_backward(dev, dev, _lib.PMOE_F32, dev, dev, _lib.PMOE_BF16, T, K, E, H, I, dev, dev,
                                      dev, None, dev, dev, dev, dev, dev, dev, _lib.PMOE_BF16, dev, 1 << 30, None)
    assert rc == -1 and b"sorted_w (the routing weight of each sorted row) is required" in lib.pmoe_last_error_string()


# PMOE_GEMM_* kinds: gate_up fwd, down fwd, down dgrad, down wgrad, gate_up dgrad, gate_up wgrad
_KINDS = range(6)


@pytest.mark.parametrize("cus,ep_share", [
    (256, [256, 256, 128, 256, 256, 256]),   # MI355X
    (304, [256, 128, 128, 256, 128, 256]),   # a 304-CU part: two rounds either way for down fwd / gate_up dgrad
])
def test_expert_gemm_tile_rows(lib, cus, ep_share):
    """The grouped-GEMM engine's tile choice (host-only query, no launch): the
    benchmark layers take 256-row tiles in every GEMM; one GPU's share at EP=8
    of config 2 takes 128-row tiles where that keeps the number of rounds of
    tiles per CU (each 128-row tile about 0.75 of a 256-row one): on 256 CUs
    down dgrad only; the decode batch's forward GEMMs take the 32-row
    few-token tiles; fp32 operands take the register-staged engine's 64-row
    tiles."""
    from pluggy_amd import _lib

    bf, f32 = _lib.PMOE_BF16, _lib.PMOE_F32
    rows = lambda kind, P, E, H, I, dt=bf: lib.pmoe_expert_gemm_tile_rows(kind, P, E, H, I, dt, cus)  # noqa: E731
    for P, E, H, I in ((65536, 128, 2048, 768), (131072, 128, 4096, 1536)):  # configs 2 / 4 and 3
        assert [rows(k, P, E, H, I) for k in _KINDS] == [256] * 6
    assert [rows(k, 8326, 16, 2048, 768) for k in _KINDS] == ep_share
    assert [rows(k, 512, 128, 2048, 768) for k in _KINDS] == [32, 32, 256, 256, 256, 256]
    assert rows(0, 4096, 8, 512, 1024, f32) == 64
    assert lib.pmoe_expert_gemm_tile_rows(7, 100, 8, 64, 64, bf, cus) == -1
