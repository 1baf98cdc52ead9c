"""ctypes binding of ``libpmoe.so`` (the C ABI declared in ``include/pmoe.h``).

The library is loaded from the package directory. There is no fallback: when
the library is missing, or a tensor is not on a ROCm device, calls raise.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libpmoe.so")

PMOE_F32 = 0
PMOE_BF16 = 1
PMOE_F16 = 2
PMOE_BF16X3 = 3  # an fp32 router weight given as its bf16 pieces (pmoe_router_split_weight)

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_SZ = ctypes.c_size_t
_F32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/pmoe.h
SIGNATURES = {
    "pmoe_version": (ctypes.c_char_p, []),
    "pmoe_last_error_string": (ctypes.c_char_p, []),
    "pmoe_router_forward_workspace_size": (_SZ, [_I64, _I64, _I64]),
    "pmoe_router_forward": (_INT, [_P, _INT, _P, _INT, _P, _I64, _I64, _I64, _I64, _INT, _P, _P, _INT, _P, _P, _P,
                                   _P, _P, _P, _SZ, _P]),
    "pmoe_router_backward_workspace_size": (_SZ, [_I64, _I64, _I64]),
    "pmoe_router_split_weight": (_INT, [_P, _I64, _I64, _P, _P]),
    "pmoe_router_backward": (_INT, [_P, _INT, _P, _INT, _P, _P, _P, _P, _INT, _P, _I64, _I64, _I64, _I64, _INT, _P,
                                    _P, _P, _SZ, _P]),
    "pmoe_permute_workspace_size": (_SZ, [_I64, _I64, _I64]),
    "pmoe_permute": (_INT, [_P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _SZ, _P]),
    "pmoe_count_invalid_ids": (_INT, [_P, _I64, _I64, _P, _P]),
    "pmoe_dispatch": (_INT, [_P, _INT, _P, _I64, _I64, _I64, _P, _P]),
    "pmoe_sort_rows": (_INT, [_P, _P, _INT, _I64, _I64, _P, _P, _P]),
    "pmoe_permute_rows": (_INT, [_P, _P, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "pmoe_gate_up_swiglu": (_INT, [_P, _P, _P, _I64, _P, _P, _INT, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "pmoe_down_proj": (_INT, [_P, _P, _P, _INT, _I64, _I64, _I64, _I64, _P, _P]),
    "pmoe_combine": (_INT, [_P, _P, _INT, _P, _INT, _I64, _I64, _I64, _P, _P]),
    "pmoe_combine_backward": (_INT, [_P, _P, _P, _INT, _P, _INT, _I64, _I64, _I64, _P, _P, _P]),
    "pmoe_down_proj_backward": (_INT, [_P, _P, _P, _I64, _P, _P, _P, _P, _INT, _I64, _I64, _I64, _I64, _P, _P,
                                       _INT, _P, _I64, _P]),
    "pmoe_gate_up_backward": (_INT, [_P, _P, _P, _I64, _P, _P, _INT, _I64, _I64, _I64, _I64, _P, _P, _INT, _P]),
    "pmoe_pair_weight_grad": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _P, _INT, _P]),
    "pmoe_dispatch_backward": (_INT, [_P, _P, _P, _INT, _I64, _I64, _I64, _P, _P]),
    "pmoe_rmsnorm_forward": (_INT, [_P, _INT, _P, _F32, _I64, _I64, _P, _INT, _P, _P]),
    "pmoe_combine_residual": (_INT, [_P, _P, _INT, _P, _INT, _P, _INT, _I64, _I64, _I64, _P, _P]),
    "pmoe_combine_residual_backward": (_INT, [_P, _INT, _P, _P, _INT, _P, _INT, _I64, _I64, _I64, _P, _P, _P]),
    "pmoe_dispatch_rmsnorm_backward_workspace_size": (_SZ, [_I64, _I64]),
    "pmoe_dispatch_rmsnorm_backward": (_INT, [_P, _P, _P, _INT, _P, _INT, _P, _P, _P, _I64, _I64, _I64, _P, _P,
                                              _INT, _P, _SZ, _P]),
    "pmoe_expert_ffn_forward_workspace_size": (_SZ, [_I64, _I64, _I64]),
    "pmoe_expert_ffn_forward": (_INT, [_P, _P, _P, _INT, _P, _P, _INT, _I64, _I64, _I64, _I64, _I64, _P, _P, _P,
                                       _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "pmoe_expert_ffn_forward_noalloc": (_INT, [_P, _P, _P, _INT, _P, _P, _INT, _I64, _I64, _I64, _I64, _I64, _P,
                                               _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "pmoe_expert_ffn_backward_workspace_size": (_SZ, [_I64, _I64, _I64, _I64, _INT]),
    "pmoe_expert_gemm_tile_rows": (_INT, [_INT, _I64, _I64, _I64, _I64, _INT, _INT]),
    "pmoe_expert_ffn_backward": (_INT, [_P, _P, _INT, _P, _P, _INT, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P,
                                        _P, _P, _P, _P, _P, _P, _INT, _P, _SZ, _P]),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load and declare ``libpmoe.so``; raises RuntimeError when it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"pmoe HIP library not found at {LIB_PATH}; build it with `python -m pluggy_amd.build`")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise RuntimeError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.pmoe_last_error_string().decode(errors="replace")
        raise RuntimeError(f"{name} failed (status {rc}): {msg}")


def size(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return PMOE_BF16
    if dt == torch.float32:
        return PMOE_F32
    if dt == torch.float16:
        return PMOE_F16
    raise TypeError(f"pmoe supports bf16, fp16 and fp32 tensors, got {dt}")


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor):
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("pluggy_amd runs on ROCm GPU tensors only (there is no CPU fallback); "
                               f"got a tensor on {t.device}")


def workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(1, nbytes), dtype=torch.uint8, device=device)
