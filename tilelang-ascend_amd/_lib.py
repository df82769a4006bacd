"""ctypes binding of ``libdsa_mi355x.so`` (the C ABI declared in ``include/dsa_mi355x.h``).

The shared library is the only compute path: if it is missing, or a tensor is
not on a HIP device, the call raises -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

import torch

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libdsa_mi355x.so"

KIND_FP8_E4M3 = 0
KIND_BF16 = 1
KIND_FP16 = 2
KIND_FP32 = 3
KIND_INT8 = 4

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_vp = ctypes.c_void_p
_c_size = ctypes.c_size_t
_c_float = ctypes.c_float

# name -> (restype, argtypes); must match include/dsa_mi355x.h
SIGNATURES = {
    "dsa_abi_version": (_c_int, []),
    "dsa_last_error_message": (ctypes.c_char_p, []),
    "dsa_topk_select": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_int, _c_vp, _c_vp, _c_vp]),
    "dsa_topk_select_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "dsa_topk_select_ws": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_int, _c_vp, _c_vp, _c_vp, _c_size,
                                    _c_vp]),
    "dsa_indexer_logits": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                    _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_int, _c_vp, _c_i64, _c_vp]),
    "dsa_lightning_indexer_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "dsa_lightning_indexer": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                       _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_int, _c_i64, _c_vp, _c_vp, _c_vp,
                                       _c_size, _c_vp]),
    "dsa_lightning_indexer_fused_applies": (_c_int, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "dsa_lightning_indexer_fused_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "dsa_lightning_indexer_fused": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64,
                                             _c_i64, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_int, _c_i64, _c_vp,
                                             _c_vp, _c_vp, _c_size, _c_vp]),
    "dsa_lightning_indexer_fused_fallback_rows": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp]),
    "dsa_indexer_logits_tnd": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                        _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_int, _c_vp, _c_i64,
                                        _c_vp]),
    "dsa_lightning_indexer_tnd_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "dsa_lightning_indexer_tnd": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                           _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_int, _c_i64, _c_vp,
                                           _c_vp, _c_vp, _c_size, _c_vp]),
    "dsa_lightning_indexer_tnd_fused_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "dsa_lightning_indexer_tnd_fused": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64,
                                                 _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_int,
                                                 _c_i64, _c_vp, _c_vp, _c_vp, _c_size, _c_vp]),
    "dsa_sparse_flash_mla_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "dsa_sparse_flash_mla": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp,
                                      _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp,
                                      _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_float, _c_vp, _c_vp, _c_vp, _c_size,
                                      _c_vp]),
    "dsa_sparse_attn_sink_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "dsa_sparse_attn_sink": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                      _c_vp, _c_float, _c_vp, _c_vp, _c_vp, _c_size, _c_vp]),
    "dsa_act_quant": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_int, _c_vp, _c_vp, _c_int, _c_vp]),
    "dsa_sparse_mla_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "dsa_sparse_mla_fwd": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64,
                                    _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_float, _c_int, _c_vp, _c_vp, _c_vp,
                                    _c_size, _c_vp]),
    "dsa_sparse_mla_noalloc_max_workspace": (_c_size, []),
    "dsa_sparse_mla_fwd_noalloc": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
                                            _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_float, _c_int, _c_vp,
                                            _c_vp, _c_vp]),
    "dsa_sparse_attention_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "dsa_sparse_attention_fwd": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
                                          _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_float, _c_int,
                                          _c_vp, _c_vp, _c_vp, _c_size, _c_vp]),
}

_lib: Optional[ctypes.CDLL] = None


class DSAError(RuntimeError):
    """A C-ABI call returned a non-zero hipError_t."""


def library_path() -> Path:
    return Path(os.environ.get("DSA_MI355X_LIB", str(LIB_PATH)))


def load_library() -> ctypes.CDLL:
    """Load the HIP library once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise ImportError(
            f"{path} is missing: build it with `python tilelang-ascend_amd/build.py` "
            "(or __graft_entry__.build()); there is no fallback path")
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


TORCH_OPS_PATH = PKG_DIR / "libdsa_torch_ops.so"
_torch_ops_loaded = False


def load_torch_ops():
    """Register ``torch.ops.dsa.*`` (loads libdsa_torch_ops.so once) and return the namespace."""
    global _torch_ops_loaded
    if not _torch_ops_loaded:
        load_library()
        if not TORCH_OPS_PATH.exists():
            raise ImportError(f"{TORCH_OPS_PATH} is missing: build it with `python tilelang-ascend_amd/build.py`")
        torch.ops.load_library(str(TORCH_OPS_PATH))
        _torch_ops_loaded = True
    return torch.ops.dsa


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load_library().dsa_last_error_message()
        msg = msg.decode() if msg else ""
        raise DSAError(f"{what} failed with hipError {rc}: {msg}")


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_device(*tensors: Optional[torch.Tensor]) -> torch.device:
    """All given tensors must sit on one HIP device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"tensors must be on a HIP (cuda) device, got {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors must be on one device, got {dev} and {t.device}")
    if dev is None:
        raise ValueError("no device tensor given")
    return dev


def require_contiguous(name: str, t: torch.Tensor) -> None:
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
