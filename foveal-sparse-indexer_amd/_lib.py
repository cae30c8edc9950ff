"""ctypes binding of libfsi_amd.so (the C ABI in include/fsi.h) plus the host
plumbing every op shares: device checks, stream handles, workspaces, status
codes -> Python exceptions.

There is no CPU path: every op requires its tensors on a ROCm GPU and raises if
the HIP library is not built or not loadable.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libfsi_amd.so"

FSI_OK = 0
FSI_ERR_INVALID_ARG = -1
FSI_ERR_SHAPE = -2
FSI_ERR_INDEX_RANGE = -3
FSI_ERR_CAPACITY = -4
FSI_ERR_DTYPE = -5
FSI_ERR_HIP = -6
FSI_ERR_ALIGN = -7
FSI_ERR_WORKSPACE = -8

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2  # fsi_sram_indexer_attention only

ACTIVATIONS = {"swiglu": 0, "silu": 1, "gelu": 2, "relu": 3, "relu2": 4}
ROUNDING = {"eager": 0, "fused": 1, "fp32": 2}

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_ptr = ctypes.c_void_p
_c_size = ctypes.c_size_t

# Every exported symbol with its (restype, argtypes).  Kept in the same order as include/fsi.h.
SIGNATURES: dict[str, tuple] = {
    "fsi_abi_version": (_c_int, []),
    "fsi_status_string": (ctypes.c_char_p, [_c_int]),
    "fsi_last_error": (ctypes.c_char_p, []),
    "fsi_pattention_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "fsi_pattention_fwd": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_int, _c_ptr, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_ptr, _c_i64, _c_ptr, _c_size, _c_ptr, _c_ptr],
    ),
    "fsi_pattention_packed_size": (_c_size, [_c_i64, _c_i64, _c_i64]),
    "fsi_pattention_pack": (
        _c_int,
        [_c_ptr, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr, _c_size,
         _c_ptr],
    ),
    "fsi_pattention_packed_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "fsi_pattention_fwd_packed": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_ptr,
         _c_i64, _c_ptr, _c_size, _c_ptr, _c_ptr],
    ),
    "fsi_swiglu": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_int, _c_int, _c_ptr]),
    "fsi_swiglu_bwd": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_int, _c_ptr]),
    "fsi_mlp_router_workspace_size": (_c_size, [_c_i64, _c_i64]),
    "fsi_mlp_router": (
        _c_int,
        [_c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_int,
         _c_ptr, _c_ptr, _c_ptr, _c_size, _c_ptr],
    ),
    "fsi_masked_softmax": (
        _c_int, [_c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "fsi_masked_softmax_bwd": (
        _c_int, [_c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "fsi_route_from_scores": (
        _c_int,
        [_c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_int, ctypes.c_float, _c_int, _c_int, _c_int, _c_ptr,
         _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr],
    ),
    "fsi_score_and_route": (
        _c_int,
        [_c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, ctypes.c_float, _c_int,
         _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr],
    ),
    "fsi_decode_route": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64,
         ctypes.c_float, _c_int, _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr],
    ),
    "fsi_index_rms_norm": (_c_int, [_c_ptr, _c_int, _c_i64, _c_i64, _c_ptr, _c_ptr]),
    "fsi_index_pool_kv": (_c_int, [_c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr]),
    "fsi_kv_page_pool": (
        _c_int, [_c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_ptr],
    ),
    "fsi_block_scores": (_c_int, [_c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr]),
    "fsi_additive_context": (
        _c_int, [_c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr, _c_ptr],
    ),
    "fsi_dense_block_targets_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "fsi_dense_block_targets": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float,
         _c_ptr, _c_i64, _c_ptr, _c_size, _c_ptr],
    ),
    "fsi_index_rms_norm_bwd": (_c_int, [_c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_ptr, _c_ptr]),
    "fsi_index_pool_kv_bwd": (
        _c_int, [_c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr],
    ),
    "fsi_block_scores_bwd": (
        _c_int, [_c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr],
    ),
    "fsi_additive_context_bwd_workspace_size": (_c_size, [_c_i64, _c_i64]),
    "fsi_additive_context_bwd": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_size,
         _c_ptr],
    ),
    "fsi_distill_kl_workspace_size": (_c_size, [_c_i64, _c_i64]),
    "fsi_distill_kl_fwd": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr, _c_i64, _c_i64, _c_i64,
         ctypes.c_float, _c_ptr, _c_ptr, _c_ptr, _c_size, _c_ptr],
    ),
    "fsi_distill_kl_bwd": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr, _c_i64, _c_i64, _c_i64,
         ctypes.c_float, _c_ptr, _c_ptr, _c_ptr, _c_ptr],
    ),
    "fsi_kv_write": (
        _c_int,
        [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr,
         _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr],
    ),
    "fsi_kv_read": (
        _c_int, [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr],
    ),
    "fsi_decode_attn_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "fsi_decode_attn": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_ptr, _c_ptr, _c_size, _c_ptr, _c_ptr],
    ),
    "fsi_decode_step_attn": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, ctypes.c_float, _c_int, _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr,
         _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         ctypes.c_float, _c_int, _c_ptr, _c_ptr, _c_size, _c_ptr, _c_ptr],
    ),
    "fsi_decode_attn_dense_workspace_size": (_c_size, [_c_i64] * 7),
    "fsi_decode_attn_dense": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64,
         _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_int, _c_ptr, _c_ptr,
         _c_size, _c_ptr, _c_ptr],
    ),
    "fsi_decode_attn_noalloc": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_ptr, _c_ptr, _c_ptr],
    ),
    "fsi_sparse_attn_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "fsi_decode_attn_bwd_q": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64,
         _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         ctypes.c_float, _c_int, _c_ptr, _c_ptr, _c_ptr]),
    "fsi_sparse_attn_bwd_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "fsi_sparse_attn_bwd": (
        _c_int,
        [_c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64,
         _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64,
         _c_ptr, _c_i64, _c_i64, ctypes.c_float, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_size, _c_ptr, _c_ptr]),
    "fsi_sparse_attn": (
        _c_int,
        [_c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64,
         _c_ptr, _c_i64, _c_i64, ctypes.c_float, _c_int, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_size,
         _c_ptr, _c_ptr],
    ),
    "fsi_sram_indexer_attention": (
        _c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         ctypes.c_float, ctypes.c_float, _c_ptr, _c_ptr, _c_ptr],
    ),
    "fsi_block_sparse_linear_workspace_size": (_c_size, [_c_i64, _c_i64]),
    "fsi_block_sparse_linear": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr,
         _c_i64, _c_ptr, _c_size, _c_ptr, _c_ptr],
    ),
    "fsi_blockwise_matmul_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "fsi_blockwise_matmul": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int,
         _c_ptr, _c_i64, _c_ptr, _c_size, _c_ptr],
    ),
    "fsi_tile_route": (
        _c_int,
        [_c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_ptr, _c_ptr, _c_ptr, _c_ptr],
    ),
}

ROUTE_MAX_BLOCKS = 65536
SCORE_ROUTE_MAX_KEYS = 65536
ROUTE_MAX_RANKED = 256

_lib = None
_lib_lock = threading.Lock()


def library_path() -> Path:
    return LIB_PATH


def lib() -> ctypes.CDLL:
    """Load libfsi_amd.so (after torch, so both share torch's HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"HIP library {LIB_PATH} is not built; run __graft_entry__.build() "
                    "(or python foveal-sparse-indexer_amd/build.py) first"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


_EXC = {
    FSI_ERR_INVALID_ARG: ValueError,
    FSI_ERR_SHAPE: ValueError,
    FSI_ERR_INDEX_RANGE: IndexError,
    FSI_ERR_CAPACITY: RuntimeError,
    FSI_ERR_DTYPE: TypeError,
    FSI_ERR_HIP: RuntimeError,
    FSI_ERR_ALIGN: ValueError,
    FSI_ERR_WORKSPACE: RuntimeError,
}


def check(status: int, what: str) -> None:
    """Map a C-ABI status code to the Python exception type the reference raises."""
    if status == FSI_OK:
        return
    L = lib()
    msg = L.fsi_last_error().decode(errors="replace")
    kind = L.fsi_status_string(status).decode(errors="replace")
    raise _EXC.get(status, RuntimeError)(f"{what}: {kind}: {msg}")


def require_gpu(*tensors: torch.Tensor, what: str = "op") -> torch.device:
    """All tensors must live on one ROCm GPU.  There is deliberately no CPU fallback."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                f"{what}: tensors must be on a ROCm GPU (got {t.device}); "
                "the MI355X build has no CPU path"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{what}: tensors on different devices ({dev} vs {t.device})")
    if dev is None:
        raise RuntimeError(f"{what}: no tensor arguments")
    return dev


def dtype_code(dt: torch.dtype, what: str) -> int:
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float32:
        return DTYPE_F32
    raise TypeError(f"{what}: dtype {dt} not supported (bfloat16 or float32)")


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------------------
# Workspaces: one zero-initialised byte buffer per (device, stream).  Kernels
# leave their arrival counters at zero, so a buffer is zeroed only when it is
# (re)allocated.  Calls on one stream are ordered, so they can share it.  A HIP
# graph captured on a stream replays its launches on the buffer that stream had
# at capture time, so once a capture has used a stream's buffer, growing it keeps
# the old one alive (in _ws_kept) for as long as the process runs.
# ---------------------------------------------------------------------------
_ws: dict[tuple[int, int], torch.Tensor] = {}
_ws_captured: set[tuple[int, int]] = set()
_ws_kept: list[torch.Tensor] = []
_err: dict[int, torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int, stream: int) -> torch.Tensor:
    key = (device.index, stream)
    capturing = torch.cuda.is_current_stream_capturing()
    buf = _ws.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None and (capturing or key in _ws_captured):
            _ws_kept.append(buf)  # a captured graph may still launch kernels on it
        size = max(int(nbytes * 1.25) + 4096, 1 << 20)
        buf = torch.zeros(size, dtype=torch.uint8, device=device)
        _ws[key] = buf
    if capturing:
        _ws_captured.add(key)
    return buf


def error_word(device: torch.device) -> torch.Tensor:
    e = _err.get(device.index)
    if e is None:
        e = torch.zeros(64, dtype=torch.int32, device=device)
        _err[device.index] = e
    return e


def checks_enabled() -> bool:
    return os.environ.get("FSI_CHECK", "0") not in ("", "0")


def raise_device_errors(device: torch.device, what: str) -> None:
    """Synchronise and raise if a kernel recorded an out-of-range index.  Only
    called when FSI_CHECK is set (it costs a host sync)."""
    e = error_word(device)
    code = int(e[0].item())
    if code != 0:
        e.zero_()
        raise _EXC.get(code, RuntimeError)(f"{what}: device reported: {lib().fsi_status_string(code).decode()}")


# ---------------------------------------------------------------------------
# torch.library registration.  Every kernel launch of the package is a custom op
# torch.ops.fsi.<name>: its schema comes from the launch function's annotations,
# `fake` gives the output shapes / dtypes for FakeTensor tracing (torch.compile,
# torch.export), and the modules' autograd Functions call the forward and
# backward ops, so a compiled graph holds the HIP launches as single nodes.
# ---------------------------------------------------------------------------
NAMESPACE = "fsi"


def fsi_op(name: str, fake, mutates_args=()):
    """Decorator: register `fn` as torch.ops.fsi.<name> and return the op (calling
    it dispatches through torch.ops)."""

    def deco(fn):
        op = torch.library.custom_op(f"{NAMESPACE}::{name}", fn, mutates_args=mutates_args)
        op.register_fake(fake)
        return op

    return deco
