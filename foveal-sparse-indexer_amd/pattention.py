"""Fused non-softmax Pattention and SwiGLU on MI355X.

Drop-in for foveal_indexer/pattention_triton.py: `triton_pattention`
(:204-277), `triton_fused_swiglu` (:98-104) and `TritonSwiGLUPattentionMLP`
(:314-375).  The `triton_*` names are kept for compatibility; the kernels are
hand-written HIP for gfx950 (csrc/pattention.hip), not Triton.
"""
from __future__ import annotations

from typing import Literal, Optional, Tuple

import torch
import torch.nn as nn
from torch import Tensor

from . import _lib

# The reference exports HAS_TRITON to say "the GPU kernel path exists".  Here the
# kernel path is the HIP library.
HAS_HIP = _lib.LIB_PATH.exists()
HAS_TRITON = HAS_HIP


def is_triton_available() -> bool:
    """The reference's GPU-kernel predicate (triton_ops.py:252-253): True when the
    kernel library is built and a GPU is visible.  The kernels are HIP, not Triton."""
    return HAS_HIP and torch.cuda.is_available()


def _as_index_tensor(active_blocks, device: torch.device) -> Tensor:
    if isinstance(active_blocks, Tensor):
        t = active_blocks
    else:
        t = torch.as_tensor(active_blocks)
    return t.reshape(-1).to(device=device, dtype=torch.int32).contiguous()


def _rows_contig(t: Tensor) -> Tensor:
    """2-D view with unit stride along the last dim (copies only when needed)."""
    if t.dim() != 2:
        raise ValueError(f"expected a 2-D tensor, got shape {tuple(t.shape)}")
    if t.stride(1) != 1 or t.stride(0) < t.shape[1]:
        t = t.contiguous()
    return t


def pattention_forward(
    x2d: Tensor,
    k_gate: Tensor,
    k_up: Optional[Tensor],
    v: Tensor,
    active_blocks: Optional[Tensor],
    block_n: int,
    activation: str = "swiglu",
    rounding: str = "fp32",
    out: Optional[Tensor] = None,
) -> Tensor:
    """out[M, D_out] = act(x K_gate[S]^T [, x K_up[S]^T]) V[S] on the GPU.

    x2d: (M, K); k_gate/k_up: (N_p, K); v: (N_p, D_out); active_blocks: int
    block ids (or None for all channels).  rounding selects the bf16 rounding
    points ("eager", "fused" or "fp32"; see include/fsi.h)."""
    what = "pattention"
    dev = _lib.require_gpu(x2d, k_gate, k_up, v, what=what)
    dt = x2d.dtype
    for t in (k_gate, k_up, v):
        if t is not None and t.dtype != dt:
            raise TypeError(f"{what}: mixed dtypes {dt} and {t.dtype}")
    code = _lib.dtype_code(dt, what)
    act = _lib.ACTIVATIONS.get(activation.lower())
    if act is None:
        raise ValueError(f"{what}: unknown activation {activation!r}")
    if act == 0 and k_up is None:
        raise ValueError(f"{what}: k_up required for swiglu")
    rnd = _lib.ROUNDING[rounding]

    x2d = _rows_contig(x2d)
    k_gate = _rows_contig(k_gate)
    # V may be stored [N_p, D_out] row-major or, as FovealPattentionMLP keeps it,
    # as the transpose of a row-major [D_out, N_p] (a dense MLP's down_proj layout).
    if v.dim() != 2:
        raise ValueError(f"{what}: v must be 2-D, got {tuple(v.shape)}")
    v_transposed = v.stride(0) == 1 and v.stride(1) >= v.shape[0] and v.shape[1] > 1
    if v_transposed and code != _lib.DTYPE_BF16:
        v_transposed = False  # the fp32 kernels read V as [N_p, D_out]
    if not v_transposed:
        v = _rows_contig(v)
    if k_up is not None:
        k_up = _rows_contig(k_up)
        if k_up.stride(0) != k_gate.stride(0):
            k_up = k_up.contiguous()
            k_gate = k_gate.contiguous()
    M, K = x2d.shape
    N_p, K2 = k_gate.shape
    if K2 != K:
        raise ValueError(f"{what}: x has K={K} but k_gate has {K2}")
    if k_up is not None and tuple(k_up.shape) != (N_p, K):
        raise ValueError(f"{what}: k_up shape {tuple(k_up.shape)} != {(N_p, K)}")
    if v.shape[0] != N_p:
        raise ValueError(f"{what}: v has {v.shape[0]} rows, k_gate has {N_p}")
    D_out = v.shape[1]

    idx = _as_index_tensor(active_blocks, dev) if active_blocks is not None else None
    if out is None:
        return _pattention_op(x2d, k_gate, k_up, v, idx, block_n, act, rnd, v_transposed)
    return _pattention_launch(x2d, k_gate, k_up, v, idx, block_n, act, rnd, v_transposed, out)


def _pattention_launch(x2d: Tensor, k_gate: Tensor, k_up: Optional[Tensor], v: Tensor, idx: Optional[Tensor],
                       block_n: int, act: int, rnd: int, v_transposed: bool, out: Tensor) -> Tensor:
    what = "pattention"
    dev = x2d.device
    M, K = x2d.shape
    N_p = k_gate.shape[0]
    D_out = v.shape[1]
    n_active = 0 if idx is None else idx.numel()
    n_channels = N_p if idx is None else n_active * block_n
    if idx is not None and n_active == 0:
        # An empty block list contributes nothing (pattention_triton.py:141 loop never runs).  The
        # ABI reads a null list as "all blocks", and an empty tensor's data pointer is null.
        return out.zero_()
    code = _lib.dtype_code(x2d.dtype, what)
    ldv = v.stride(1) if v_transposed else v.stride(0)
    stream = _lib.stream_handle(dev)
    L = _lib.lib()
    ws_bytes = L.fsi_pattention_workspace_size(M, K, D_out, max(n_channels, 1), code)
    ws = _lib.workspace(dev, ws_bytes, stream)
    err = _lib.error_word(dev)
    st = L.fsi_pattention_fwd(
        x2d.data_ptr(), x2d.stride(0), k_gate.data_ptr(), _lib.ptr(k_up), k_gate.stride(0),
        v.data_ptr(), ldv, int(v_transposed), _lib.ptr(idx), n_active, block_n, M, K, N_p, D_out, code, act, rnd,
        out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(), err.data_ptr(), stream,
    )
    _lib.check(st, what)
    if _lib.checks_enabled():
        _lib.raise_device_errors(dev, what)
    return out


@_lib.fsi_op("pattention", lambda x2d, k_gate, k_up, v, idx, block_n, act, rnd, v_transposed:
             x2d.new_empty((x2d.shape[0], v.shape[1])))
def _pattention_op(x2d: Tensor, k_gate: Tensor, k_up: Optional[Tensor], v: Tensor, idx: Optional[Tensor],
                   block_n: int, act: int, rnd: int, v_transposed: bool) -> Tensor:
    """fsi_pattention_fwd into a new (M, D_out) tensor (arguments prepared by pattention_forward)."""
    out = torch.empty((x2d.shape[0], v.shape[1]), dtype=x2d.dtype, device=x2d.device)
    return _pattention_launch(x2d, k_gate, k_up, v, idx, block_n, act, rnd, v_transposed, out)


class PackedPattentionWeights:
    """k_gate, k_up and v repacked into the MFMA operand layout of the decode
    path (fsi_pattention_pack): one uint8 device buffer plus the shapes and the
    identity of the tensors it was built from."""

    def __init__(self, buf: Tensor, N_p: int, K: int, D_out: int, block_n: int, key: tuple):
        self.buf, self.N_p, self.K, self.D_out, self.block_n, self.key = buf, N_p, K, D_out, block_n, key


def _weights_key(*ts: Tensor) -> tuple:
    return tuple((t.data_ptr(), t._version, tuple(t.shape), tuple(t.stride())) for t in ts)


PACKED_PREFILL_MIN_M = 256


def packed_decode_supported(M: int, K: int, D_out: int, N_p: int, block_n: int, n_channels: int) -> bool:
    """Shapes fsi_pattention_fwd_packed takes (include/fsi.h): decode (1..64 tokens,
    at most 8192 active channels) and prefill (256 tokens and more, at most 2048
    active blocks)."""
    nc = K // 256
    common = (K % 256 == 0 and nc in (1, 2, 4, 8, 16, 32) and D_out % 16 == 0 and block_n >= 32
              and block_n & (block_n - 1) == 0 and N_p % block_n == 0 and n_channels >= 1)
    if not common:
        return False
    if 1 <= M <= 64:
        return n_channels <= 8192
    return M >= PACKED_PREFILL_MIN_M and n_channels // block_n <= 2048


def pack_pattention_weights(k_gate: Tensor, k_up: Tensor, v: Tensor, block_n: int) -> PackedPattentionWeights:
    """Repack bf16 k_gate / k_up (N_p, K) and v (N_p, D_out), in either storage
    order, for pattention_decode_packed.  One pass over the weights."""
    what = "pack_pattention_weights"
    dev = _lib.require_gpu(k_gate, k_up, v, what=what)
    if not (k_gate.dtype == k_up.dtype == v.dtype == torch.bfloat16):
        raise TypeError(f"{what}: bfloat16 weights required")
    key = _weights_key(k_gate, k_up, v)
    k_gate, k_up = _rows_contig(k_gate), _rows_contig(k_up)
    if k_up.stride(0) != k_gate.stride(0) or k_gate.stride(0) % 8:
        k_gate, k_up = k_gate.contiguous(), k_up.contiguous()
    v_transposed = v.stride(0) == 1 and v.stride(1) >= v.shape[0] and v.shape[1] > 1
    if not v_transposed:
        v = _rows_contig(v)
    N_p, K = k_gate.shape
    D_out = v.shape[1]
    if tuple(k_up.shape) != (N_p, K) or v.shape[0] != N_p:
        raise ValueError(f"{what}: k_gate {tuple(k_gate.shape)}, k_up {tuple(k_up.shape)}, v {tuple(v.shape)}")
    buf = _pack_op(k_gate, k_up, v, bool(v_transposed), int(block_n))
    return PackedPattentionWeights(buf, N_p, K, D_out, block_n, key)


def unpack_pattention_weights(packed: PackedPattentionWeights,
                              blocks: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """Inverse of pack_pattention_weights: k_gate, k_up (N_p, K) and v (N_p, D_out)
    rebuilt from the packed buffer as new contiguous bf16 tensors (tensor views and
    one permuted copy each, no kernel of this library).  With `blocks` (block
    ids of block_n channels) only those blocks' rows, in that order.

    Buffer layout (fsi_pattention_pack): gate tiles at byte 0, up tiles at
    align256(2 N_p K), down tiles at twice that.  Gate / up tile (ct, s) holds
    W[16 ct + r][32 s + 8 q + e] at element (16 q + r) 8 + e; down tile (b, dt, cl)
    holds V[b block_n + 32 cl + 8 q + e][16 dt + r] at the same position."""
    N_p, K, D, bn = packed.N_p, packed.K, packed.D_out, packed.block_n
    mat = (2 * N_p * K + 255) // 256 * 256
    buf = packed.buf

    def rows(off: int) -> Tensor:
        t = buf[off:off + 2 * N_p * K].view(torch.bfloat16).view(N_p // bn, bn // 16, K // 32, 4, 16, 8)
        if blocks is not None:
            t = t.index_select(0, blocks)
        return t.permute(0, 1, 4, 2, 3, 5).reshape(-1, K)

    d = buf[2 * mat:2 * mat + 2 * N_p * D].view(torch.bfloat16).view(N_p // bn, D // 16, bn // 32, 4, 16, 8)
    if blocks is not None:
        d = d.index_select(0, blocks)
    v = d.permute(0, 2, 3, 5, 1, 4).reshape(-1, D)
    return rows(0), rows(mat), v


@_lib.fsi_op("pattention_pack", lambda k_gate, k_up, v, v_transposed, block_n: k_gate.new_empty(
    (_lib.lib().fsi_pattention_packed_size(k_gate.shape[0], k_gate.shape[1], v.shape[1]),), dtype=torch.uint8))
def _pack_op(k_gate: Tensor, k_up: Tensor, v: Tensor, v_transposed: bool, block_n: int) -> Tensor:
    """fsi_pattention_pack into a new byte buffer (arguments prepared by pack_pattention_weights)."""
    what = "pack_pattention_weights"
    N_p, K = k_gate.shape
    D_out = v.shape[1]
    ldv = v.stride(1) if v_transposed else v.stride(0)
    L = _lib.lib()
    nbytes = L.fsi_pattention_packed_size(N_p, K, D_out)
    buf = torch.empty(nbytes, dtype=torch.uint8, device=k_gate.device)
    st = L.fsi_pattention_pack(k_gate.data_ptr(), k_up.data_ptr(), k_gate.stride(0), v.data_ptr(), ldv,
                               int(v_transposed), N_p, K, D_out, block_n, _lib.DTYPE_BF16, buf.data_ptr(), nbytes,
                               _lib.stream_handle(k_gate.device))
    _lib.check(st, what)
    return buf


def pattention_decode_packed(
    x2d: Tensor,
    packed: PackedPattentionWeights,
    active_blocks: Optional[Tensor],
    rounding: str = "fused",
    out: Optional[Tensor] = None,
) -> Tensor:
    """SwiGLU Pattention of bf16 tokens over packed weights: the same result as
    pattention_forward(x2d, k_gate, k_up, v, active_blocks, block_n, "swiglu",
    rounding) up to fp32 summation order.  1..64 tokens run the decode kernels,
    256 and more the prefill GEMMs reading the same packed tiles."""
    what = "pattention_decode_packed"
    dev = _lib.require_gpu(x2d, packed.buf, what=what)
    if x2d.dtype != torch.bfloat16:
        raise TypeError(f"{what}: x dtype {x2d.dtype} (bfloat16 only)")
    x2d = _rows_contig(x2d)
    if x2d.stride(0) % 8 or x2d.data_ptr() % 16:
        x2d = x2d.contiguous()
    M, K = x2d.shape
    if K != packed.K:
        raise ValueError(f"{what}: x has K={K}, weights {packed.K}")
    idx = _as_index_tensor(active_blocks, dev) if active_blocks is not None else None
    rnd = _lib.ROUNDING[rounding]
    if out is None:
        return _packed_op(x2d, packed.buf, idx, packed.N_p, packed.D_out, packed.block_n, rnd)
    return _packed_launch(x2d, packed.buf, idx, packed.N_p, packed.D_out, packed.block_n, rnd, out)


def _packed_launch(x2d: Tensor, buf: Tensor, idx: Optional[Tensor], N_p: int, D_out: int, block_n: int, rnd: int,
                   out: Tensor) -> Tensor:
    what = "pattention_decode_packed"
    dev = x2d.device
    M, K = x2d.shape
    n_active = 0 if idx is None else idx.numel()
    n_ch = N_p if idx is None else n_active * block_n
    if idx is not None and n_active == 0:
        return out.zero_()
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    ws = _lib.workspace(dev, L.fsi_pattention_packed_workspace_size(M, K, D_out, n_ch, block_n), stream)
    err = _lib.error_word(dev)
    st = L.fsi_pattention_fwd_packed(
        x2d.data_ptr(), x2d.stride(0), buf.data_ptr(), _lib.ptr(idx), n_active, block_n, M, K, N_p, D_out,
        _lib.DTYPE_BF16, rnd, out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(), err.data_ptr(), stream)
    _lib.check(st, what)
    if _lib.checks_enabled():
        _lib.raise_device_errors(dev, what)
    return out


@_lib.fsi_op("pattention_packed", lambda x2d, buf, idx, N_p, D_out, block_n, rnd:
             x2d.new_empty((x2d.shape[0], D_out)))
def _packed_op(x2d: Tensor, buf: Tensor, idx: Optional[Tensor], N_p: int, D_out: int, block_n: int,
               rnd: int) -> Tensor:
    """fsi_pattention_fwd_packed into a new (M, D_out) bf16 tensor."""
    out = torch.empty((x2d.shape[0], D_out), dtype=torch.bfloat16, device=x2d.device)
    return _packed_launch(x2d, buf, idx, N_p, D_out, block_n, rnd, out)


def triton_pattention(
    x: Tensor,
    k_gate: Tensor,
    v: Tensor,
    k_up: Optional[Tensor] = None,
    active_blocks: Optional[Tensor] = None,
    activation: Literal["swiglu", "silu", "gelu", "relu", "relu2"] = "swiglu",
    block_n: int = 64,
) -> Tensor:
    """Fused non-softmax Pattention (pattention_triton.py:204-277).

    Same signature and output as the reference op.  bf16 rounds the activation
    once from the fp32 accumulators before the V contraction, as the
    reference's fused kernel does (pattention_triton.py:197).  GeLU is the exact
    erf form of the reference's PyTorch path (pattention_triton.py:300).
    Unknown activation names fall back to SwiGLU like the reference kernel's
    code map (pattention_triton.py:245-246)."""
    act = activation.lower() if activation.lower() in _lib.ACTIVATIONS else "swiglu"
    orig_shape = x.shape
    x2d = x.reshape(-1, x.shape[-1])
    out = pattention_forward(x2d, k_gate, k_up, v, active_blocks, block_n, act, rounding="fp32")
    if len(orig_shape) > 2:
        return out.reshape(*orig_shape[:-1], v.shape[-1])
    return out


@_lib.fsi_op("swiglu", lambda g, u, rounding: torch.empty_like(g, memory_format=torch.contiguous_format))
def _swiglu_launch(g: Tensor, u: Tensor, rounding: str) -> Tensor:
    what = "swiglu"
    dev = _lib.require_gpu(g, u, what=what)
    if g.shape != u.shape or g.dtype != u.dtype:
        raise ValueError(f"{what}: g {tuple(g.shape)}/{g.dtype} vs u {tuple(u.shape)}/{u.dtype}")
    code = _lib.dtype_code(g.dtype, what)
    g_c, u_c = g.contiguous(), u.contiguous()
    out = torch.empty_like(g_c)
    st = _lib.lib().fsi_swiglu(g_c.data_ptr(), u_c.data_ptr(), out.data_ptr(), g_c.numel(), code,
                               _lib.ROUNDING[rounding], _lib.stream_handle(dev))
    _lib.check(st, what)
    return out


@_lib.fsi_op("swiglu_bwd", lambda dout, g, u: (torch.empty_like(g), torch.empty_like(u)))
def _swiglu_bwd_op(dout: Tensor, g: Tensor, u: Tensor) -> Tuple[Tensor, Tensor]:
    what = "swiglu backward"
    dev = _lib.require_gpu(dout, g, u, what=what)
    code = _lib.dtype_code(g.dtype, what)
    d = dout.to(g.dtype).contiguous()
    dg, du = torch.empty_like(g), torch.empty_like(u)
    st = _lib.lib().fsi_swiglu_bwd(d.data_ptr(), g.data_ptr(), u.data_ptr(), dg.data_ptr(), du.data_ptr(),
                                   g.numel(), code, _lib.stream_handle(dev))
    _lib.check(st, what)
    return dg, du


class FusedSwiGLUFunction(torch.autograd.Function):
    """silu(g) * u with its exact backward on the HIP kernels
    (TritonFusedSwiGLUFunction, pattention_triton.py:73-96): the forward rounds
    silu(g) * u once from fp32, the backward computes du = dout * silu(g) and
    dg = dout * u * s (1 + g (1 - s)), s = sigmoid(g), in fp32."""

    @staticmethod
    def forward(ctx, g: Tensor, u: Tensor) -> Tensor:
        g_c, u_c = g.contiguous(), u.contiguous()
        ctx.save_for_backward(g_c, u_c)
        return _swiglu_launch(g_c, u_c, "fused")

    @staticmethod
    def backward(ctx, dout: Tensor):
        g, u = ctx.saved_tensors
        return _swiglu_bwd_op(dout, g, u)


def triton_fused_swiglu(g: Tensor, u: Tensor) -> Tensor:
    """silu(g) * u in fp32, rounded once, with exact gradients
    (pattention_triton.py:30-104).  The `triton_` name is kept; the kernels are HIP."""
    return FusedSwiGLUFunction.apply(g, u)


def fused_swiglu(g: Tensor, u: Tensor, rounding: str = "fused") -> Tensor:
    """silu(g) * u with the given bf16 rounding points ("fused": one rounding;
    "eager": silu(g) rounded first, as torch's eager F.silu(g) * u).  The fused
    form is differentiable (FusedSwiGLUFunction); the eager form is forward-only."""
    if rounding == "fused":
        return FusedSwiGLUFunction.apply(g, u)
    if torch.is_grad_enabled() and (g.requires_grad or u.requires_grad):
        raise NotImplementedError("swiglu: the eager-rounding form has no backward; use rounding='fused'")
    return _swiglu_launch(g, u, rounding)


def _aligned_rows(t: Tensor) -> Tensor:
    """Contiguous rows whose start is 16-byte aligned (the GEMM's direct loads)."""
    t = _rows_contig(t)
    if t.data_ptr() % 16 or t.stride(0) % 8:
        t = t.contiguous()
        if t.data_ptr() % 16:
            t = t.clone()
    return t


def dense_block_targets(norm_h: Tensor, gate_w: Tensor, up_w: Tensor, down_w: Tensor, block_size: int = 64,
                        temperature: float = 1.0) -> Tensor:
    """Block-energy distillation targets of a dense SwiGLU MLP
    (archive/hy_mt2/llm_pattention/train_foveal_pattention_speedrun.py:176-185):
    act = silu(h W_gate^T) * (h W_up^T) over all channels, block energy =
    mean over the block of |act| times the block mean of W_down's column norms,
    P = softmax(energy / temperature) in fp32.

    norm_h: (..., D) bf16 (the MLP input after post_attention_layernorm);
    gate_w, up_w: (I, D) bf16; down_w: (D, I) bf16 (nn.Linear layouts).
    Returns (..., I // block_size) float32.  One fused GEMM whose epilogue
    reduces |act| in registers: the (tokens, I) activation is never stored.
    """
    what = "dense_block_targets"
    dev = _lib.require_gpu(norm_h, gate_w, up_w, down_w, what=what)
    for name, t in (("norm_h", norm_h), ("gate_w", gate_w), ("up_w", up_w), ("down_w", down_w)):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{what}: {name} must be bfloat16, got {t.dtype}")
    D = norm_h.shape[-1]
    I = gate_w.shape[0]
    if gate_w.shape != (I, D) or up_w.shape != (I, D) or down_w.shape != (D, I):
        raise ValueError(f"{what}: gate {tuple(gate_w.shape)}, up {tuple(up_w.shape)}, down {tuple(down_w.shape)} "
                         f"do not match hidden size {D}")
    if block_size < 32 or block_size % 32 or I % block_size:
        raise ValueError(f"{what}: block_size {block_size} must be a multiple of 32 dividing {I}")
    lead = norm_h.shape[:-1]
    h = _aligned_rows(norm_h.reshape(-1, D))
    gw, uw, dw = _aligned_rows(gate_w), _aligned_rows(up_w), _aligned_rows(down_w)
    nb = I // block_size
    if h.shape[0] == 0:
        return torch.empty((*lead, nb), dtype=torch.float32, device=dev)
    if gw.stride(0) != uw.stride(0):
        uw = uw.contiguous()
        gw = gw.contiguous()
    return _block_targets_op(h, gw, uw, dw, block_size, float(temperature)).reshape(*lead, nb)


@_lib.fsi_op("dense_block_targets", lambda h, gw, uw, dw, block_size, temperature:
             h.new_empty((h.shape[0], gw.shape[0] // block_size), dtype=torch.float32))
def _block_targets_op(h: Tensor, gw: Tensor, uw: Tensor, dw: Tensor, block_size: int, temperature: float) -> Tensor:
    """fsi_dense_block_targets: (M, I / block_size) fp32 (arguments prepared by dense_block_targets)."""
    what = "dense_block_targets"
    dev = h.device
    M, D = h.shape
    I = gw.shape[0]
    nb = I // block_size
    out = torch.empty((M, nb), dtype=torch.float32, device=dev)
    lib = _lib.lib()
    ws = torch.empty(lib.fsi_dense_block_targets_workspace_size(M, D, I, block_size), dtype=torch.uint8, device=dev)
    st = lib.fsi_dense_block_targets(h.data_ptr(), h.stride(0), gw.data_ptr(), uw.data_ptr(), gw.stride(0),
                                     dw.data_ptr(), dw.stride(0), M, D, I, block_size, temperature,
                                     out.data_ptr(), nb, ws.data_ptr(), ws.numel(), _lib.stream_handle(dev))
    _lib.check(st, what)
    return out


class TritonSwiGLUPattentionMLP(nn.Module):
    """Drop-in SwiGLU MLP via fused Pattention (pattention_triton.py:314-375)."""

    def __init__(
        self,
        hidden_dim: int = 2048,
        num_param_tokens: int = 6144,
        block_size: int = 64,
        activation: str = "swiglu",
        dtype: torch.dtype = torch.bfloat16,
    ):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.num_param_tokens = num_param_tokens
        self.block_size = block_size
        self.activation = activation
        self.num_blocks = num_param_tokens // block_size
        self.k_gate = nn.Parameter(torch.empty(num_param_tokens, hidden_dim, dtype=dtype))
        self.k_up = nn.Parameter(torch.empty(num_param_tokens, hidden_dim, dtype=dtype))
        self.v = nn.Parameter(torch.empty(num_param_tokens, hidden_dim, dtype=dtype))
        nn.init.normal_(self.k_gate, std=hidden_dim ** -0.5)
        nn.init.normal_(self.k_up, std=hidden_dim ** -0.5)
        nn.init.normal_(self.v, std=num_param_tokens ** -0.5)

    @classmethod
    def from_dense_mlp(cls, dense_mlp: nn.Module, block_size: int = 64) -> "TritonSwiGLUPattentionMLP":
        hidden_dim = dense_mlp.gate_proj.in_features
        intermediate_dim = dense_mlp.gate_proj.out_features
        dtype = dense_mlp.gate_proj.weight.dtype
        device = dense_mlp.gate_proj.weight.device
        mlp = cls(hidden_dim=hidden_dim, num_param_tokens=intermediate_dim, block_size=block_size,
                  activation="swiglu", dtype=dtype).to(device)
        with torch.no_grad():
            mlp.k_gate.copy_(dense_mlp.gate_proj.weight)
            mlp.k_up.copy_(dense_mlp.up_proj.weight)
            mlp.v.copy_(dense_mlp.down_proj.weight.t())
        return mlp

    def forward(self, x: Tensor, active_blocks: Optional[Tensor] = None) -> Tensor:
        return triton_pattention(x, self.k_gate, self.v, k_up=self.k_up, active_blocks=active_blocks,
                                 activation=self.activation, block_n=self.block_size)


def convert_llm_mlp_to_pattention(
    model: nn.Module,
    layers: Optional[list] = None,
    block_size: int = 64,
    activation: str = "swiglu",
) -> nn.Module:
    """Replace `model.model.layers[i].mlp` with TritonSwiGLUPattentionMLP
    (pattention_triton.py:378-395)."""
    model_layers = getattr(model, "model", model).layers
    target_layers = layers if layers is not None else list(range(len(model_layers)))
    for idx in target_layers:
        if hasattr(model_layers[idx], "mlp") and not isinstance(model_layers[idx].mlp, TritonSwiGLUPattentionMLP):
            model_layers[idx].mlp = TritonSwiGLUPattentionMLP.from_dense_mlp(model_layers[idx].mlp,
                                                                            block_size=block_size)
    return model
