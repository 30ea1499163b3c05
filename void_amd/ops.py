"""Float SpMM on VOID tiles (void/ops.py:148-213): C = A @ B on the MFMA
kernels of libvoid_amd.so: void_spmm_bf16 / void_spmm_f16 when the tiles and
B share a 16-bit dtype, void_spmm_f32 (fp32 tiles and B) otherwise."""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib, _runtime

# Longest work item of the float kernel: it holds an item's block columns in
# one register per lane.
F32_CHUNK = 64


_K16 = {torch.bfloat16: "void_spmm_bf16", torch.float16: "void_spmm_f16"}


def _fits16(a, b: torch.Tensor, c: torch.Tensor) -> bool:
    """What void_spmm_bf16 / void_spmm_f16 take: row-major B and C with
    16-byte aligned rows, N % 8 == 0, and operands within 31-bit offsets."""
    M, K = a.shape
    N = b.shape[1]
    lim = 1 << 31
    return (N % 8 == 0 and b.stride(0) % 8 == 0 and b.data_ptr() % 16 == 0 and
            c.data_ptr() % 16 == 0 and c.stride(0) % 4 == 0 and
            a.n_blocks * 2048 < lim and ((K + 31) // 32) * 32 * b.stride(0) * 2 < lim and
            M * c.stride(0) * c.element_size() < lim)


def float_spmm(a, b: torch.Tensor, *, out: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
               activation: int = _lib.ACT_NONE, bias_per_row: bool = False,
               plan: Optional["_runtime.DevicePlan"] = None) -> torch.Tensor:
    """activation(A @ B + bias) for a float VOIDTensor A; the output has B's
    dtype (f32, bf16 or f16), as the reference's kernels write.  bias is [N]
    (per column), or [M] with bias_per_row (fusion.py:202-304).  ``plan``
    (work items of at most 64 tiles) replaces the default partition."""
    if b.dim() != 2:
        raise ValueError("B must be 2-D")
    M, K = a.shape
    if K != b.shape[0]:
        raise ValueError(f"A is {M}x{K} but B has {b.shape[0]} rows")
    _runtime.require_gpu(b, "B")
    N = b.shape[1]
    out_dtype = b.dtype if b.dtype in (torch.float32, torch.bfloat16, torch.float16) else torch.float32
    if out is None:
        out = torch.empty(M, N, dtype=out_dtype, device=b.device)
    elif out.shape != (M, N):
        raise ValueError(f"out must be [{M}, {N}]")
    if a.n_blocks == 0:
        out.zero_()
        if bias is not None:
            out[:] = (bias[:, None] if bias_per_row else bias[None, :]).to(out.dtype)
        return out
    _runtime.require_gpu(a.values, "A")
    if a.values.device != b.device:
        raise ValueError(f"A on {a.values.device}, B on {b.device}")
    if bias is not None:
        if bias.shape != ((M,) if bias_per_row else (N,)):
            raise ValueError(f"bias must be [{M if bias_per_row else N}]")
        bias = bias.to(device=b.device, dtype=torch.float32).contiguous()
    lib = _lib.lib()
    target = out if (out.stride(1) == 1 and out.stride(0) >= N) else torch.empty_like(out)
    # 16-bit tiles times a B of the same dtype run on the 16-bit MFMA (the
    # reference's tl.dot takes them as they are); everything else on the fp32
    # kernel, whose products of widened 16-bit values are the same numbers.
    entry = "void_spmm_f32"
    bk = None
    if a.values.dtype == b.dtype and b.dtype in _K16:
        bk = b if b.stride(1) == 1 else b.contiguous()
        if not _fits16(a, bk, target):
            bk = None
    if bk is not None:
        entry = _K16[b.dtype]
        dbsr = a.device_bsr(b.dtype)
    else:
        bk = b.to(torch.float32).contiguous()
        dbsr = a.device_bsr()
    if plan is None:
        plan = dbsr.plan(F32_CHUNK)
    elif plan.chunk > F32_CHUNK:
        raise ValueError(f"the float kernel takes work items of at most {F32_CHUNK} tiles, got {plan.chunk}")
    ws, ws_bytes = plan.workspace(N, out.device)
    cplan = _lib.Plan(items=plan.items.data_ptr(), n_items=plan.n_items, n_split_tiles=plan.n_split_tiles,
                      n_slots=plan.n_slots, chunk_tiles=plan.chunk)
    dense = _lib.DenseArgs(b=bk.data_ptr(), ldb=bk.stride(0), b_col_major=0, N=N, b_scale=1.0, b_scale_vec=None,
                           bias=bias.data_ptr() if bias is not None else None, c=target.data_ptr(),
                           ldc=target.stride(0), out_dtype=_runtime.out_code(target.dtype), activation=activation,
                           bias_per_row=int(bias_per_row))
    desc = dbsr.desc()
    st = getattr(lib, entry)(ctypes.byref(desc), ctypes.byref(dense), ctypes.byref(cplan),
                             ws.data_ptr() if ws is not None else None, ws_bytes,
                             torch.cuda.current_stream(out.device).cuda_stream)
    _lib.check(st, entry)
    if target is not out:
        out.copy_(target)
    return out


def void_spmm(a, b: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """C = A @ B for a float VOIDTensor (ops.py:148-213); C has B's dtype."""
    from .int_quant import Int8VOIDTensor
    from .fp8 import FP8VOIDTensor
    if isinstance(a, (Int8VOIDTensor, FP8VOIDTensor)):
        raise TypeError("void_spmm takes a float VOIDTensor; use void_spmm_int8 / void_spmm_fp8 for quantised tiles")
    return float_spmm(a, b, out=out)


# The reference's tensor-core threshold on K (ops.py:28); on gfx950 every
# 32-wide tile feeds the MFMA.
MIN_TENSOR_CORE_K = 16


def compute_optimal_tile_n(N: int) -> int:
    """The reference's TILE_N rule (ops.py:31-42), kept for its callers; the
    gfx950 kernels compute 128-column panels whatever N."""
    if N >= 128:
        return 128
    if N >= 64:
        return 64
    if N >= 32:
        return 32
    if N >= 16:
        return 16
    return 1 << max(0, (int(N) - 1).bit_length())


__all__ = ["void_spmm", "float_spmm", "compute_optimal_tile_n", "MIN_TENSOR_CORE_K"]
