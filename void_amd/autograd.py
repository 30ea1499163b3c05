"""Differentiable float SpMM on VOID tiles (void/autograd.py:99-352).

Forward: C = A @ B on the fp32 kernel (void_spmm_f32).  Backward:
  dL/dB        = A^T @ dL/dC, the same kernel on the transposed tiles with
                 block rows and columns swapped (autograd.py:175-189);
  dL/dA_values = dL/dC @ B^T on the nonzero tiles only, the SDDMM kernel
                 void_sddmm_f32 (autograd.py:191-215).
The block structure's device ordering is computed once per structure and
reused across steps; only the tile values are regathered, since an
optimiser updates them in place.
"""

from __future__ import annotations

from typing import Any, Optional, Tuple

import torch
from torch.autograd import Function

from . import _runtime
from .format import VOIDTensor, build_bsr_layout
from .ops import float_spmm

_LAYOUTS: dict = {}


def _layout(block_rows: torch.Tensor, block_cols: torch.Tensor, shape: Tuple[int, int]):
    # Keyed on the structure tensors' identity and in-place version; each
    # entry holds the tensors themselves, so their memory cannot be handed
    # to other structure tensors (same address, version 0) while cached.
    key = (_runtime.source_key(block_rows, block_cols), int(block_rows.numel()), tuple(shape),
           str(block_rows.device))
    hit = _LAYOUTS.get(key)
    if hit is None:
        n_br, n_bc = (shape[0] + 31) // 32, (shape[1] + 31) // 32
        lay = build_bsr_layout(block_rows, block_cols, n_br, n_bc, block_rows.device)
        if len(_LAYOUTS) > 64:
            _LAYOUTS.clear()
        hit = _LAYOUTS[key] = (lay, block_rows, block_cols)
    return hit[0]


def _vt(values, block_rows, block_cols, shape, tile_size, n_blocks) -> VOIDTensor:
    vt = VOIDTensor(values=values, block_rows=block_rows, block_cols=block_cols,
                    morton_codes=torch.empty(0, dtype=torch.int64, device=values.device), shape=tuple(shape),
                    tile_size=tuple(tile_size), nnz_original=0, n_blocks=n_blocks, density=0.0, dtype=values.dtype)
    if n_blocks and values.is_cuda:
        # The device copy (fp32 or 16-bit, as the SpMM needs) is built on
        # first use from this cached block-row order.
        vt._bsr_layout = _layout(block_rows, block_cols, vt.shape)
    return vt


class VOIDSpMMFunction(Function):
    """C = A @ B with gradients for the tile values and for B (autograd.py:99-216)."""

    @staticmethod
    def forward(ctx: Any, a_values, a_block_rows, a_block_cols, a_shape, a_tile_size, a_n_blocks, b):
        c = float_spmm(_vt(a_values.detach(), a_block_rows, a_block_cols, a_shape, a_tile_size, a_n_blocks), b)
        ctx.save_for_backward(a_values, a_block_rows, a_block_cols, b)
        ctx.a_shape, ctx.a_tile_size, ctx.a_n_blocks = tuple(a_shape), tuple(a_tile_size), a_n_blocks
        return c

    @staticmethod
    def backward(ctx: Any, grad_output: torch.Tensor):
        a_values, rows, cols, b = ctx.saved_tensors
        M, K = ctx.a_shape
        grad_a = grad_b = None
        if ctx.needs_input_grad[6]:
            at = _vt(a_values.detach().permute(0, 2, 1).contiguous(), cols, rows, (K, M),
                     ctx.a_tile_size[::-1], ctx.a_n_blocks)
            grad_b = float_spmm(at, grad_output.contiguous()).to(b.dtype)
        if ctx.needs_input_grad[0]:
            grad_a = _runtime.sddmm_tiles(grad_output, b, rows, cols, (M, K), a_values.dtype,
                                          layout=_layout(rows, cols, (M, K)) if rows.is_cuda else None)
        return grad_a, None, None, None, None, None, grad_b


class VOIDSpMM(torch.nn.Module):
    """A VOID matrix as a module with trainable tile values (autograd.py:219-285)."""

    def __init__(self, void_tensor: VOIDTensor, requires_grad: bool = True):
        super().__init__()
        if requires_grad:
            self.values = torch.nn.Parameter(void_tensor.values.clone())
        else:
            self.register_buffer("values", void_tensor.values.clone())
        self.register_buffer("block_rows", void_tensor.block_rows)
        self.register_buffer("block_cols", void_tensor.block_cols)
        self.shape = void_tensor.shape
        self.tile_size = void_tensor.tile_size
        self.n_blocks = void_tensor.n_blocks

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        squeeze = x.dim() == 1
        if squeeze:
            x = x.unsqueeze(1)
        y = VOIDSpMMFunction.apply(self.values, self.block_rows, self.block_cols, self.shape, self.tile_size,
                                   self.n_blocks, x)
        return y.squeeze(1) if squeeze else y

    def get_void_tensor(self) -> VOIDTensor:
        return VOIDTensor(values=self.values.data, block_rows=self.block_rows, block_cols=self.block_cols,
                          morton_codes=torch.empty(0, device=self.values.device), shape=self.shape,
                          tile_size=self.tile_size, nnz_original=0, n_blocks=self.n_blocks, density=0.0)


class SparseLinear(torch.nn.Module):
    """nn.Linear with a VOID weight: y = x W^T + b (autograd.py:288-352)."""

    def __init__(self, in_features: int, out_features: int, void_tensor: VOIDTensor, bias: bool = True,
                 dtype: Optional[torch.dtype] = None):
        super().__init__()
        if tuple(void_tensor.shape) != (out_features, in_features):
            raise ValueError(f"weight is {tuple(void_tensor.shape)}, expected ({out_features}, {in_features})")
        self.in_features = in_features
        self.out_features = out_features
        self.sparse_weight = VOIDSpMM(void_tensor, requires_grad=True)
        dtype = dtype or void_tensor.dtype
        if bias:
            self.bias = torch.nn.Parameter(torch.zeros(out_features, dtype=dtype))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x_flat = x.reshape(-1, self.in_features)
        y = self.sparse_weight(x_flat.T).T
        if self.bias is not None:
            y = y + self.bias
        return y.reshape(x.shape[:-1] + (self.out_features,))

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}"


__all__ = ["VOIDSpMMFunction", "VOIDSpMM", "SparseLinear"]
