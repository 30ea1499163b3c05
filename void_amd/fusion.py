"""Fused SpMM + activation on quantised VOID tensors.

Mirrors the activation helpers and ``void_spmm_gelu`` / ``void_spmm_relu`` /
``void_spmm_silu`` of ``void/fusion.py``.  The reference fuses bias and
activation into its fp32 SpMM kernel (void_spmm_activation_kernel,
fusion.py:98-198); here the same epilogue (``+ bias[n]``, then the
activation, then the cast to the output dtype) runs in registers at the end
of the INT8 or FP8 gfx950 kernel.  GELU is the tanh form of fusion.py:38-43.
"""

from __future__ import annotations

from enum import Enum
from typing import Optional, Union

import torch


class ActivationType(Enum):
    """fusion.py:24-31."""
    NONE = "none"
    RELU = "relu"
    GELU = "gelu"
    SILU = "silu"
    TANH = "tanh"
    SIGMOID = "sigmoid"


_CODES = {"none": 0, "relu": 1, "gelu": 2, "silu": 3, "swish": 3, "tanh": 4, "sigmoid": 5}


def get_activation_code(activation: Union[str, ActivationType]) -> int:
    """Activation name -> kernel code (fusion.py:77-91); unknown names map to 0.

    Codes 4 (tanh) and 5 (sigmoid) exist in the reference's table but not in
    the gfx950 epilogue, which raises for them.
    """
    if isinstance(activation, ActivationType):
        activation = activation.value
    code = _CODES.get(str(activation).lower(), 0)
    if code > 3:
        raise NotImplementedError(f"activation {activation!r} is not fused by the gfx950 kernel")
    return code


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """tanh-form GELU exactly as written in fusion.py:38-43."""
    inner = 0.7978845608 * (x + 0.044715 * x * x * x)
    return x * 0.5 * (1.0 + (2.0 * torch.sigmoid(2.0 * inner) - 1.0))


def apply_activation_torch(x: torch.Tensor, activation: str) -> torch.Tensor:
    """Activation of an all-empty matrix (no tiles): the reference's own torch
    calls for that case (fusion.py:466-476; GELU there is torch's erf form)."""
    if activation == "relu":
        return torch.relu(x)
    if activation == "gelu":
        return torch.nn.functional.gelu(x)
    if activation in ("silu", "swish"):
        return torch.nn.functional.silu(x)
    return x


def _spmm_activation(a, b: torch.Tensor, bias: Optional[torch.Tensor], out: Optional[torch.Tensor],
                     activation: str, b_scale=None, out_dtype: Optional[torch.dtype] = None,
                     epilogue: Optional[str] = None) -> torch.Tensor:
    from .fp8 import FP8VOIDTensor, void_spmm_fp8
    from .int_quant import Int8VOIDTensor, void_spmm_int8
    if out_dtype is None:
        out_dtype = out.dtype if out is not None else (b.dtype if b.is_floating_point()
                                                       and b.dtype in (torch.float32, torch.bfloat16,
                                                                       torch.float16) else torch.float32)
    if isinstance(a, Int8VOIDTensor):
        if epilogue is None and b.dtype == torch.int8 and b_scale is not None:
            epilogue = "per_block"
        return void_spmm_int8(a, b, b_scale=b_scale, out=out, epilogue=epilogue, out_dtype=out_dtype,
                              activation=activation, bias=bias)
    if isinstance(a, FP8VOIDTensor):
        return void_spmm_fp8(a, b, output_dtype=out_dtype, b_scale=b_scale, activation=activation,
                             bias=bias, out=out)
    from .format import VOIDTensor
    if isinstance(a, VOIDTensor):
        # Float tiles: the reference's own case (fusion.py:444-511), fp32 MFMA
        # kernel; output in B's dtype.  An all-empty A keeps the reference's
        # torch activation of the bias (fusion.py:466-476).
        from .ops import float_spmm
        if a.n_blocks == 0:
            res = torch.zeros(a.shape[0], b.shape[1], dtype=b.dtype, device=b.device) if out is None else out.zero_()
            if bias is not None:
                res[:, :] = bias[None, :]
                res = apply_activation_torch(res, activation)
                if out is not None and res is not out:
                    out.copy_(res)
                    res = out
            return res
        return float_spmm(a, b, out=out, bias=bias, activation=get_activation_code(activation))
    raise TypeError(f"unsupported sparse operand {type(a).__name__}")


def void_spmm_gelu(a, b: torch.Tensor, bias: Optional[torch.Tensor] = None,
                   out: Optional[torch.Tensor] = None, *, b_scale=None,
                   out_dtype: Optional[torch.dtype] = None, epilogue: Optional[str] = None) -> torch.Tensor:
    """C = GELU(A @ B + bias) (fusion.py:381-399).

    Float VOIDTensor A: the reference's case, fp32 kernel, output in B's
    dtype.

    Int8VOIDTensor A: float B is quantised per tensor as void_spmm_int8
    does; an int8 B with b_scale (scalar or per column) uses the per-block
    epilogue (true dequantisation) unless ``epilogue`` says otherwise.
    Output dtype: ``out_dtype``, else out's dtype, else B's float dtype,
    else float32.
    """
    return _spmm_activation(a, b, bias, out, "gelu", b_scale, out_dtype, epilogue)


def void_spmm_relu(a, b: torch.Tensor, bias: Optional[torch.Tensor] = None,
                   out: Optional[torch.Tensor] = None, **kw) -> torch.Tensor:
    """C = ReLU(A @ B + bias) (fusion.py:402-420)."""
    return _spmm_activation(a, b, bias, out, "relu", kw.get("b_scale"), kw.get("out_dtype"), kw.get("epilogue"))


def void_spmm_silu(a, b: torch.Tensor, bias: Optional[torch.Tensor] = None,
                   out: Optional[torch.Tensor] = None, **kw) -> torch.Tensor:
    """C = SiLU(A @ B + bias) (fusion.py:423-441)."""
    return _spmm_activation(a, b, bias, out, "silu", kw.get("b_scale"), kw.get("out_dtype"), kw.get("epilogue"))


def _void_spmm_activation_row_bias(a, b: torch.Tensor, bias: Optional[torch.Tensor], out: Optional[torch.Tensor],
                                   activation: str) -> torch.Tensor:
    """activation(A @ B + bias[:, None]) with a per-row bias [M] for float A
    (fusion.py:307-377): the fp32 kernel with bias_per_row, output in B's dtype;
    B is made contiguous as the reference does."""
    from .format import VOIDTensor
    from .ops import float_spmm
    if not isinstance(a, VOIDTensor):
        raise TypeError("the row-bias activation SpMM takes a float VOIDTensor")
    b = b.contiguous()
    if a.n_blocks == 0:
        res = torch.zeros(a.shape[0], b.shape[1], dtype=b.dtype, device=b.device) if out is None else out.zero_()
        if bias is not None:
            res[:, :] = bias[:, None]
            res = apply_activation_torch(res, activation)
            if out is not None and res is not out:
                out.copy_(res)
                res = out
        return res
    return float_spmm(a, b, out=out, bias=bias, activation=get_activation_code(activation), bias_per_row=True)


class FusedSparseLinear(torch.nn.Module):
    """Sparse linear layer y = activation(W x + b) in one kernel
    (fusion.py:756-836): W is a float VOIDTensor [out_features, in_features],
    b a per-output-feature (row) bias, the product W @ x^T runs on the fp32
    MFMA kernel with the bias and activation fused (void_spmm_f32 with
    bias_per_row), as the reference's row-bias activation kernel does
    (fusion.py:202-304).  Buffers and fields match the reference so that its
    state dicts load; ``from_packed`` loads a packed BSR blob straight into
    the device layout."""

    def __init__(self, in_features: int, out_features: int, void_tensor, activation: str = "gelu",
                 bias: bool = True):
        super().__init__()
        if tuple(void_tensor.shape) != (out_features, in_features):
            raise ValueError(f"weight is {tuple(void_tensor.shape)}, expected ({out_features}, {in_features})")
        self.in_features = in_features
        self.out_features = out_features
        self.activation = activation
        self.register_buffer("values", void_tensor.values.clone())
        self.register_buffer("block_rows", void_tensor.block_rows)
        self.register_buffer("block_cols", void_tensor.block_cols)
        self.register_buffer("morton_codes", void_tensor.morton_codes)
        self.shape = void_tensor.shape
        self.tile_size = void_tensor.tile_size
        self.n_blocks = void_tensor.n_blocks
        if bias:
            self.bias = torch.nn.Parameter(torch.zeros(out_features))
        else:
            self.register_parameter("bias", None)
        self._vt = None
        if getattr(void_tensor, "_device_bsr", None):
            self._vt = self.get_void_tensor()
            self._vt._device_bsr.update(void_tensor._device_bsr)

    @classmethod
    def from_packed(cls, blob_or_path, device="cuda", activation: str = "gelu", bias: bool = True):
        from .packed import load_packed, unpack
        vt = unpack(blob_or_path, device) if isinstance(blob_or_path, (bytes, bytearray, memoryview)) \
            else load_packed(blob_or_path, device)
        out_f, in_f = vt.shape
        return cls(in_f, out_f, vt, activation=activation, bias=bias).to(device)

    def get_void_tensor(self):
        """The weight as a VOIDTensor over the module's buffers (fusion.py:793-806)."""
        from .format import VOIDTensor
        vt = self._vt
        if vt is None or vt.values is not self.values:
            vt = VOIDTensor(values=self.values, block_rows=self.block_rows, block_cols=self.block_cols,
                            morton_codes=self.morton_codes, shape=tuple(self.shape), tile_size=tuple(self.tile_size),
                            nnz_original=0, n_blocks=self.n_blocks, density=0.0, dtype=self.values.dtype)
            self._vt = vt
        return vt

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        from .ops import float_spmm
        x_flat = x.reshape(-1, self.in_features)
        b = x_flat.t().contiguous()  # [in, batch], row-major, as the reference passes it
        bias = self.bias.detach() if self.bias is not None else None
        vt = self.get_void_tensor()
        if vt.n_blocks == 0:
            y = torch.zeros(self.out_features, b.shape[1], dtype=b.dtype, device=b.device)
            if bias is not None:
                y = apply_activation_torch(y + bias[:, None].to(y.dtype), self.activation)
        else:
            y = _void_spmm_activation_row_bias(vt, b, bias, None, self.activation)
        return y.t().reshape(x.shape[:-1] + (self.out_features,))

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"activation={self.activation}, bias={self.bias is not None}")


__all__ = ["ActivationType", "FusedSparseLinear", "get_activation_code", "gelu_tanh", "void_spmm_gelu",
           "void_spmm_relu", "void_spmm_silu"]
