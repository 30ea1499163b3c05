"""FP8 (E4M3 / E5M2) quantisation of VOID tensors and the FP8 block-sparse SpMM.

Mirrors ``void/fp8.py``: FP8Config / FP8ScalingInfo with the amax-history
scaling rule, quantize_to_fp8 / dequantize_from_fp8, FP8VOIDTensor and
void_spmm_fp8.  The reference kernel upcasts the FP8 tiles to fp32 and runs
an fp32 (TF32) dot (fp8.py:577-671); here an E4M3 B operand feeds gfx950's
fp8 x fp8 MFMA with fp32 accumulation directly, and per-tile scales are
applied to each tile's fp32 partial product in registers.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum
from typing import Dict, Literal, Optional, Tuple, Union

import torch

from . import _lib, _runtime, tuning


class FP8Format(Enum):
    E4M3 = "e4m3"
    E5M2 = "e5m2"


FP8_MAX = {FP8Format.E4M3: 448.0, FP8Format.E5M2: 57344.0}
FP8_MIN = {FP8Format.E4M3: -448.0, FP8Format.E5M2: -57344.0}


@dataclass
class FP8Config:
    """fp8.py:37-66."""
    format: FP8Format = FP8Format.E4M3
    scale_mode: Literal["per_tensor", "per_block", "per_row"] = "per_tensor"
    margin: float = 0.0
    amax_history_len: int = 16

    @property
    def max_value(self) -> float:
        return FP8_MAX[self.format]

    @property
    def torch_dtype(self) -> torch.dtype:
        return torch.float8_e4m3fn if self.format == FP8Format.E4M3 else torch.float8_e5m2


@dataclass
class FP8ScalingInfo:
    """Scale, inverse scale and amax history (fp8.py:69-105)."""
    scale: torch.Tensor
    scale_inv: torch.Tensor
    amax: torch.Tensor
    amax_history: torch.Tensor
    config: FP8Config = field(default_factory=FP8Config)

    def update_amax(self, new_amax: torch.Tensor) -> None:
        self.amax_history = torch.roll(self.amax_history, shifts=1, dims=-1)
        if self.amax_history.dim() == 1:
            self.amax_history[0] = new_amax
        else:
            self.amax_history[..., 0] = new_amax
        self.amax = new_amax

    def compute_scale(self) -> Tuple[torch.Tensor, torch.Tensor]:
        if self.amax_history.dim() == 1:
            smoothed = self.amax_history.max()
        else:
            smoothed = self.amax_history.max(dim=-1).values
        fp8_max = self.config.max_value * (1.0 - self.config.margin)
        self.scale = torch.clamp(smoothed / fp8_max, min=1e-12)
        self.scale_inv = 1.0 / self.scale
        return self.scale, self.scale_inv


def create_scaling_info(shape: Tuple[int, ...], config: FP8Config,
                        device: Union[str, torch.device] = "cuda") -> FP8ScalingInfo:
    """fp8.py:108-152."""
    if config.scale_mode == "per_tensor":
        scale_shape: Tuple[int, ...] = ()
    elif config.scale_mode in ("per_block", "per_row"):
        scale_shape = (shape[0],)
    else:
        raise ValueError(f"Unknown scale_mode: {config.scale_mode}")
    hist = (config.amax_history_len,) if scale_shape == () else scale_shape + (config.amax_history_len,)
    return FP8ScalingInfo(
        scale=torch.ones(scale_shape, dtype=torch.float32, device=device),
        scale_inv=torch.ones(scale_shape, dtype=torch.float32, device=device),
        amax=torch.zeros(scale_shape, dtype=torch.float32, device=device),
        amax_history=torch.zeros(hist, dtype=torch.float32, device=device),
        config=config)


def compute_amax(tensor: torch.Tensor, scale_mode: str = "per_tensor") -> torch.Tensor:
    """fp8.py:159-182."""
    if scale_mode == "per_tensor":
        return tensor.abs().max()
    if scale_mode in ("per_block", "per_row"):
        return tensor.view(tensor.shape[0], -1).abs().max(dim=1).values
    raise ValueError(f"Unknown scale_mode: {scale_mode}")


def quantize_to_fp8(tensor: torch.Tensor, config: Optional[FP8Config] = None,
                    scaling_info: Optional[FP8ScalingInfo] = None) -> Tuple[torch.Tensor, FP8ScalingInfo]:
    """clamp(x * scale_inv, +-max).to(fp8) with amax-history scaling (fp8.py:185-229)."""
    config = config or FP8Config()
    if scaling_info is None:
        scaling_info = create_scaling_info(tensor.shape, config, tensor.device)
    scaling_info.update_amax(compute_amax(tensor, config.scale_mode))
    _, scale_inv = scaling_info.compute_scale()
    if config.scale_mode == "per_tensor":
        scaled = tensor * scale_inv
    else:
        scaled = tensor * scale_inv.view((tensor.shape[0],) + (1,) * (tensor.dim() - 1))
    scaled = torch.clamp(scaled, -config.max_value, config.max_value)
    return scaled.to(config.torch_dtype), scaling_info


def dequantize_from_fp8(tensor: torch.Tensor, scaling_info: FP8ScalingInfo,
                        output_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """fp32(x) * scale (fp8.py:232-257)."""
    f = tensor.to(torch.float32)
    if scaling_info.config.scale_mode == "per_tensor":
        r = f * scaling_info.scale
    else:
        r = f * scaling_info.scale.view((tensor.shape[0],) + (1,) * (tensor.dim() - 1))
    return r.to(output_dtype)


@dataclass
class FP8VOIDTensor:
    """VOID tensor with FP8 tiles (fp8.py:438-570)."""
    values_fp8: torch.Tensor
    scaling_info: FP8ScalingInfo
    block_rows: torch.Tensor
    block_cols: torch.Tensor
    morton_codes: torch.Tensor
    shape: Tuple[int, int]
    tile_size: Tuple[int, int]
    nnz_original: int
    n_blocks: int
    density: float
    _device_bsr: Dict[str, "_runtime.DeviceBsr"] = field(default_factory=dict, repr=False)

    @classmethod
    def from_void_tensor(cls, void_tensor, config: Optional[FP8Config] = None) -> "FP8VOIDTensor":
        config = config or FP8Config(scale_mode="per_block")
        if (config.format == FP8Format.E4M3 and config.scale_mode == "per_block" and config.margin == 0.0
                and _runtime.device_tile_quant_ok(void_tensor.values)):
            # GPU tiles: the gfx950 quantiser (void_quantize_tiles_fp8).  Its
            # scale is the true fp32 quotient amax / 448, as the reference
            # computes on the CPU; torch on a GPU divides a tensor by a Python
            # scalar as a multiplication by the reciprocal, which can differ in
            # the last bit, so the scale is taken from the kernel, not from
            # compute_scale().
            codes, scale, amax = _runtime.quantize_tiles_fp8(void_tensor.values)
            info = create_scaling_info(void_tensor.values.shape, config, void_tensor.values.device)
            info.update_amax(amax)
            info.scale = scale
            info.scale_inv = 1.0 / scale
            values_fp8 = codes.view(config.torch_dtype)
        else:
            values_fp8, info = quantize_to_fp8(void_tensor.values, config=config)
        return cls(values_fp8=values_fp8, scaling_info=info, block_rows=void_tensor.block_rows,
                   block_cols=void_tensor.block_cols, morton_codes=void_tensor.morton_codes,
                   shape=void_tensor.shape, tile_size=void_tensor.tile_size,
                   nnz_original=void_tensor.nnz_original, n_blocks=void_tensor.n_blocks,
                   density=void_tensor.density)

    def to_void_tensor(self, output_dtype: torch.dtype = torch.float16):
        from .format import VOIDTensor
        values = dequantize_from_fp8(self.values_fp8, self.scaling_info, output_dtype=output_dtype)
        return VOIDTensor(values=values, block_rows=self.block_rows, block_cols=self.block_cols,
                          morton_codes=self.morton_codes, shape=self.shape, tile_size=self.tile_size,
                          nnz_original=self.nnz_original, n_blocks=self.n_blocks, density=self.density,
                          dtype=output_dtype)

    def to(self, device: Union[str, torch.device]) -> "FP8VOIDTensor":
        si = self.scaling_info
        return FP8VOIDTensor(
            values_fp8=self.values_fp8.to(device),
            scaling_info=FP8ScalingInfo(scale=si.scale.to(device), scale_inv=si.scale_inv.to(device),
                                        amax=si.amax.to(device), amax_history=si.amax_history.to(device),
                                        config=si.config),
            block_rows=self.block_rows.to(device), block_cols=self.block_cols.to(device),
            morton_codes=self.morton_codes.to(device), shape=self.shape, tile_size=self.tile_size,
            nnz_original=self.nnz_original, n_blocks=self.n_blocks, density=self.density)

    def cuda(self) -> "FP8VOIDTensor":
        return self.to("cuda")

    @property
    def memory_bytes(self) -> int:
        return (self.values_fp8.numel() + self.scaling_info.scale.numel() * 4
                + (self.block_rows.numel() + self.block_cols.numel()) * 4)

    def device_bsr(self) -> "_runtime.DeviceBsr":
        """Block-row-major device copy of the tiles (built once per device,
        gathered again when the codes or scales change in place)."""
        key = str(self.values_fp8.device)
        scales = self.scaling_info.scale.reshape(-1)
        src = _runtime.source_key(self.values_fp8, self.scaling_info.scale)
        d = self._device_bsr.get(key)
        if d is None:
            if self.values_fp8.dtype != torch.float8_e4m3fn:
                raise NotImplementedError(f"the FP8 kernel takes E4M3FN tiles, got {self.values_fp8.dtype}")
            per_tensor = self.scaling_info.config.scale_mode == "per_tensor"
            d = _runtime.make_device_bsr(self.values_fp8, scales, self.block_rows, self.block_cols,
                                         self.shape, self.tile_size, self.values_fp8.device, per_tensor)
            d.src_key = src
            self._device_bsr[key] = d
        elif d.src_key != src:
            d.refresh(self.values_fp8, scales)
            d.src_key = src
        return d

    def __repr__(self) -> str:
        return (f"FP8VOIDTensor(shape={self.shape}, tile_size={self.tile_size}, n_blocks={self.n_blocks}, "
                f"format={self.scaling_info.config.format.value}, "
                f"scale_mode={self.scaling_info.config.scale_mode})")


def quantize_dense_fp8(b: torch.Tensor) -> Tuple[torch.Tensor, float]:
    """Per-tensor E4M3 quantisation of a dense operand: (fp8 tensor, scale)."""
    q, info = quantize_to_fp8(b.float(), FP8Config(scale_mode="per_tensor"))
    return q, float(info.scale.item())


def void_spmm_fp8(a: FP8VOIDTensor, b: torch.Tensor, output_dtype: torch.dtype = torch.float16, *,
                  b_scale: Optional[Union[float, torch.Tensor]] = None, activation: str = "none",
                  bias: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                  chunk_tiles: Optional[int] = None) -> torch.Tensor:
    """FP8 block-sparse SpMM C = A @ B (fp8.py:674-742) on the gfx950 kernels.

    A float B (fp32, bf16, fp16) keeps the reference's semantics: the kernel
    computes sum_t s_t dec(A_t) @ B with B as given (fp8.py:624-671 upcasts
    both operands).  A bf16 / fp16 B runs on the 16-bit MFMA with A decoded
    exactly to its type (exact products); an fp32 B on the bf16 MFMA with A
    decoded exactly and B split into bf16 hi + lo (within 2^-16 relative per
    product).
    A float8_e4m3fn B runs on the fp8 x fp8 MFMA and is taken as the codes'
    values, as the reference's upcast does.
    b_scale (default 1.0; a scalar or N per-column scales) multiplies the
    result in either case.  Output dtype float32 / bfloat16 / float16.
    """
    if b.dim() != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"B must be [K={a.shape[1]}, N], got {tuple(b.shape)}")
    M, K = a.shape
    N = b.shape[1]
    if bias is not None and tuple(bias.shape) != (N,):
        raise ValueError(f"bias must be [{N}], got {tuple(bias.shape)}")
    _runtime.require_gpu(b, "B")
    if b.dtype == torch.float8_e5m2:
        raise NotImplementedError("E5M2 B operands are not supported by the gfx950 kernels")
    float_b = b.dtype != torch.float8_e4m3fn
    if float_b and not b.is_floating_point():
        raise TypeError(f"B must be float8_e4m3fn or a float tensor, got {b.dtype}")
    from .int_quant import _b_scale_args
    scalar_scale, scale_vec, _ = _b_scale_args(b_scale, N, b.device)
    if out is None:
        out = torch.empty(M, N, dtype=output_dtype, device=b.device)
    elif out.shape != (M, N) or out.dtype != output_dtype:
        raise ValueError(f"out must be [{M}, {N}] {output_dtype}")
    if a.n_blocks == 0:
        out.zero_()
        if bias is not None or activation != "none":
            from .fusion import apply_activation_torch
            out.copy_(apply_activation_torch(out.float() + (bias if bias is not None else 0), activation))
        return out
    _runtime.require_gpu(a.values_fp8, "A")
    if a.values_fp8.device != b.device:
        raise ValueError(f"A on {a.values_fp8.device}, B on {b.device}")
    from .fusion import get_activation_code
    if bias is not None:
        bias = bias.to(device=b.device, dtype=torch.float32).contiguous()
    dbsr = a.device_bsr()
    chunk = chunk_tiles or tuning.select_chunk("fp8", a.n_blocks, N, dbsr.max_row)
    act = get_activation_code(activation)
    if not float_b:
        return _runtime.launch("fp8", dbsr, b.view(torch.uint8), b_scale=scalar_scale,
                               b_scale_vec=scale_vec, out=out, epilogue=_lib.EPI_PER_BLOCK, activation=act,
                               bias=bias, chunk=chunk)
    if chunk > tuning.FP32_B_MAX_CHUNK:
        raise ValueError(f"a float B takes chunk_tiles <= {tuning.FP32_B_MAX_CHUNK}, got {chunk}")
    if b.dtype in (torch.bfloat16, torch.float16):
        # A 16-bit B is taken as it is, on the 16-bit MFMA (A decoded exactly
        # to its type), when its rows and the output's are 16-byte aligned
        # and N % 8 == 0; otherwise it is widened to fp32 below.
        b16 = b if b.stride(1) == 1 else b.contiguous()
        if (N % 8 == 0 and b16.stride(0) % 8 == 0 and b16.data_ptr() % 16 == 0 and a.n_blocks * 1024 < (1 << 31)
                and (K + 31) // 32 * 32 * b16.stride(0) * 2 < (1 << 31) and M * N * out.element_size() < (1 << 31)):
            kind = "fp8_bf16b" if b.dtype == torch.bfloat16 else "fp8_f16b"
            aligned = out.stride(1) == 1 and out.data_ptr() % 16 == 0 and out.stride(0) % 4 == 0
            tgt = out if aligned else torch.empty(M, N, dtype=output_dtype, device=b.device)
            _runtime.launch(kind, dbsr, b16, b_scale=scalar_scale, b_scale_vec=scale_vec,
                            out=tgt, epilogue=_lib.EPI_PER_BLOCK, activation=act, bias=bias, chunk=chunk)
            if tgt is not out:
                out.copy_(tgt)
            return out
    # fp32 B, row-major with 16-byte aligned rows and N % 4 == 0 (the ring
    # kernel's layout); other widths run on zero-padded columns.  The kernel
    # addresses B and C with 31-bit byte offsets: a larger B or C runs in
    # column slices that fit, each B slice copied contiguous and each result
    # slice copied into place.
    lim = 1 << 31
    k_rows = (K + 31) // 32 * 32
    esz = out.element_size()
    width = N
    if k_rows * ((N + 3) // 4 * 4) * 4 >= lim or M * ((N + 3) // 4 * 4) * esz >= lim:
        width = min((lim - 1) // (k_rows * 4), (lim - 1) // max(M * esz, 1)) // 128 * 128
        if width < 128:
            raise ValueError(f"fp8 SpMM with an fp32 B: K={K} or M={M} too large for 31-bit offsets")
    for n0 in range(0, N, width):
        n1 = min(N, n0 + width)
        whole = n0 == 0 and n1 == N
        _launch_f32b(dbsr, b if whole else b[:, n0:n1], out if whole else None, output_dtype, scalar_scale,
                     None if scale_vec is None else scale_vec[n0:n1], act, None if bias is None else bias[n0:n1],
                     chunk, dst=out[:, n0:n1])
    return out


def _launch_f32b(dbsr, b: torch.Tensor, out: Optional[torch.Tensor], output_dtype: torch.dtype, scalar_scale: float,
                 scale_vec: Optional[torch.Tensor], act: int, bias: Optional[torch.Tensor], chunk: int,
                 dst: torch.Tensor) -> None:
    """One E4M3 x fp32-B launch over B's columns, written to dst.  out, when
    given, is dst itself and takes the result directly (N % 4 == 0)."""
    K, N = b.shape
    M = dst.shape[0]
    N4 = (N + 3) // 4 * 4
    if N4 == N:
        b32 = b.to(torch.float32).contiguous()
        if b32.data_ptr() % 16:
            b32 = b32.clone()
        tgt = out if out is not None else torch.empty(M, N, dtype=output_dtype, device=b.device)
        _runtime.launch("fp8_f32b", dbsr, b32, b_scale=scalar_scale, b_scale_vec=scale_vec,
                        out=tgt, epilogue=_lib.EPI_PER_BLOCK, activation=act, bias=bias, chunk=chunk)
        if out is None:
            dst.copy_(tgt)
        return
    b32 = torch.zeros(K, N4, dtype=torch.float32, device=b.device)
    b32[:, :N] = b
    pad = lambda v, fill: torch.cat([v, torch.full((N4 - N,), fill, dtype=v.dtype, device=v.device)])
    wide = torch.empty(M, N4, dtype=output_dtype, device=b.device)
    _runtime.launch("fp8_f32b", dbsr, b32, b_scale=scalar_scale,
                    b_scale_vec=None if scale_vec is None else pad(scale_vec, 1.0), out=wide,
                    epilogue=_lib.EPI_PER_BLOCK, activation=act, bias=None if bias is None else pad(bias, 0.0),
                    chunk=chunk)
    dst.copy_(wide[:, :N])


def void_tensor_to_fp8(void_tensor, format: str = "e4m3", scale_mode: str = "per_block") -> FP8VOIDTensor:
    """fp8.py:749-766."""
    fmt = FP8Format.E4M3 if format == "e4m3" else FP8Format.E5M2
    return FP8VOIDTensor.from_void_tensor(void_tensor, FP8Config(format=fmt, scale_mode=scale_mode))


__all__ = [
    "FP8Format", "FP8_MAX", "FP8_MIN", "FP8Config", "FP8ScalingInfo", "FP8VOIDTensor",
    "create_scaling_info", "compute_amax", "quantize_to_fp8", "dequantize_from_fp8",
    "quantize_dense_fp8", "void_spmm_fp8", "void_tensor_to_fp8",
]
