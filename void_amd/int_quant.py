"""INT8 quantisation of VOID tensors and the INT8 block-sparse SpMM.

Mirrors ``void/int_quant.py``: the same config/dataclass names and the same
quantisation arithmetic (min-max, ``round`` half-to-even, clamp), with the
per-block Python loop of ``quantize_void_tensor`` (int_quant.py:363-369)
replaced by one batched computation that produces bit-identical results.
``void_spmm_int8`` launches the gfx950 kernel of ``libvoid_amd.so``.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum
from typing import Dict, Literal, Optional, Tuple, Union

import torch

from . import _lib, _runtime, tuning


class IntFormat(Enum):
    """Integer formats (int_quant.py:12-17)."""
    INT8 = "int8"
    UINT8 = "uint8"
    INT4 = "int4"
    UINT4 = "uint4"


class ScaleMode(Enum):
    """Scale granularity (int_quant.py:20-24)."""
    PER_TENSOR = "per_tensor"
    PER_CHANNEL = "per_channel"
    PER_BLOCK = "per_block"


@dataclass
class IntQuantConfig:
    """Quantisation configuration (int_quant.py:27-80)."""
    format: IntFormat = IntFormat.INT8
    symmetric: bool = True
    scale_mode: ScaleMode = ScaleMode.PER_BLOCK
    calibration_method: Literal["minmax", "percentile", "mse"] = "minmax"
    percentile: float = 99.9

    @property
    def bits(self) -> int:
        return 8 if self.format in (IntFormat.INT8, IntFormat.UINT8) else 4

    @property
    def is_signed(self) -> bool:
        return self.format in (IntFormat.INT8, IntFormat.INT4)

    @property
    def qmin(self) -> int:
        return {IntFormat.INT8: -128, IntFormat.UINT8: 0, IntFormat.INT4: -8, IntFormat.UINT4: 0}[self.format]

    @property
    def qmax(self) -> int:
        return {IntFormat.INT8: 127, IntFormat.UINT8: 255, IntFormat.INT4: 7, IntFormat.UINT4: 15}[self.format]


@dataclass
class QuantizationParams:
    """x = (q - zero_point) * scale (int_quant.py:83-102)."""
    scale: torch.Tensor
    zero_point: torch.Tensor
    config: IntQuantConfig
    original_shape: Tuple[int, ...]

    def to(self, device) -> "QuantizationParams":
        return QuantizationParams(self.scale.to(device), self.zero_point.to(device), self.config,
                                  self.original_shape)


@dataclass
class Int8VOIDTensor:
    """Quantised VOID tensor (int_quant.py:105-175).

    values int8 [n_blocks, 32, 32] in the Morton order of the source VOIDTensor,
    scales float32 [n_blocks] (per block) or an expanded per-tensor scale.
    """
    values: torch.Tensor
    scales: torch.Tensor
    zero_points: torch.Tensor
    block_rows: torch.Tensor
    block_cols: torch.Tensor
    shape: Tuple[int, int]
    tile_size: Tuple[int, int]
    n_blocks: int
    config: IntQuantConfig
    _row_ptr: Optional[torch.Tensor] = None
    _block_indices: Optional[torch.Tensor] = None
    _device_bsr: Dict[str, "_runtime.DeviceBsr"] = field(default_factory=dict, repr=False)

    @property
    def device(self) -> torch.device:
        return self.values.device

    @property
    def dtype(self) -> torch.dtype:
        return self.values.dtype

    @property
    def block_grid(self) -> Tuple[int, int]:
        return ((self.shape[0] + self.tile_size[0] - 1) // self.tile_size[0],
                (self.shape[1] + self.tile_size[1] - 1) // self.tile_size[1])

    def to(self, device: Union[str, torch.device]) -> "Int8VOIDTensor":
        return Int8VOIDTensor(
            values=self.values.to(device), scales=self.scales.to(device),
            zero_points=self.zero_points.to(device), block_rows=self.block_rows.to(device),
            block_cols=self.block_cols.to(device), shape=self.shape, tile_size=self.tile_size,
            n_blocks=self.n_blocks, config=self.config)

    def cuda(self) -> "Int8VOIDTensor":
        return self.to("cuda")

    def get_row_block_info(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """(row_ptr, block_indices), block_indices = argsort(row * n_bc + col) (int_quant.py:158-175)."""
        if self._row_ptr is None or self._block_indices is None:
            n_br, n_bc = self.block_grid
            counts = torch.zeros(n_br, dtype=torch.int32, device=self.device)
            counts.scatter_add_(0, self.block_rows.long(), torch.ones_like(self.block_rows))
            self._row_ptr = torch.zeros(n_br + 1, dtype=torch.int32, device=self.device)
            self._row_ptr[1:] = torch.cumsum(counts, dim=0)
            keys = self.block_rows.long() * n_bc + self.block_cols.long()
            self._block_indices = torch.argsort(keys, stable=True).to(torch.int32)
        return self._row_ptr, self._block_indices

    def device_bsr(self) -> "_runtime.DeviceBsr":
        """Block-row-major device copy of the tiles (built once per device,
        gathered again when the values or scales change in place, since the
        reference reads them on every call)."""
        key = str(self.values.device)
        src = _runtime.source_key(self.values, self.scales)
        d = self._device_bsr.get(key)
        if d is not None and d.src_key != src:
            d.refresh(self.values, self.scales)
            d.src_key = src
        if d is None:
            if self.values.dtype != torch.int8:
                raise NotImplementedError(
                    f"the INT8 kernel takes int8 tiles; {self.config.format.value} values are stored as "
                    f"{self.values.dtype}")
            if not self.config.symmetric:
                raise NotImplementedError("the INT8 kernel takes symmetric (zero-point 0) quantisation")
            per_tensor = self.config.scale_mode == ScaleMode.PER_TENSOR
            d = _runtime.make_device_bsr(self.values, self.scales, self.block_rows, self.block_cols,
                                         self.shape, self.tile_size, self.values.device, per_tensor)
            d.src_key = src
            self._device_bsr[key] = d
        return d


def compute_scale_minmax(tensor: torch.Tensor, config: IntQuantConfig,
                         dim: Optional[Union[int, Tuple[int, ...]]] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Min-max scale / zero point (int_quant.py:178-214)."""
    if dim is not None:
        min_val = tensor.amin(dim=dim, keepdim=True)
        max_val = tensor.amax(dim=dim, keepdim=True)
    else:
        min_val = tensor.min()
        max_val = tensor.max()
    if config.symmetric:
        abs_max = torch.maximum(min_val.abs(), max_val.abs())
        scale = abs_max / max(abs(config.qmin), config.qmax)
        zero_point = torch.zeros_like(scale, dtype=torch.int8)
    else:
        scale = (max_val - min_val) / (config.qmax - config.qmin)
        zero_point = (config.qmin - min_val / scale).round().to(torch.int8)
    scale = torch.clamp(scale, min=1e-8)
    return scale, zero_point


def compute_scale_percentile(tensor: torch.Tensor, config: IntQuantConfig,
                             dim: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Percentile-clipped scale (int_quant.py:217-251)."""
    p_low = (100 - config.percentile) / 2
    p_high = 100 - p_low
    if dim is not None:
        shape = tensor.shape
        flat = tensor.transpose(dim, -1).reshape(-1, shape[dim])
        min_val = torch.quantile(flat, p_low / 100, dim=0)
        max_val = torch.quantile(flat, p_high / 100, dim=0)
        min_val = min_val.view(*shape[:dim], 1, *shape[dim + 1:])
        max_val = max_val.view(*shape[:dim], 1, *shape[dim + 1:])
    else:
        min_val = torch.quantile(tensor.flatten(), p_low / 100)
        max_val = torch.quantile(tensor.flatten(), p_high / 100)
    if config.symmetric:
        abs_max = torch.maximum(min_val.abs(), max_val.abs())
        scale = abs_max / max(abs(config.qmin), config.qmax)
        zero_point = torch.zeros_like(scale, dtype=torch.int8)
    else:
        scale = (max_val - min_val) / (config.qmax - config.qmin)
        zero_point = (config.qmin - min_val / scale).round().to(torch.int8)
    scale = torch.clamp(scale, min=1e-8)
    return scale, zero_point


def _apply_quant(tensor: torch.Tensor, scale: torch.Tensor, zero_point: torch.Tensor,
                 config: IntQuantConfig) -> torch.Tensor:
    if config.symmetric:
        q = (tensor / scale).round().clamp(config.qmin, config.qmax)
    else:
        q = ((tensor / scale) + zero_point.float()).round().clamp(config.qmin, config.qmax)
    return q.to(torch.int8 if config.format in (IntFormat.INT8, IntFormat.INT4) else torch.uint8)


def quantize_tensor(tensor: torch.Tensor, config: IntQuantConfig) -> Tuple[torch.Tensor, QuantizationParams]:
    """Quantise a tensor (int_quant.py:254-305)."""
    if config.scale_mode == ScaleMode.PER_CHANNEL:
        dim = tuple(range(1, tensor.dim()))
    else:
        dim = None
    if config.calibration_method == "minmax":
        scale, zero_point = compute_scale_minmax(tensor, config, dim)
    elif config.calibration_method == "percentile":
        scale, zero_point = compute_scale_percentile(tensor, config, dim)
    else:
        raise ValueError(f"Unknown calibration method: {config.calibration_method}")
    q = _apply_quant(tensor, scale, zero_point, config)
    return q, QuantizationParams(scale=scale.to(torch.float32), zero_point=zero_point, config=config,
                                 original_shape=tensor.shape)


def quantize_per_column(b: torch.Tensor, config: Optional[IntQuantConfig] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Symmetric INT8 quantisation of a K x N matrix with one scale per column.

    The per-column analogue of quantize_tensor's min-max rule: scale[n] =
    max(|min_k b|, |max_k b|) / 128 clamped at 1e-8, q = clamp(round(b / scale)).
    Used for B operands with per-column (per-token) scales.
    """
    config = config or IntQuantConfig(scale_mode=ScaleMode.PER_CHANNEL)
    scale, zp = compute_scale_minmax(b, config, dim=0)
    return _apply_quant(b, scale, zp, config), scale.reshape(-1).to(torch.float32)


def dequantize_tensor(quantized: torch.Tensor, params: QuantizationParams) -> torch.Tensor:
    """q * scale, or (q - zp) * scale (int_quant.py:308-325)."""
    if params.config.symmetric:
        return quantized.float() * params.scale
    return (quantized.float() - params.zero_point.float()) * params.scale


def quantize_void_tensor(void_tensor, config: Optional[IntQuantConfig] = None) -> Int8VOIDTensor:
    """Quantise a VOIDTensor (int_quant.py:328-388), all blocks at once.

    PER_BLOCK: the reference quantises every tile separately with the
    per-tensor rule; the batched amin/amax over each tile gives the same
    scale and the same elementwise quantisation.
    """
    if config is None:
        config = IntQuantConfig(format=IntFormat.INT8, symmetric=True, scale_mode=ScaleMode.PER_BLOCK)
    n_blocks = void_tensor.n_blocks
    tm, tk = void_tensor.tile_size
    values = void_tensor.values
    if config.scale_mode == ScaleMode.PER_BLOCK:
        if config.calibration_method != "minmax":
            raise ValueError(f"per-block quantisation uses minmax calibration, got {config.calibration_method}")
        if (config.format == IntFormat.INT8 and config.symmetric
                and _runtime.device_tile_quant_ok(values)):
            # GPU tiles: the gfx950 quantiser (void_quantize_tiles_i8), same arithmetic.
            q, scales = _runtime.quantize_tiles_i8(values)
            zero_points = torch.zeros(n_blocks, dtype=torch.int8, device=values.device)
        elif n_blocks:
            scale, zp = compute_scale_minmax(values, config, dim=(1, 2))
            q = _apply_quant(values, scale, zp, config)
            scales = scale.reshape(n_blocks).to(torch.float32)
            zero_points = (zp.reshape(n_blocks).to(torch.int8) if not config.symmetric
                           else torch.zeros(n_blocks, dtype=torch.int8, device=values.device))
        else:
            q = torch.zeros_like(values, dtype=torch.int8)
            scales = torch.zeros(0, dtype=torch.float32, device=values.device)
            zero_points = torch.zeros(0, dtype=torch.int8, device=values.device)
    else:
        q_flat, params = quantize_tensor(values.reshape(-1), config)
        q = q_flat.view(n_blocks, tm, tk)
        scales = params.scale.expand(n_blocks)
        zero_points = (params.zero_point.expand(n_blocks) if not config.symmetric
                       else torch.zeros(n_blocks, dtype=torch.int8, device=values.device))
    return Int8VOIDTensor(values=q, scales=scales, zero_points=zero_points,
                          block_rows=void_tensor.block_rows.clone(), block_cols=void_tensor.block_cols.clone(),
                          shape=void_tensor.shape, tile_size=void_tensor.tile_size, n_blocks=n_blocks,
                          config=config)


def dequantize_void_tensor(int8_tensor: Int8VOIDTensor):
    """Int8VOIDTensor -> float VOIDTensor (int_quant.py:391-428).

    The reference builds VOIDTensor without its required morton_codes /
    nnz_original / density fields and raises TypeError; this version fills
    them in (Morton codes recomputed, nnz counted from the dequantised tiles).
    """
    from .format import VOIDTensor, morton_encode_batch
    q = int8_tensor.values.float()
    s = int8_tensor.scales.reshape(-1, 1, 1)
    if int8_tensor.config.symmetric:
        values = q * s
    else:
        values = (q - int8_tensor.zero_points.float().reshape(-1, 1, 1)) * s
    br = int8_tensor.block_rows.cpu().numpy()
    bc = int8_tensor.block_cols.cpu().numpy()
    n_br, n_bc = int8_tensor.block_grid
    return VOIDTensor(
        values=values, block_rows=int8_tensor.block_rows.clone(), block_cols=int8_tensor.block_cols.clone(),
        morton_codes=torch.from_numpy(morton_encode_batch(br, bc).astype("int64")).to(values.device),
        shape=int8_tensor.shape, tile_size=int8_tensor.tile_size,
        nnz_original=int((values != 0).sum().item()), n_blocks=int8_tensor.n_blocks,
        density=int8_tensor.n_blocks / max(n_br * n_bc, 1))


def _b_scale_args(b_scale, N: int, device) -> Tuple[float, Optional[torch.Tensor], bool]:
    """Split a B scale into (scalar, per-column tensor or None, per-column?).

    A one-element tensor is a per-tensor scale: it reaches the kernel as N
    copies on the device (the same products as the scalar, without reading
    it back to the host, which would stall the stream and break graph
    capture), and keeps the per-tensor defaults."""
    if b_scale is None:
        return 1.0, None, False
    if isinstance(b_scale, torch.Tensor):
        if b_scale.numel() == 1 and b_scale.dim() <= 1 and N != 1:
            return 1.0, b_scale.reshape(1).to(device=device, dtype=torch.float32).expand(N).contiguous(), False
        if b_scale.numel() != N:
            raise ValueError(f"b_scale has {b_scale.numel()} entries, expected 1 or N={N}")
        return 1.0, b_scale.reshape(-1).to(device=device, dtype=torch.float32).contiguous(), True
    return float(b_scale), None, False


def _quantize_b_per_tensor(b: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """A float B quantised per tensor as the reference does (symmetric int8,
    min-max scale), the scale left on the device: for a contiguous fp32 B
    on the gfx950 kernels (void_quantize_b_i8), otherwise with quantize_tensor."""
    if b.dtype == torch.float32 and b.is_contiguous() and b.data_ptr() % 16 == 0:
        q = torch.empty(b.shape, dtype=torch.int8, device=b.device)
        scale = torch.empty(1, dtype=torch.float32, device=b.device)
        partials = torch.empty(1024, dtype=torch.int32, device=b.device)
        st = _lib.lib().void_quantize_b_i8(b.data_ptr(), b.numel(), q.data_ptr(), scale.data_ptr(),
                                           partials.data_ptr(), torch.cuda.current_stream(b.device).cuda_stream)
        _lib.check(st, "void_quantize_b_i8")
        return q, scale
    cfg = IntQuantConfig(format=IntFormat.INT8, symmetric=True, scale_mode=ScaleMode.PER_TENSOR)
    q, params = quantize_tensor(b, cfg)
    return q, params.scale.reshape(1)


def void_spmm_int8(
    a: Int8VOIDTensor,
    b: torch.Tensor,
    b_scale: Optional[Union[float, torch.Tensor]] = None,
    out: Optional[torch.Tensor] = None,
    *,
    epilogue: Optional[str] = None,
    out_dtype: Optional[torch.dtype] = None,
    activation: str = "none",
    bias: Optional[torch.Tensor] = None,
    chunk_tiles: Optional[int] = None,
) -> torch.Tensor:
    """INT8 block-sparse SpMM C = A @ B (int_quant.py:543-612) on the gfx950 kernel.

    Reference behaviour kept: a float B is quantised per tensor (its scale
    stays on the device: no host sync); an int8 B without b_scale uses 1.0;
    ``out`` is fully overwritten; the default epilogue is the reference's
    row-mean scaling.

    Additions (keyword-only, defaults preserve the reference):
      b_scale   may be a tensor of N per-column scales;
      epilogue  "row_mean" (default for a scalar b_scale), "per_block" (true
                per-tile dequantisation; default for per-column b_scale) or
                "raw_i32" (int32 accumulators, the bit-exact check);
      out_dtype float32 (default), bfloat16, float16 (int32 for raw_i32);
      activation / bias  fused epilogue, as void_spmm_activation_kernel.
    """
    M, K = a.shape
    if b.dim() != 2 or b.shape[0] != K:
        raise ValueError(f"B must be [K={K}, N], got {tuple(b.shape)}")
    N = b.shape[1]
    if bias is not None and tuple(bias.shape) != (N,):
        raise ValueError(f"bias must be [{N}], got {tuple(bias.shape)}")
    _runtime.require_gpu(b, "B")
    if b.dtype != torch.int8:
        b, b_scale = _quantize_b_per_tensor(b)
    scalar_scale, scale_vec, per_column = _b_scale_args(b_scale, N, b.device)
    per_column = per_column and b_scale.numel() != 1 if isinstance(b_scale, torch.Tensor) else per_column
    if epilogue is None:
        epilogue = "per_block" if per_column else "row_mean"
    if epilogue not in _lib.EPILOGUES:
        raise ValueError(f"unknown epilogue {epilogue!r}")
    if out_dtype is None:
        out_dtype = out.dtype if out is not None else (torch.int32 if epilogue == "raw_i32" else torch.float32)
    if (epilogue == "raw_i32") != (out_dtype == torch.int32):
        raise ValueError("epilogue 'raw_i32' goes with an int32 output")
    if out is None:
        out = torch.empty(M, N, dtype=out_dtype, device=b.device)
    elif out.shape != (M, N) or out.dtype != out_dtype:
        raise ValueError(f"out must be [{M}, {N}] {out_dtype}, got {tuple(out.shape)} {out.dtype}")
    if a.n_blocks == 0:
        out.zero_()
        if bias is not None or activation != "none":
            from .fusion import apply_activation_torch
            out.copy_(apply_activation_torch(out.float() + (bias if bias is not None else 0), activation))
        return out
    _runtime.require_gpu(a.values, "A")
    if a.values.device != b.device:
        raise ValueError(f"A on {a.values.device}, B on {b.device}")
    from .fusion import get_activation_code
    dbsr = a.device_bsr()
    chunk = chunk_tiles or tuning.select_chunk("int8", a.n_blocks, N, dbsr.max_row)
    if bias is not None:
        bias = bias.to(device=b.device, dtype=torch.float32).contiguous()
    return _runtime.launch("int8", dbsr, b, b_scale=scalar_scale, b_scale_vec=scale_vec, out=out,
                           epilogue=_lib.EPILOGUES[epilogue], activation=get_activation_code(activation),
                           bias=bias, chunk=chunk)


def get_quantization_error(original: torch.Tensor, config: IntQuantConfig) -> dict:
    """Quantisation error statistics (int_quant.py:615-645)."""
    q, params = quantize_tensor(original, config)
    rec = dequantize_tensor(q, params)
    abs_err = (original - rec).abs()
    rel_err = abs_err / (original.abs() + 1e-8)
    return {
        "config": str(config),
        "mean_abs_error": abs_err.mean().item(),
        "max_abs_error": abs_err.max().item(),
        "mean_rel_error": rel_err.mean().item(),
        "max_rel_error": rel_err.max().item(),
        "snr_db": (10 * torch.log10(original.pow(2).mean() / abs_err.pow(2).mean())).item(),
        "compression_ratio": original.element_size() / (config.bits / 8),
    }


__all__ = [
    "IntFormat", "ScaleMode", "IntQuantConfig", "QuantizationParams", "Int8VOIDTensor",
    "compute_scale_minmax", "compute_scale_percentile", "quantize_tensor", "quantize_per_column",
    "dequantize_tensor", "quantize_void_tensor", "dequantize_void_tensor", "void_spmm_int8",
    "get_quantization_error",
]
