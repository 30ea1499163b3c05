"""void_amd — MI355X (gfx950) quantised block-sparse SpMM with the VOID API.

Drop-in for the quantised SpMM path of the reference package ``void``:
csr_to_void / dense_to_void (tile format), quantize_void_tensor /
void_spmm_int8 (INT8), void_tensor_to_fp8 / void_spmm_fp8 (FP8 E4M3),
void_spmm_gelu (fused activation) and the Stream-K workload helpers.  The
SpMM itself runs only in the hand-written HIP kernels of libvoid_amd.so.
"""

from .format import (
    MIN_TENSOR_CORE_TILE,
    VOIDTensor,
    csr_to_void,
    dense_to_void,
    morton_decode,
    morton_encode,
    morton_encode_batch,
    void_to_csr,
)
from .int_quant import (
    Int8VOIDTensor,
    IntFormat,
    IntQuantConfig,
    QuantizationParams,
    ScaleMode,
    compute_scale_minmax,
    dequantize_tensor,
    dequantize_void_tensor,
    get_quantization_error,
    quantize_per_column,
    quantize_tensor,
    quantize_void_tensor,
    void_spmm_int8,
)
from .fp8 import (
    FP8Config,
    FP8Format,
    FP8ScalingInfo,
    FP8VOIDTensor,
    compute_amax,
    create_scaling_info,
    dequantize_from_fp8,
    quantize_to_fp8,
    void_spmm_fp8,
    void_tensor_to_fp8,
)
from .fusion import (ActivationType, FusedSparseLinear, get_activation_code, void_spmm_gelu, void_spmm_relu,
                     void_spmm_silu)
from .packed import load_packed, pack, save_packed, unpack
from .ops import MIN_TENSOR_CORE_K, compute_optimal_tile_n, void_spmm
from .autograd import SparseLinear, VOIDSpMM, VOIDSpMMFunction
from .stream_k import StreamKWorkload, analyze_workload_balance, compute_stream_k_workload, void_spmm_stream_k

__version__ = "0.1.0"

__all__ = [
    "MIN_TENSOR_CORE_TILE", "VOIDTensor", "csr_to_void", "dense_to_void", "void_to_csr",
    "morton_encode", "morton_decode", "morton_encode_batch",
    "IntFormat", "ScaleMode", "IntQuantConfig", "QuantizationParams", "Int8VOIDTensor",
    "compute_scale_minmax", "quantize_tensor", "quantize_per_column", "dequantize_tensor",
    "quantize_void_tensor", "dequantize_void_tensor", "void_spmm_int8", "get_quantization_error",
    "FP8Format", "FP8Config", "FP8ScalingInfo", "FP8VOIDTensor", "create_scaling_info", "compute_amax",
    "quantize_to_fp8", "dequantize_from_fp8", "void_spmm_fp8", "void_tensor_to_fp8",
    "ActivationType", "get_activation_code", "void_spmm_gelu", "void_spmm_relu", "void_spmm_silu",
    "StreamKWorkload", "compute_stream_k_workload", "analyze_workload_balance", "void_spmm_stream_k",
    "void_spmm", "compute_optimal_tile_n", "MIN_TENSOR_CORE_K", "FusedSparseLinear", "SparseLinear", "VOIDSpMM",
    "VOIDSpMMFunction", "pack", "unpack", "save_packed", "load_packed",
]
