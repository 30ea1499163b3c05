"""Packed BSR blob: one contiguous little-endian buffer holding a VOID
tensor in the device layout (header, row_ptr, col_idx, scales, tiles in
block-row-major order), so that pruned weights load with one read and one
host-to-device copy, without the argsort of get_row_block_info
(void/format.py:201-237).  The consumer in the reference is
FusedSparseLinear (void/fusion.py:756-836), whose buffers are the VOID
tensor fields.

Layout (offsets in bytes; sections 256-byte aligned):

    0   magic  b"VOIDBSR\\0"
    8   u32    version (1)
    12  u32    kind: 0 float32 tiles, 1 int8 tiles, 2 float8_e4m3fn tiles,
               3 bfloat16 tiles, 4 float16 tiles
    16  i64    M          24 i64 K
    32  i64    n_blocks   40 i64 n_block_rows
    48  u32    tile (32)  52 u32 flags (bit 0: one per-tensor scale)
    56  u64    offset of row_ptr  (int32 [n_block_rows + 1])
    64  u64    offset of col_idx  (int32 [n_blocks])
    72  u64    offset of scales   (float32 [n_blocks], [1] per-tensor, [0] float)
    80  u64    offset of tiles    (n_blocks x 32 x 32 elements)
    88  u64    total size
    96  i64    nnz_original       104..255 zero
"""

from __future__ import annotations

import struct
from pathlib import Path
from typing import Union

import numpy as np
import torch

from . import _runtime
from .format import VOIDTensor, build_bsr_layout, morton_encode_batch

MAGIC = b"VOIDBSR\0"
VERSION = 1
KIND_F32, KIND_I8, KIND_FP8, KIND_BF16, KIND_F16 = 0, 1, 2, 3, 4
_FLOAT_KINDS = {KIND_F32: torch.float32, KIND_BF16: torch.bfloat16, KIND_F16: torch.float16}
_ELT_BYTES = {KIND_F32: 4, KIND_I8: 1, KIND_FP8: 1, KIND_BF16: 2, KIND_F16: 2}
_HEADER = struct.Struct("<8sIIqqqqIIQQQQQq")
_ALIGN = 256


def _align(x: int) -> int:
    return (x + _ALIGN - 1) // _ALIGN * _ALIGN


def _parts(t):
    """(kind, tiles[n,32,32] in Morton order, scales, per_tensor) of a VOID tensor."""
    from .fp8 import FP8VOIDTensor
    from .int_quant import Int8VOIDTensor, ScaleMode
    if isinstance(t, Int8VOIDTensor):
        if t.values.dtype != torch.int8 or not t.config.symmetric:
            raise NotImplementedError("packed blobs hold symmetric int8 tiles")
        per_tensor = t.config.scale_mode == ScaleMode.PER_TENSOR
        return KIND_I8, t.values, t.scales, per_tensor
    if isinstance(t, FP8VOIDTensor):
        if t.values_fp8.dtype != torch.float8_e4m3fn or t.scaling_info.config.scale_mode != "per_block":
            raise NotImplementedError("packed blobs hold per-block E4M3 tiles")
        return KIND_FP8, t.values_fp8.view(torch.uint8), t.scaling_info.scale, False
    if isinstance(t, VOIDTensor):
        # 16-bit tiles keep their dtype (and feed the 16-bit kernel when
        # loaded); other float dtypes are stored as fp32.
        if t.values.dtype == torch.bfloat16:
            return KIND_BF16, t.values.view(torch.int16), None, False
        if t.values.dtype == torch.float16:
            return KIND_F16, t.values.view(torch.int16), None, False
        return KIND_F32, t.values.to(torch.float32), None, False
    raise TypeError(f"cannot pack {type(t).__name__}")


def pack(t) -> bytes:
    """The blob of a VOIDTensor, Int8VOIDTensor or FP8VOIDTensor (32x32 tiles)."""
    if tuple(t.tile_size) != (32, 32):
        raise NotImplementedError("packed blobs hold 32x32 tiles")
    kind, tiles, scales, per_tensor = _parts(t)
    M, K = t.shape
    n_br, n_bc = (M + 31) // 32, (K + 31) // 32
    lay = build_bsr_layout(t.block_rows, t.block_cols, n_br, n_bc, torch.device("cpu"))
    order = lay.order.numpy()
    tiles_np = tiles.detach().cpu().contiguous().numpy()[order] if t.n_blocks else tiles.detach().cpu().numpy()
    if kind in _FLOAT_KINDS:
        sc = np.zeros(0, np.float32)
    else:
        s = scales.detach().cpu().to(torch.float32).numpy().reshape(-1)
        sc = s[:1].copy() if per_tensor else s[order].copy()
    sections = [lay.row_ptr_host.astype("<i4"), lay.col_idx.numpy().astype("<i4"), sc.astype("<f4"),
                np.ascontiguousarray(tiles_np)]
    offs, pos = [], _ALIGN
    for a in sections:
        offs.append(pos)
        pos = _align(pos + a.nbytes)
    buf = bytearray(pos)
    nnz = int(getattr(t, "nnz_original", 0))
    _HEADER.pack_into(buf, 0, MAGIC, VERSION, kind, M, K, t.n_blocks, n_br, 32, int(per_tensor), *offs, pos, nnz)
    for o, a in zip(offs, sections):
        buf[o:o + a.nbytes] = a.tobytes()
    return bytes(buf)


def save_packed(t, path: Union[str, Path]) -> None:
    Path(path).write_bytes(pack(t))


def unpack(blob: Union[bytes, bytearray, memoryview], device: Union[str, torch.device] = "cpu"):
    """A VOID tensor from a blob.  On a GPU the blob crosses PCIe once and the
    tensor's block-row-major device copy (the kernels' operand) is set up from
    it directly; the Morton-ordered fields are derived on the device."""
    mv = memoryview(blob)
    if len(mv) < _HEADER.size:
        raise ValueError("blob too short")
    (magic, version, kind, M, K, nb, n_br, tile, flags, o_rp, o_ci, o_sc, o_ti, total, nnz) = \
        _HEADER.unpack_from(mv, 0)
    if magic != MAGIC or version != VERSION:
        raise ValueError("not a VOID packed BSR blob (version 1)")
    if tile != 32 or n_br != (M + 31) // 32 or total > len(mv) or kind not in _ELT_BYTES:
        raise ValueError("corrupt VOID packed BSR blob header")
    per_tensor = bool(flags & 1)
    elt = _ELT_BYTES[kind]
    n_sc = 0 if kind in _FLOAT_KINDS else (1 if per_tensor else nb)
    for o, n in ((o_rp, 4 * (n_br + 1)), (o_ci, 4 * nb), (o_sc, 4 * n_sc), (o_ti, elt * 1024 * nb)):
        if o % _ALIGN or o + n > total:
            raise ValueError("corrupt VOID packed BSR blob sections")
    dev = torch.device(device)
    raw = torch.frombuffer(bytearray(mv[:total]), dtype=torch.uint8)
    if dev.type == "cuda":
        raw = raw.to(dev)  # the one host-to-device copy
    row_ptr = raw[o_rp:o_rp + 4 * (n_br + 1)].view(torch.int32)
    col_idx = raw[o_ci:o_ci + 4 * nb].view(torch.int32)
    scales = raw[o_sc:o_sc + 4 * n_sc].view(torch.float32)
    tiles_bytes = raw[o_ti:o_ti + elt * 1024 * nb]
    rp_host = np.frombuffer(mv[o_rp:o_rp + 4 * (n_br + 1)], dtype="<i4").astype(np.int32)
    ci_host = np.frombuffer(mv[o_ci:o_ci + 4 * nb], dtype="<i4").astype(np.int32)
    if np.any(np.diff(rp_host) < 0) or rp_host[0] != 0 or rp_host[-1] != nb or \
            (nb and (ci_host.min() < 0 or ci_host.max() >= (K + 31) // 32)):
        raise ValueError("corrupt VOID packed BSR blob index arrays")
    # Morton order of the tiles (the VOID tensor's own order)
    br_host = np.repeat(np.arange(n_br, dtype=np.int64), np.diff(rp_host))
    morton = morton_encode_batch(br_host, ci_host.astype(np.int64)).astype(np.int64)
    perm = np.argsort(morton, kind="stable")
    perm_t = torch.from_numpy(perm).to(dev)
    block_rows = torch.from_numpy(br_host.astype(np.int32)).to(dev).index_select(0, perm_t)
    block_cols = col_idx.index_select(0, perm_t)
    morton_t = torch.from_numpy(morton).to(dev).index_select(0, perm_t)
    n_br_c = (M + 31) // 32
    density = nb / (n_br_c * ((K + 31) // 32)) if M and K else 0.0
    # BSR position p holds the tensor's tile order[p] (perm's inverse), for
    # gathering again after in-place changes of the tensor's values.
    order = torch.empty_like(perm_t)
    order[perm_t] = torch.arange(nb, dtype=perm_t.dtype, device=dev)
    dbsr = _runtime.DeviceBsr(tiles=tiles_bytes.view(nb, 32, 32 * elt), scales=scales if n_sc else
                              torch.ones(1, dtype=torch.float32, device=dev), row_ptr=row_ptr, col_idx=col_idx,
                              row_ptr_host=rp_host, col_idx_host=ci_host, per_tensor=per_tensor or n_sc == 0,
                              M=M, K=K, n_blocks=nb, n_block_rows=n_br, order=order)
    key = str(dev)
    if kind in _FLOAT_KINDS:
        dt = _FLOAT_KINDS[kind]
        vals = tiles_bytes.view(dt).view(nb, 32, 32).index_select(0, perm_t)
        vt = VOIDTensor(values=vals, block_rows=block_rows, block_cols=block_cols, morton_codes=morton_t,
                        shape=(M, K), tile_size=(32, 32), nnz_original=nnz, n_blocks=nb, density=density, dtype=dt)
        dbsr.src_key = _runtime.source_key(vals)
        # The device copy under the key the float SpMM looks up for this dtype.
        vt._device_bsr[key if dt == torch.float32 else f"{dev}/{dt}"] = dbsr
        return vt
    if kind == KIND_I8:
        from .int_quant import Int8VOIDTensor, IntQuantConfig, ScaleMode
        vals = tiles_bytes.view(torch.int8).view(nb, 32, 32).index_select(0, perm_t)
        cfg = IntQuantConfig(scale_mode=ScaleMode.PER_TENSOR if per_tensor else ScaleMode.PER_BLOCK)
        sc = scales.expand(nb) if per_tensor else scales.index_select(0, perm_t)
        q = Int8VOIDTensor(values=vals, scales=sc, zero_points=torch.zeros(nb, dtype=torch.int8, device=dev),
                           block_rows=block_rows, block_cols=block_cols, shape=(M, K), tile_size=(32, 32),
                           n_blocks=nb, config=cfg)
        dbsr.src_key = _runtime.source_key(vals, sc)
        q._device_bsr[key] = dbsr
        return q
    from .fp8 import FP8Config, FP8VOIDTensor, create_scaling_info
    cfg = FP8Config(scale_mode="per_block")
    vals = tiles_bytes.view(torch.float8_e4m3fn).view(nb, 32, 32).index_select(0, perm_t)
    sc = scales.index_select(0, perm_t)
    info = create_scaling_info((nb, 32, 32), cfg, dev)
    info.update_amax(sc * 448.0)
    info.scale, info.scale_inv = sc, 1.0 / sc
    f8 = FP8VOIDTensor(values_fp8=vals, scaling_info=info, block_rows=block_rows, block_cols=block_cols,
                       morton_codes=morton_t, shape=(M, K), tile_size=(32, 32), nnz_original=nnz, n_blocks=nb,
                       density=density)
    dbsr.src_key = _runtime.source_key(vals, info.scale)
    f8._device_bsr[key] = dbsr
    return f8


def load_packed(path: Union[str, Path], device: Union[str, torch.device] = "cpu"):
    return unpack(Path(path).read_bytes(), device)


__all__ = ["pack", "unpack", "save_packed", "load_packed", "MAGIC", "VERSION"]
