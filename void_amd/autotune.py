"""The reference's autotuning API (void/autotune.py:15-104, 268-381,
414-492) over the fixed gfx950 launch configuration of ``tuning``.

The reference benchmarks TILE_N x num_warps x num_stages per problem shape
and keeps the winner in a JSON cache.  On MI355X the kernel shape is fixed
(one 32-row block-row x 128-column panel per workgroup of four wave64s, a
two-stage LDS-DMA ring), so there is nothing to search: the calls below
keep their names, arguments and return types for callers of the reference,
and report that one configuration.  Nothing is benchmarked and nothing is
written to disk.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass
from typing import Dict, List, Optional

import torch

from . import tuning


@dataclass
class KernelConfig:
    """Launch configuration (autotune.py:15-36): tile sizes, waves (the
    reference's warps) and pipeline stages."""
    TILE_M: int
    TILE_K: int
    TILE_N: int
    num_warps: int
    num_stages: int = 3

    def __hash__(self):
        return hash((self.TILE_M, self.TILE_K, self.TILE_N, self.num_warps, self.num_stages))

    def to_dict(self):
        return asdict(self)

    @classmethod
    def from_dict(cls, d):
        return cls(**d)


def gfx950_config(tile_m: int = tuning.TILE, tile_k: int = tuning.TILE) -> KernelConfig:
    """The one configuration the gfx950 kernels run."""
    return KernelConfig(TILE_M=tile_m, TILE_K=tile_k, TILE_N=tuning.PANEL_COLUMNS,
                        num_warps=tuning.WAVES_PER_WORKGROUP, num_stages=2)


class AutotuneCache:
    """In-memory stand-in for the reference's per-GPU JSON cache
    (autotune.py:39-103): same keys and get / set, never persisted."""

    def __init__(self, cache_dir: Optional[str] = None):
        self.cache_dir = cache_dir
        self.cache: Dict[str, KernelConfig] = {}

    def make_key(self, op: str, M: int, K: int, N: int, tile_m: int, tile_k: int) -> str:
        """Shape rounded down to powers of two, as the reference keys its cache."""
        p2 = lambda x: 1 << max(0, int(x).bit_length() - 1)
        return f"{op}_M{p2(M)}_K{p2(K)}_N{p2(N)}_TM{tile_m}_TK{tile_k}"

    def get(self, key: str) -> Optional[KernelConfig]:
        return self.cache.get(key)

    def set(self, key: str, config: KernelConfig) -> None:
        self.cache[key] = config


_autotune_cache = AutotuneCache()


def generate_spmm_configs(N: int, tile_m: int, tile_k: int) -> List[KernelConfig]:
    """Candidate configurations (autotune.py:345-381): on gfx950 only the
    fixed one."""
    return [gfx950_config(tile_m, tile_k)]


def autotune_spmm(void_tensor, b: torch.Tensor, use_cache: bool = True) -> KernelConfig:
    """The configuration the SpMM of this problem runs (autotune.py:268-342),
    recorded in the cache under the reference's key."""
    M, K = void_tensor.shape
    tm, tk = void_tensor.tile_size
    key = _autotune_cache.make_key("spmm", M, K, b.shape[1], tm, tk)
    cfg = _autotune_cache.get(key) if use_cache else None
    if cfg is None:
        cfg = gfx950_config(tm, tk)
        if use_cache:
            _autotune_cache.set(key, cfg)
    return cfg


def void_spmm_with_autotune(a, b: torch.Tensor, out: Optional[torch.Tensor] = None,
                            config: Optional[KernelConfig] = None) -> torch.Tensor:
    """void_spmm with a configuration argument (autotune.py:414-483).  The
    configuration is accepted and ignored: the gfx950 kernels have one."""
    if config is not None and not isinstance(config, KernelConfig):
        raise TypeError("config must be a KernelConfig")
    from .ops import void_spmm
    return void_spmm(a, b, out=out)


def clear_autotune_cache() -> None:
    """Empty the configuration cache (autotune.py:486-492)."""
    global _autotune_cache
    _autotune_cache = AutotuneCache()


__all__ = ["KernelConfig", "AutotuneCache", "generate_spmm_configs", "autotune_spmm", "void_spmm_with_autotune",
           "clear_autotune_cache", "gfx950_config"]
