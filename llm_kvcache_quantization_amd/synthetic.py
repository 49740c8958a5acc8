"""Seeded synthetic workloads of the five benchmark configurations.

Distributions (per configuration ``cfg`` and layer ``l``, seed 1234 + 1000 cfg + l):

* K ~ N(0, 1), with 4 fixed outlier channels per KV head scaled x20.  The indices come
  from ``randperm(128)[:4]`` per head and are shared by calibration and cache.
* V ~ N(0, 1); q ~ N(0, 1) [B, Hq, 128].
* inv_tau ~ U(0.8, 1.2) [L, Hq].

Static tables come from a separate 512-token calibration sample with the same
distribution (:mod:`calib`).  Small instances are drawn with a CPU generator, so tests
and fixtures are reproducible.  Full-size caches are drawn on the GPU by ``bench.py``.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import torch

BASE_SEED = 1234
HEAD_DIM = 128
OUTLIER_SCALE = 20.0
N_OUTLIER = 4
CALIB_TOKENS = 512


@dataclass(frozen=True)
class Config:
    index: int
    name: str
    q_heads: int
    kv_heads: int
    layers: int
    batch: int
    context: int  # uniform context, or the upper bound of a ragged draw
    k_format: str  # "int8" | "int4_asym"
    v_format: str
    ragged_min: Optional[int] = None
    outlier_channels: bool = False
    group_size: int = 32

    @property
    def n_rep(self) -> int:
        return self.q_heads // self.kv_heads


CONFIGS: List[Config] = [
    Config(0, "qwen2.5-1.5b/int8-g32/b1/ctx4096/1L", 12, 2, 1, 1, 4096, "int8", "int8"),
    Config(1, "qwen2.5-1.5b/int8-g32/b4/ctx8192/28L", 12, 2, 28, 4, 8192, "int8", "int8"),
    Config(2, "qwen2.5-1.5b/int4-asym-g32+4fp16ch/b16/ctx32768/1L", 12, 2, 1, 16, 32768,
           "int4_asym", "int4_asym", outlier_channels=True),
    Config(3, "qwen2.5-7b/int4-asym-g32+4fp16ch/b8/ctx32768/28L", 28, 4, 28, 8, 32768,
           "int4_asym", "int4_asym", outlier_channels=True),
    Config(4, "qwen2.5-14b/k-int8-g32+v-int4-asym-g32/b8/ragged4096-65536/48L", 40, 8, 48, 8,
           65536, "int8", "int4_asym", ragged_min=4096),
]


def seed_for(cfg: int, layer: int) -> int:
    return BASE_SEED + 1000 * cfg + layer


def outlier_channels(cfg: Config, layer: int) -> torch.Tensor:
    """int64 [Hkv, 4]: the channels of K scaled x20 (randperm(128)[:4] per head)."""
    g = torch.Generator().manual_seed(seed_for(cfg.index, layer) + 7)
    return torch.stack([torch.randperm(HEAD_DIM, generator=g)[:N_OUTLIER] for _ in range(cfg.kv_heads)])


def context_lengths(cfg: Config) -> torch.Tensor:
    """int32 [B]: uniform, or seeded-uniform in [ragged_min, context] for ragged configs."""
    if cfg.ragged_min is None:
        return torch.full((cfg.batch,), cfg.context, dtype=torch.int32)
    g = torch.Generator().manual_seed(seed_for(cfg.index, 0) + 99)
    return torch.randint(cfg.ragged_min, cfg.context + 1, (cfg.batch,), generator=g, dtype=torch.int32)


def inv_tau(cfg: Config) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed_for(cfg.index, 0) + 11)
    return (0.8 + 0.4 * torch.rand(cfg.layers, cfg.q_heads, generator=g)).to(torch.float16)


def draw_kv(cfg: Config, layer: int, batch: int, tokens: int, generator: torch.Generator,
            device="cpu", ch: Optional[torch.Tensor] = None):
    """K, V fp16 [batch, Hkv, tokens, 128] with the x20 outlier channels on K."""
    k = torch.randn(batch, cfg.kv_heads, tokens, HEAD_DIM, generator=generator, device=device)
    v = torch.randn(batch, cfg.kv_heads, tokens, HEAD_DIM, generator=generator, device=device)
    ch = outlier_channels(cfg, layer) if ch is None else ch
    for h in range(cfg.kv_heads):
        k[:, h, :, ch[h].to(device)] *= OUTLIER_SCALE
    return k.to(torch.float16), v.to(torch.float16)


def draw_q(cfg: Config, batch: int, generator: torch.Generator, device="cpu") -> torch.Tensor:
    return torch.randn(batch, cfg.q_heads, HEAD_DIM, generator=generator, device=device).to(torch.float16)


@dataclass
class LayerTables:
    """Static tables of one layer for its configuration's formats."""

    k_scale: Optional[torch.Tensor] = None  # int8: fp16 [Hkv, G]; asym: fp16 [Hkv, 4]
    v_scale: Optional[torch.Tensor] = None
    k_zp: Optional[torch.Tensor] = None
    v_zp: Optional[torch.Tensor] = None
    k_outlier_idx: Optional[torch.Tensor] = None  # int32 [Hkv, 4]


def calibrate(cfg: Config, layer: int) -> LayerTables:
    """Static tables from the seeded 512-token calibration sample of (cfg, layer)."""
    from . import calib

    g = torch.Generator().manual_seed(seed_for(cfg.index, layer) + 500_000)
    k, v = draw_kv(cfg, layer, 1, CALIB_TOKENS, g)
    t = LayerTables()
    if cfg.k_format == "int8":
        t.k_scale = calib.int8_static_scale(k, cfg.group_size)
    else:
        if cfg.outlier_channels:
            t.k_outlier_idx = calib.select_outlier_channels(k, N_OUTLIER)
        t.k_scale, t.k_zp = calib.asym_g32_params(k, t.k_outlier_idx)
    if cfg.v_format == "int8":
        t.v_scale = calib.int8_static_scale(v, cfg.group_size)
    else:
        t.v_scale, t.v_zp = calib.asym_g32_params(v)
    return t
