"""Device KV cache in the layout the gfx950 kernels read (mirrors model.py:238-255, 557-568).

Per non-shared layer: ``key [B, Hkv, slot_stride, D]`` (head-major rows) and ``value_t
[B, Hkv, D, slot_stride]`` (values transposed, d-major) in the parameter dtype. Sliding layers
keep a ring of ``Wc = min(window, C)`` slots, global layers ``C = prompt + new`` slots, kv-shared
layers ``None`` (model.py:557-568). ``slot_stride`` rounds the slot count up to 64 so every row
is 128-byte aligned. ``key_mask [B, C]`` (bool, 1 byte per entry) records which absolute
positions hold real tokens; ``length`` is the number of positions written so far (the
reference's scalar ``KVCache.length``).
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from .config import FULL, SLIDING, Gemma4TextConfig, is_kv_shared, layer_head_dim, layer_kv_heads


def slot_stride_for(capacity: int) -> int:
    return (capacity + 63) // 64 * 64


class LayerKVCache(NamedTuple):
    key: torch.Tensor  # [B, Hkv, slot_stride, D]
    value_t: torch.Tensor  # [B, Hkv, D, slot_stride]
    capacity: int  # logical slots: C (linear) or Wc (ring)
    ring: bool

    @property
    def slot_stride(self) -> int:
        return self.key.shape[2]

    def reference_layout(self) -> tuple[torch.Tensor, torch.Tensor]:
        """``(key, value)`` as the reference's ``[B, capacity, Hkv, D]`` arrays (copies)."""

        k = self.key[:, :, : self.capacity].permute(0, 2, 1, 3).contiguous()
        v = self.value_t[:, :, :, : self.capacity].permute(0, 3, 1, 2).contiguous()
        return k, v


class KVCache(NamedTuple):
    layers: tuple  # LayerKVCache | None per layer
    key_mask: torch.Tensor  # [B, C] bool
    length: int


def new_layer_cache(batch: int, kv_heads: int, head_dim: int, capacity: int, ring: bool, dtype, device) -> LayerKVCache:
    ss = slot_stride_for(capacity)
    key = torch.zeros((batch, kv_heads, ss, head_dim), dtype=dtype, device=device)
    value_t = torch.zeros((batch, kv_heads, head_dim, ss), dtype=dtype, device=device)
    return LayerKVCache(key, value_t, capacity, ring)


def init_kv_cache(config: Gemma4TextConfig, batch_size: int, capacity: int, dtype, device="cuda") -> KVCache:
    """model.py:557-568: bounded rings on sliding layers, full capacity on global layers,
    ``None`` on kv-shared layers; zero-filled."""

    layers = []
    for i in range(config.num_hidden_layers):
        if is_kv_shared(config, i):
            layers.append(None)
            continue
        ring = config.layer_types[i] == SLIDING
        cap = min(config.sliding_window, capacity) if ring else capacity
        layers.append(new_layer_cache(batch_size, layer_kv_heads(config, i), layer_head_dim(config, i), cap, ring,
                                      dtype, device))
    key_mask = torch.zeros((batch_size, capacity), dtype=torch.bool, device=device)
    return KVCache(tuple(layers), key_mask, 0)


__all__ = ["LayerKVCache", "KVCache", "init_kv_cache", "new_layer_cache", "slot_stride_for", "FULL", "SLIDING"]
