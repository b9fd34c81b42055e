"""Device KV cache in the layout the gfx950 kernels read (mirrors model.py:238-255, 557-568).

Per non-shared layer: ``key [B, Hkv, slot_stride / 32, D / KR, 2, 16, KR]`` (KR = min(D, 32)) and ``value_t
[B, Hkv, slot_stride / 8, D, 8]`` in the parameter dtype: the values in groups of 8 slots, each
group stored d-major, so the 8 slots of one value dim are contiguous (one 16-byte MFMA operand in
bf16) and one slot's D values lie in one 8 * D-element span (an append touches D / 8 cache lines).
``value_dmajor()`` gives the plain transposed ``[B, Hkv, D, slot_stride]`` view. The keys of each
32-slot chunk are stored in the order of the attention MFMA's A operand (block (chunk, dims/32, bb)
holds 16 lanes x 32 dims, lane col = slot 8 (col >> 2) + 4 bb + (col & 3) of the chunk), so one
operand load reads one contiguous KiB; ``key_slots()`` gives slot-major ``[B, Hkv, slot_stride, D]``.
Sliding layers
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


def key_shape(batch: int, heads: int, slots: int, head_dim: int) -> tuple:
    """Shape of the operand-ordered key layout: ``[B, H, slots / 32, D / KR, 2, 16, KR]``,
    KR = min(D, 32) dims per run (slots a multiple of 32)."""

    kr = min(head_dim, 32)
    return (batch, heads, slots // 32, head_dim // kr, 2, 16, kr)


def group_keys(k: torch.Tensor) -> torch.Tensor:
    """Slot-major keys ``[B, H, Sp, D]`` (Sp a multiple of 32) -> the kernels' operand-ordered
    layout (``key_shape``; contiguous copy). Slot 8 a + 4 bb + c of a chunk goes to half bb, lane
    4 a + c."""

    B, H, Sp, D = k.shape
    kr = min(D, 32)
    t = k.reshape(B, H, Sp // 32, 4, 2, 4, D // kr, kr).permute(0, 1, 2, 6, 4, 3, 5, 7)
    return t.reshape(key_shape(B, H, Sp, D)).contiguous()


def ungroup_keys(kt: torch.Tensor) -> torch.Tensor:
    """The operand-ordered key layout -> slot-major ``[B, H, Sp, D]`` (copy)."""

    B, H, C, NR = kt.shape[:4]
    kr = kt.shape[6]
    return kt.reshape(B, H, C, NR, 2, 4, 4, kr).permute(0, 1, 2, 5, 4, 6, 3, 7).reshape(B, H, C * 32, NR * kr)


def group_values(v: torch.Tensor) -> torch.Tensor:
    """Slot-major values ``[B, H, Sp, D]`` (Sp a multiple of 8) -> the kernels' grouped layout
    ``[B, H, Sp / 8, D, 8]`` (contiguous copy)."""

    B, H, Sp, D = v.shape
    return v.reshape(B, H, Sp // 8, 8, D).transpose(3, 4).contiguous()


def ungroup_values(vt: torch.Tensor) -> torch.Tensor:
    """The grouped layout ``[B, H, G, D, 8]`` -> slot-major ``[B, H, 8 G, D]`` (copy)."""

    B, H, G, D, _ = vt.shape
    return vt.transpose(3, 4).reshape(B, H, G * 8, D)


class LayerKVCache(NamedTuple):
    key: torch.Tensor  # [B, Hkv, slot_stride / 32, D / KR, 2, 16, KR], KR = min(D, 32)
    value_t: torch.Tensor  # [B, Hkv, slot_stride / 8, D, 8]
    capacity: int  # logical slots: C (linear) or Wc (ring)
    ring: bool

    @property
    def slot_stride(self) -> int:
        return self.key.shape[2] * 32

    @property
    def head_dim(self) -> int:
        return self.key.shape[3] * self.key.shape[6]

    def key_slots(self) -> torch.Tensor:
        """The keys as slot-major ``[B, Hkv, slot_stride, D]`` (a copy)."""

        return ungroup_keys(self.key)

    def set_keys(self, k: torch.Tensor) -> None:
        """Write ``k [B, Hkv, capacity, D]`` (slot major) into slots ``[0, capacity)`` in place."""

        full = self.key_slots()
        full[:, :, : k.shape[2]] = k
        self.key.copy_(group_keys(full))

    def value_dmajor(self) -> torch.Tensor:
        """The values as ``[B, Hkv, D, slot_stride]`` (value dim major; a copy)."""

        B, H, G, D, _ = self.value_t.shape
        return self.value_t.permute(0, 1, 3, 2, 4).reshape(B, H, D, G * 8)

    def set_values(self, v: torch.Tensor) -> None:
        """Write ``v [B, Hkv, capacity, D]`` (slot major) into slots ``[0, capacity)`` in place."""

        B, H, C, D = v.shape
        full = self.value_t.permute(0, 1, 2, 4, 3).reshape(B, H, -1, D)  # [B, H, slot_stride, D] copy
        full[:, :, :C] = v
        self.value_t.copy_(full.reshape(B, H, -1, 8, D).permute(0, 1, 2, 4, 3))

    def reference_layout(self) -> tuple[torch.Tensor, torch.Tensor]:
        """``(key, value)`` as the reference's ``[B, capacity, Hkv, D]`` arrays (copies)."""

        k = self.key_slots()[:, :, : self.capacity].permute(0, 2, 1, 3).contiguous()
        v = self.value_dmajor()[:, :, :, : self.capacity].permute(0, 3, 1, 2).contiguous()
        return k, v


class KVCache(NamedTuple):
    layers: tuple  # LayerKVCache | None per layer
    key_mask: torch.Tensor  # [B, C] bool
    length: int


def new_layer_cache(batch: int, kv_heads: int, head_dim: int, capacity: int, ring: bool, dtype, device) -> LayerKVCache:
    ss = slot_stride_for(capacity)
    key = torch.zeros(key_shape(batch, kv_heads, ss, head_dim), dtype=dtype, device=device)
    value_t = torch.zeros((batch, kv_heads, ss // 8, head_dim, 8), dtype=dtype, device=device)
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


__all__ = ["LayerKVCache", "KVCache", "init_kv_cache", "new_layer_cache", "slot_stride_for", "key_shape", "group_keys",
           "ungroup_keys", "group_values", "ungroup_values", "FULL", "SLIDING"]
