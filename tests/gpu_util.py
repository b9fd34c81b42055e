"""Conversions between device tensors (kernel layouts) and the oracle's numpy arrays."""

from __future__ import annotations

import numpy as np
import torch

from oracle import g4_oracle as O

TORCH_DTYPE = {O.F32: torch.float32, O.BF16: torch.bfloat16}
TOL = {O.F32: 1e-5, O.BF16: 2e-2}  # max-abs parity bars for attention outputs / logits


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def to_dev(a: np.ndarray, dtype: str, device) -> torch.Tensor:
    """numpy float32 (already representable in ``dtype``) -> device tensor, exactly."""

    t = torch.from_numpy(np.ascontiguousarray(a, np.float32))
    return t.to(TORCH_DTYPE[dtype]).to(device)


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw storage bits (uint16 for bf16, uint32 for f32) for bit-exact comparisons."""

    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.view(torch.int32).numpy().view(np.uint32)


def np_bits(a: np.ndarray, dtype: str) -> np.ndarray:
    return O.bf16_bits(a) if dtype == O.BF16 else np.ascontiguousarray(a, np.float32).view(np.uint32)


def cache_to_ref(layer) -> tuple[np.ndarray, np.ndarray]:
    """Kernel layout (key [B,H,Cp,D], value_t [B,H,D,Cp]) -> the reference's [B,C,H,D] pair."""

    k, v = layer.reference_layout()
    return to_np(k), to_np(v)


def load_oracle_cache(cache, ref: "O.KVCache", dtype: str):
    """Copy an oracle KVCache (reference layout) into a device KVCache; returns the device cache
    with the oracle's key_mask and length, so one call can run on exactly the oracle's inputs."""

    for ours, theirs in zip(cache.layers, ref.layers):
        if ours is not None:
            ref_to_cache(ours, theirs.key, theirs.value, dtype)
    cache.key_mask.copy_(torch.from_numpy(ref.key_mask))
    return cache._replace(length=int(ref.length))


def model_bars(dtype: str, got: np.ndarray, ref: np.ndarray, ref_f64acc: np.ndarray) -> tuple[float, float]:
    """Model-level logits bar. fp32: the reference's cross-implementation tolerance (JAX vs HF,
    rel 1e-4 of max|x|, tests/test_model_ops.py:228). bf16: 2e-2 plus how far the oracle itself
    moves when its matmuls accumulate in f64 instead of f32 on the same inputs (the precision to
    which the reference's output is determined at all). Returns (error, bar)."""

    err = float(np.abs(got - ref).max())
    if dtype == O.F32:
        return err, 1e-4 * max(1.0, float(np.abs(ref).max()))
    return err, TOL[O.BF16] + float(np.abs(ref - ref_f64acc).max())


def ref_to_cache(layer, k_ref: np.ndarray, v_ref: np.ndarray, dtype: str) -> None:
    """Write reference-layout [B,C,H,D] contents into a kernel-layout cache layer in place."""

    dev = layer.key.device
    k = to_dev(k_ref, dtype, dev).permute(0, 2, 1, 3)
    v = to_dev(v_ref, dtype, dev).permute(0, 2, 3, 1)
    layer.key[:, :, : layer.capacity].copy_(k)
    layer.value_t[:, :, :, : layer.capacity].copy_(v)
