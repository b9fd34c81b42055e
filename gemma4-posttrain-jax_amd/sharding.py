"""The rollout weight handoff of gemma4_posttrain_jax/sharding.py and inference_device.py on one GPU.

``reshard_for_rollout`` (sharding.py:213-228) casts the f32 master parameters to the rollout dtype
and ``reshard_after_rollout`` (sharding.py:231-241) casts a rollout tree back; the master is never
modified. The bf16 narrowing is the native ``g4_convert_f32_to_bf16``: the bitwise
round-to-nearest-even of inference_device.py:21-25, the same bits as XLA's f32 -> bf16 convert on
finite values. ``device_converter`` (inference_device.py:10-45) returns the converted array and the
same finiteness verdict, for the "identity" and "reshape" layouts (the others are vLLM weight
layouts, out of scope). The mesh collapses to one device: ``mesh`` must be None, and the
"replicated" and "fsdp" rollout layouts both mean the whole array on this GPU.
"""

from __future__ import annotations

from typing import Any

import torch

from . import kernels
from .config import Gemma4TextConfig
from .model import Gemma4TextParams

ROLLOUT_LAYOUTS = ("replicated", "fsdp")


def _no_mesh(mesh) -> None:
    if mesh is not None:
        raise ValueError("mesh sharding is not supported: the native rollout path runs on one GPU")


def tree_map(fn, tree: Any) -> Any:
    """Apply ``fn`` to every tensor leaf of a parameter pytree (NamedTuples, tuples, lists, None)."""

    if tree is None:
        return None
    if isinstance(tree, torch.Tensor):
        return fn(tree)
    if isinstance(tree, tuple) and hasattr(tree, "_fields"):
        return type(tree)(*(tree_map(fn, x) for x in tree))
    if isinstance(tree, (tuple, list)):
        return type(tree)(tree_map(fn, x) for x in tree)
    raise TypeError(f"unexpected parameter leaf {type(tree).__name__}")


def tree_leaves(tree: Any) -> list[torch.Tensor]:
    out: list[torch.Tensor] = []
    tree_map(lambda t: out.append(t) or t, tree)
    return out


def constrain_batch(x: torch.Tensor, mesh=None) -> torch.Tensor:
    """sharding.py:186-189: the batch-axis sharding constraint. On one GPU the whole batch is
    already on the device, so this is the identity (``mesh`` must be None)."""

    _no_mesh(mesh)
    return x


def constrain_batch_tree(tree: Any, mesh=None) -> Any:
    """sharding.py:192-199: ``constrain_batch`` over every leaf of a pytree; the identity on one
    GPU (``mesh`` must be None). The tree is returned as is, leaves of any type included."""

    _no_mesh(mesh)
    return tree


def _cast(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    if t.dtype == dtype:
        return t.clone()  # a new tree, as the reference's astype inside jit returns new buffers
    if t.dtype == torch.float32 and dtype == torch.bfloat16:
        return kernels.convert_f32_to_bf16(t)
    if t.dtype == torch.bfloat16 and dtype == torch.float32:
        return kernels.convert_bf16_to_f32(t)
    raise TypeError(f"no rollout cast from {t.dtype} to {dtype}")


def reshard_for_rollout(params_f32: Gemma4TextParams, config: Gemma4TextConfig, mesh=None, *,
                        dtype: torch.dtype = torch.bfloat16, layout: str = "replicated") -> Gemma4TextParams:
    """sharding.py:213-228: the rollout copy of the parameters in ``dtype`` (the master is untouched)."""

    _no_mesh(mesh)
    if layout not in ROLLOUT_LAYOUTS:
        raise ValueError(f"unknown rollout layout {layout!r}; expected one of {ROLLOUT_LAYOUTS}")
    return tree_map(lambda t: _cast(t, dtype), params_f32)


def reshard_after_rollout(rollout_params: Gemma4TextParams, config: Gemma4TextConfig, mesh=None, *,
                          dtype: torch.dtype = torch.float32) -> Gemma4TextParams:
    """sharding.py:231-241: cast a rollout tree back (to f32 by default; exact from bf16)."""

    _no_mesh(mesh)
    return tree_map(lambda t: _cast(t, dtype), rollout_params)


def device_converter(layout: str, shape: tuple[int, ...], shards: int = 1):
    """inference_device.py:10-45 for the "identity" / "reshape" layouts: returns
    ``convert(value) -> (bf16 array of `shape`, finite: bool tensor)``, finite meaning no input
    was inf / NaN and no value overflowed in the cast."""

    if layout not in ("identity", "reshape"):
        raise ValueError(f"layout {layout!r} is not supported on this path (vLLM weight layouts are out of scope)")
    if shards != 1:
        raise ValueError("one GPU: shards must be 1")

    def convert(value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        flag = torch.zeros(1, dtype=torch.int32, device=value.device)
        out = kernels.convert_f32_to_bf16(value, nonfinite=flag)
        return out.reshape(shape), flag[0] == 0

    return convert
