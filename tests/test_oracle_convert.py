"""The f32 -> bf16 rollout cast (inference_device.py:21-25 restated as oracle.bf16_bits), pinned
on the reference's own vectors (tests/test_inference_device.py:16-26): every finite bf16 encoding
with the low halves 0, 0x7FFF, 0x8000, 0x8001, 0xFFFF on each side of the rounding boundaries,
against torch's own round-to-nearest-even cast on the CPU (an independent implementation)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import g4_oracle as O


def boundary_vectors() -> np.ndarray:
    high = np.arange(65536, dtype=np.uint32)
    high = high[(high & 0x7F80) != 0x7F80]
    bits = ((high[:, None] << 16) | np.array([0, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32)).ravel()
    return bits.view(np.float32)


def test_bitwise_rne_matches_torch_on_every_encoding_and_boundary():
    value = boundary_vectors()
    got = O.bf16_bits(value)
    want = torch.from_numpy(value).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)
    # values just below the largest finite bf16's rounding boundary overflow to inf
    expected = O.from_bf16_bits(got)
    assert not np.isfinite(expected).all() and np.isfinite(value).all()


def test_signed_zero_and_subnormals_are_kept():
    value = np.array([0.0, -0.0, 1e-40, -1e-40, 9.2e-41], np.float32)
    got = O.bf16_bits(value)
    assert got[0] == 0 and got[1] == 0x8000
    assert (got[2:] & 0x7F80 == 0).all() and (got[2:] & 0x7F != 0).all()  # bf16 subnormals, not flushed
