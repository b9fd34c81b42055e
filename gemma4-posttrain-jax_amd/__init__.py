"""MI355X-native Gemma 4 rollout prefill + KV-cache decode (drop-in for gemma4_posttrain_jax's
``model`` / ``sampler`` generation API). Device compute runs in ``libg4rollout.so`` (gfx950 HIP
kernels, C ABI in ``include/g4_rollout.h``) plus hipBLASLt GEMMs through PyTorch-ROCm.

The directory name is not a Python identifier; ``load_package()`` in ``__graft_entry__`` imports it
as ``gemma4_posttrain_jax_amd``.
"""

__version__ = "0.1.0"
