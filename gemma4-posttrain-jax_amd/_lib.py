"""ctypes binding of ``libg4rollout.so`` (declared in ``include/g4_rollout.h``).

Loading fails loudly: there is no CPU or PyTorch fallback for any entry point. The structs below
mirror the header field by field (ctypes applies the same C alignment rules).
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int32, c_int64, c_size_t, c_uint8, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libg4rollout.so"

G4_OK = 0
G4_DTYPE_F32 = 0
G4_DTYPE_BF16 = 1
G4_CACHE_LINEAR = 0
G4_CACHE_RING = 1
G4_APPEND_NORM_K = 1
G4_APPEND_NORM_V = 2
G4_APPEND_ROPE_K = 4
G4_APPEND_NORM_Q = 8
G4_APPEND_ROPE_Q = 16
G4_DECODE_SPLIT_KEYS = -1
G4_DECODE_TWO_PASS = -2
G4_LINEAR_PLAIN = 0
G4_LINEAR_GELU_MUL = 1
G4_ERR_INVALID = -1
G4_ERR_UNSUPPORTED = -2
G4_ERR_LAUNCH = -3
G4_ERR_WORKSPACE = -4


class G4AppendArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32), ("kind", c_int32), ("batch", c_int32), ("seq", c_int32), ("kv_heads", c_int32),
        ("group", c_int32), ("head_dim", c_int32), ("capacity", c_int32), ("slot_stride", c_int32),
        ("flags", c_int32), ("eps", c_float), ("write_pos_scalar", c_int32), ("write_pos", c_void_p),
        ("k", c_void_p), ("v", c_void_p), ("q", c_void_p), ("in_row_stride", c_int64),
        ("q_norm_weight", c_void_p), ("k_norm_weight", c_void_p), ("rope_cos", c_void_p), ("rope_sin", c_void_p),
        ("cache_k", c_void_p), ("cache_vt", c_void_p), ("q_out", c_void_p), ("k_out", c_void_p),
        ("vt_out", c_void_p), ("chunk_stride", c_int32),
    ]


class G4DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32), ("kind", c_int32), ("batch", c_int32), ("kv_heads", c_int32), ("group", c_int32),
        ("head_dim", c_int32), ("capacity", c_int32), ("slot_stride", c_int32), ("window", c_int32),
        ("q_pos_scalar", c_int32), ("q_pos", c_void_p), ("key_mask", c_void_p), ("key_mask_stride", c_int32),
        ("q", c_void_p), ("cache_k", c_void_p), ("cache_vt", c_void_p), ("cache_k_w", c_void_p),
        ("new_k", c_void_p), ("new_v", c_void_p), ("out", c_void_p), ("workspace", c_void_p),
        ("workspace_bytes", c_size_t), ("prep", c_void_p), ("num_splits", c_int32),
    ]


class G4DecodePrep(ctypes.Structure):
    _fields_ = [
        ("q_raw", c_void_p), ("k_raw", c_void_p), ("v_raw", c_void_p), ("in_row_stride", c_int64),
        ("q_norm_weight", c_void_p), ("k_norm_weight", c_void_p), ("rope_cos", c_void_p), ("rope_sin", c_void_p),
        ("eps", c_float), ("flags", c_int32),
    ]


class G4PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32), ("batch", c_int32), ("seq", c_int32), ("kv_heads", c_int32), ("group", c_int32),
        ("head_dim", c_int32), ("window", c_int32), ("key_mask", c_void_p), ("key_mask_stride", c_int32),
        ("q", c_void_p), ("k", c_void_p), ("vt", c_void_p), ("k_stride", c_int32), ("out", c_void_p),
    ]


# Every symbol include/g4_rollout.h declares, with its ctypes prototype.
class G4SampleArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32), ("batch", c_int32), ("vocab", c_int32), ("proposal_width", c_int32),
        ("logits", c_void_p), ("row_stride", c_int64), ("softcap", c_float), ("temperature", c_float),
        ("split_key", c_int32), ("key", c_void_p), ("proposal", c_void_p), ("proposal_index", c_void_p), ("token_out", c_void_p),
        ("logp_out", c_void_p),
    ]


class G4SampleTopKArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_int32), ("batch", c_int32), ("vocab", c_int32), ("top_k", c_int32), ("logits", c_void_p),
        ("row_stride", c_int64), ("softcap", c_float), ("temperature", c_float), ("top_p", c_float),
        ("split_key", c_int32), ("key", c_void_p), ("token_out", c_void_p), ("logp_out", c_void_p),
    ]


class G4RolloutStepArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_int32), ("max_new", c_int32), ("step", c_int32), ("pad_id", c_int32), ("n_eos", c_int32),
        ("id_bytes", c_int32), ("eos_ids", c_void_p), ("sampled", c_void_p), ("logp", c_void_p), ("active", c_void_p),
        ("prompt_lengths", c_void_p), ("completion_ids", c_void_p), ("completion_mask", c_void_p),
        ("rollout_logps", c_void_p), ("next_token", c_void_p), ("next_pos", c_void_p), ("next_mask", c_void_p),
        ("any_active", c_void_p),
    ]


class G4LmHeadSampleArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_int32), ("vocab", c_int32), ("hidden", c_int32), ("x", c_void_p), ("embed", c_void_p),
        ("softcap", c_float), ("temperature", c_float), ("split_key", c_int32), ("key", c_void_p),
        ("token_out", c_void_p), ("logp_out", c_void_p), ("logits_out", c_void_p), ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
    ]


class G4LinearArgs(ctypes.Structure):
    _fields_ = [
        ("x", c_void_p), ("w", c_void_p), ("y", c_void_p), ("m", c_int32), ("n", c_int32), ("k", c_int32),
        ("ldy", c_int32), ("ksplit", c_int32), ("workspace", c_void_p), ("workspace_bytes", c_size_t),
        ("epilogue", c_int32),
    ]


class G4PrologueArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_int32), ("hidden", c_int32), ("vocab", c_int32), ("key_mask_stride", c_int32),
        ("tokens", c_void_p), ("positions", c_void_p), ("active", c_void_p), ("slot", c_void_p),
        ("key_mask", c_void_p), ("embed", c_void_p), ("embed_scale", c_float), ("n_tables", c_int32),
        ("rot_dim", c_int32 * 2), ("inv_freq", c_void_p * 2), ("cos_out", c_void_p * 2), ("sin_out", c_void_p * 2),
        ("x_out", c_void_p),
    ]


PROTOTYPES = {
    "g4_kv_append": (c_int32, [POINTER(G4AppendArgs), c_void_p]),
    "g4_decode_workspace_size": (c_size_t, [POINTER(G4DecodeArgs)]),
    "g4_decode_attention": (c_int32, [POINTER(G4DecodeArgs), c_void_p]),
    "g4_decode_attention_noalloc": (c_int32, [POINTER(G4DecodeArgs), c_void_p]),
    "g4_prefill_attention": (c_int32, [POINTER(G4PrefillArgs), c_void_p]),
    "g4_kv_source_layers": (c_int32, [c_int32, c_int32, POINTER(c_int32), POINTER(c_int32)]),
    "g4_ring_slot_positions": (c_int32, [c_int32, c_int32, POINTER(c_int32)]),
    "g4_sample_tokens": (c_int32, [POINTER(G4SampleArgs), c_void_p]),
    "g4_sample_top_k": (c_int32, [POINTER(G4SampleTopKArgs), c_void_p]),
    "g4_softcap_bf16": (c_int32, [c_int64, c_void_p, c_float, c_void_p, c_void_p]),
    "g4_lm_head_sample_workspace_size": (c_size_t, [POINTER(G4LmHeadSampleArgs)]),
    "g4_lm_head_sample": (c_int32, [POINTER(G4LmHeadSampleArgs), c_void_p]),
    "g4_rms_norm": (c_int32, [c_int32, c_int32, c_int32, c_void_p, c_void_p, c_float, c_void_p, c_void_p]),
    "g4_residual_norm": (c_int32, [c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                   c_float, c_void_p, c_void_p, c_void_p]),
    "g4_gelu_mul": (c_int32, [c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    "g4_residual_norm_splitk": (c_int32, [c_int32, c_int32, c_void_p, c_int32, c_void_p, c_void_p, c_void_p,
                                          c_void_p, c_float, c_void_p, c_void_p, c_void_p]),
    "g4_decode_prologue": (c_int32, [POINTER(G4PrologueArgs), c_void_p]),
    "g4_rollout_step": (c_int32, [POINTER(G4RolloutStepArgs), c_void_p]),
    "g4_linear_workspace_size": (c_size_t, [POINTER(G4LinearArgs)]),
    "g4_linear_bf16": (c_int32, [POINTER(G4LinearArgs), c_void_p]),
    "g4_convert_f32_to_bf16": (c_int32, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "g4_convert_bf16_to_f32": (c_int32, [c_void_p, c_void_p, c_int64, c_void_p]),
    "g4_init": (c_int32, []),
    "g4_last_error": (c_char_p, []),
    "g4_version": (c_char_p, []),
}

_lib = None


class G4Error(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built (no fallback path exists)."""

    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise G4Error(f"{LIB_PATH} is missing: build it with __graft_entry__.build() (hipcc, gfx950)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, argtypes) in PROTOTYPES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != G4_OK:
        msg = lib().g4_last_error().decode(errors="replace")
        raise G4Error(f"{what} failed ({rc}): {msg}")


_ready_devices: set = set()


def init_device(index: int) -> None:
    """g4_init on device ``index`` (made current around the call), once per process and device:
    the library's one-time kernel set-up, done before any graph capture needs it."""

    if index in _ready_devices:
        return
    import torch

    with torch.cuda.device(index):
        check(lib().g4_init(), "g4_init")
    _ready_devices.add(index)


def kv_source_layers(layer_types: list[int], num_kv_shared_layers: int) -> list[int]:
    n = len(layer_types)
    arr_in = (c_int32 * n)(*layer_types)
    arr_out = (c_int32 * n)()
    check(lib().g4_kv_source_layers(n, num_kv_shared_layers, arr_in, arr_out), "g4_kv_source_layers")
    return list(arr_out)


def ring_slot_positions(last_written: int, window_capacity: int) -> list[int]:
    out = (c_int32 * window_capacity)()
    check(lib().g4_ring_slot_positions(last_written, window_capacity, out), "g4_ring_slot_positions")
    return list(out)


__all__ = [
    "G4AppendArgs", "G4DecodeArgs", "G4PrefillArgs", "G4LinearArgs", "G4PrologueArgs", "G4DecodePrep", "G4Error", "PROTOTYPES", "LIB_PATH", "lib", "check", "init_device",
    "kv_source_layers", "ring_slot_positions", "c_uint8",
]
