"""PyTorch-tensor front end of the native kernels: shape checks, then one C-ABI call each.

Tensors are device buffers only; every computation runs in ``libg4rollout.so`` on the current
torch stream. bf16 tensors are passed by their raw bits (torch.bfloat16 storage is the same
16-bit format the kernels use).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .kvcache import LayerKVCache, key_shape

_DTYPES = {torch.float32: _lib.G4_DTYPE_F32, torch.bfloat16: _lib.G4_DTYPE_BF16}


def _code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; the kernels take float32 or bfloat16") from None


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("kernel operands must be device tensors")
    return t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check_rows(t: torch.Tensor, name: str, B: int, S: int, n: int, D: int, row_stride: int) -> None:
    """``t`` is a [B, S, n, D] view whose tokens are ``row_stride`` elements apart."""

    if tuple(t.shape) != (B, S, n, D):
        raise ValueError(f"{name}: shape {tuple(t.shape)} != {(B, S, n, D)}")
    bad = (D > 1 and t.stride(3) != 1) or (n > 1 and t.stride(2) != D)
    bad = bad or (S > 1 and t.stride(1) != row_stride) or (B > 1 and t.stride(0) != S * row_stride)
    if bad:
        raise ValueError(f"{name}: strides {t.stride()} do not follow rows of {row_stride} elements")


def kv_append(
    layer: LayerKVCache,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    write_pos: int | torch.Tensor,
    flags: int = 0,
    eps: float = 1e-6,
    q: torch.Tensor | None = None,
    q_out: torch.Tensor | None = None,
    q_norm_weight: torch.Tensor | None = None,
    k_norm_weight: torch.Tensor | None = None,
    rope_cos: torch.Tensor | None = None,
    rope_sin: torch.Tensor | None = None,
    k_out: torch.Tensor | None = None,
    vt_out: torch.Tensor | None = None,
) -> None:
    """g4_kv_append: k/v ``[B, S, Hkv, D]`` (and optional q ``[B, S, Hkv, R, D]``) views of rows
    sharing one row stride; writes ``layer`` in place (model.py:368-390 + 463-482)."""

    B, S, H, D = k.shape
    rs = k.stride(1) if S > 1 else (k.stride(0) if B > 1 else H * D)
    _check_rows(k, "k", B, S, H, D, rs)
    _check_rows(v, "v", B, S, H, D, rs)
    if k.dtype != layer.key.dtype or v.dtype != k.dtype:
        raise TypeError("k/v/cache dtypes differ")
    if tuple(layer.key.shape[:2]) != (B, H) or layer.head_dim != D:
        raise ValueError(f"cache {tuple(layer.key.shape)} does not match k {tuple(k.shape)}")
    R = 0
    if q is not None:
        R = q.shape[3]
        if tuple(q.shape) != (B, S, H, R, D) or q.stride(4) != 1 or q.stride(3) != D or q.stride(2) != R * D:
            raise ValueError(f"q: shape {tuple(q.shape)} / strides {q.stride()}")
        if (S > 1 and q.stride(1) != rs) or (B > 1 and q.stride(0) != S * rs):
            raise ValueError("q must share k's row stride")
        if q_out is None or tuple(q_out.shape) != (B, S, H, R, D) or not q_out.is_contiguous():
            raise ValueError("q_out must be a contiguous [B, S, Hkv, R, D] tensor")
    chunk_stride = 0
    if k_out is not None or vt_out is not None:
        if k_out is None or vt_out is None:
            raise ValueError("k_out and vt_out go together")
        chunk_stride = k_out.shape[2] * 32
        if (tuple(k_out.shape) != key_shape(B, H, chunk_stride, D)
                or tuple(vt_out.shape) != (B, H, chunk_stride // 8, D, 8)):
            raise ValueError("k_out / vt_out shapes")
        if not (k_out.is_contiguous() and vt_out.is_contiguous()):
            raise ValueError("k_out / vt_out must be contiguous")
    if isinstance(write_pos, torch.Tensor):
        if write_pos.dtype != torch.int32 or tuple(write_pos.shape) != (B,) or not write_pos.is_contiguous():
            raise ValueError("write_pos must be a contiguous int32 [B] tensor")
        wp_ptr, wp_scalar = _ptr(write_pos), 0
    else:
        wp_ptr, wp_scalar = None, int(write_pos)
    if flags & (_lib.G4_APPEND_ROPE_K | _lib.G4_APPEND_ROPE_Q):
        for t in (rope_cos, rope_sin):
            if t is None or t.dtype != torch.float32 or tuple(t.shape) != (B, S, D) or not t.is_contiguous():
                raise ValueError("rope_cos/rope_sin must be contiguous float32 [B, S, D]")
    a = _lib.G4AppendArgs(
        dtype=_code(k), kind=_lib.G4_CACHE_RING if layer.ring else _lib.G4_CACHE_LINEAR, batch=B, seq=S, kv_heads=H,
        group=R, head_dim=D, capacity=layer.capacity, slot_stride=layer.slot_stride, flags=flags, eps=eps,
        write_pos_scalar=wp_scalar, write_pos=wp_ptr, k=_ptr(k), v=_ptr(v), q=_ptr(q), in_row_stride=rs,
        q_norm_weight=_ptr(q_norm_weight), k_norm_weight=_ptr(k_norm_weight), rope_cos=_ptr(rope_cos),
        rope_sin=_ptr(rope_sin), cache_k=_ptr(layer.key), cache_vt=_ptr(layer.value_t), q_out=_ptr(q_out),
        k_out=_ptr(k_out), vt_out=_ptr(vt_out), chunk_stride=chunk_stride,
    )
    _lib.check(_lib.lib().g4_kv_append(ctypes.byref(a), _stream()), "g4_kv_append")


def prepare_q(
    q: torch.Tensor,
    q_out: torch.Tensor,
    *,
    flags: int,
    eps: float,
    q_norm_weight: torch.Tensor | None,
    rope_cos: torch.Tensor | None,
    rope_sin: torch.Tensor | None,
) -> None:
    """g4_kv_append with q only (kv-shared layers): q ``[B, S, Hkv, R, D]`` view -> ``q_out``."""

    B, S, H, R, D = q.shape
    rs = q.stride(1) if S > 1 else (q.stride(0) if B > 1 else H * R * D)
    if q.stride(4) != 1 or q.stride(3) != D or q.stride(2) != R * D or (B > 1 and q.stride(0) != S * rs):
        raise ValueError(f"q strides {q.stride()}")
    if tuple(q_out.shape) != (B, S, H, R, D) or not q_out.is_contiguous() or q_out.dtype != q.dtype:
        raise ValueError("q_out must be a contiguous [B, S, Hkv, R, D] tensor in q's dtype")
    if flags & _lib.G4_APPEND_ROPE_Q:
        for t in (rope_cos, rope_sin):
            if t is None or t.dtype != torch.float32 or tuple(t.shape) != (B, S, D) or not t.is_contiguous():
                raise ValueError("rope_cos/rope_sin must be contiguous float32 [B, S, D]")
    a = _lib.G4AppendArgs(
        dtype=_code(q), kind=_lib.G4_CACHE_LINEAR, batch=B, seq=S, kv_heads=H, group=R, head_dim=D, capacity=S,
        slot_stride=(S + 63) // 64 * 64, flags=flags, eps=eps, write_pos_scalar=0, write_pos=None, k=None, v=None,
        q=_ptr(q), in_row_stride=rs, q_norm_weight=_ptr(q_norm_weight), k_norm_weight=None, rope_cos=_ptr(rope_cos),
        rope_sin=_ptr(rope_sin), cache_k=None, cache_vt=None, q_out=_ptr(q_out), k_out=None, vt_out=None,
        chunk_stride=0,
    )
    _lib.check(_lib.lib().g4_kv_append(ctypes.byref(a), _stream()), "g4_kv_append")


def decode_attention(
    layer: LayerKVCache,
    q: torch.Tensor,
    key_mask: torch.Tensor,
    *,
    q_pos: int | torch.Tensor,
    window: int,
    out: torch.Tensor | None = None,
    new_k: torch.Tensor | None = None,
    new_v: torch.Tensor | None = None,
    num_splits: int = 0,
    no_alloc: bool = False,
) -> torch.Tensor:
    """g4_decode_attention: q ``[B, Hkv, R, D]`` against ``layer``; returns ``[B, Hkv, R, D]``.
    With ``new_k``/``new_v`` (``[B, Hkv, D]``) the token's K/V is stored at ``q_pos`` first.
    ``num_splits``: 0 lets the library choose; 1 or 2 workgroups per (b, kv head) in one pass;
    ``_lib.G4_DECODE_SPLIT_KEYS`` splits the key range (long rows). A workspace of the size the
    library asks for is allocated from torch's caching allocator on the current stream; with
    ``no_alloc`` the call goes to g4_decode_attention_noalloc, which uses the library's own
    per-device scratch (``out`` must then be given for the call to allocate nothing at all)."""

    B, H, R, D = q.shape
    if not q.is_contiguous() or q.dtype != layer.key.dtype:
        raise ValueError("q must be contiguous and in the cache dtype")
    if tuple(layer.key.shape[:2]) != (B, H) or layer.head_dim != D:
        raise ValueError(f"cache {tuple(layer.key.shape)} does not match q {tuple(q.shape)}")
    if key_mask.dtype != torch.bool or key_mask.dim() != 2 or key_mask.shape[0] != B or key_mask.stride(1) != 1:
        raise ValueError("key_mask must be a [B, C] bool tensor with unit inner stride")
    if out is None:
        out = torch.empty_like(q)
    elif tuple(out.shape) != (B, H, R, D) or not out.is_contiguous() or out.dtype != q.dtype:
        raise ValueError("out must be a contiguous [B, Hkv, R, D] tensor in q's dtype")
    for name, t in (("new_k", new_k), ("new_v", new_v)):
        if t is not None and (tuple(t.shape) != (B, H, D) or not t.is_contiguous() or t.dtype != q.dtype):
            raise ValueError(f"{name} must be a contiguous [B, Hkv, D] tensor in q's dtype")
    if isinstance(q_pos, torch.Tensor):
        if q_pos.dtype != torch.int32 or tuple(q_pos.shape) != (B,) or not q_pos.is_contiguous():
            raise ValueError("q_pos must be a contiguous int32 [B] tensor")
        qp_ptr, qp_scalar = _ptr(q_pos), 0
    else:
        qp_ptr, qp_scalar = None, int(q_pos)
    a = _lib.G4DecodeArgs(
        dtype=_code(q), kind=_lib.G4_CACHE_RING if layer.ring else _lib.G4_CACHE_LINEAR, batch=B, kv_heads=H,
        group=R, head_dim=D, capacity=layer.capacity, slot_stride=layer.slot_stride, window=window,
        q_pos_scalar=qp_scalar, q_pos=qp_ptr, key_mask=_ptr(key_mask), key_mask_stride=key_mask.stride(0),
        q=_ptr(q), cache_k=_ptr(layer.key), cache_vt=_ptr(layer.value_t), cache_k_w=_ptr(layer.key),
        new_k=_ptr(new_k), new_v=_ptr(new_v), out=_ptr(out), workspace=None, workspace_bytes=0, prep=None,
        num_splits=num_splits,
    )
    if no_alloc:
        _lib.check(_lib.lib().g4_decode_attention_noalloc(ctypes.byref(a), _stream()), "g4_decode_attention_noalloc")
        return out
    need = _lib.lib().g4_decode_workspace_size(ctypes.byref(a))
    ws = None
    if need:
        ws = torch.empty(need, dtype=torch.uint8, device=q.device)
        a.workspace, a.workspace_bytes = ws.data_ptr(), need
    _lib.check(_lib.lib().g4_decode_attention(ctypes.byref(a), _stream()), "g4_decode_attention")
    return out


def decode_attention_fused(
    layer: LayerKVCache,
    q_raw: torch.Tensor,
    key_mask: torch.Tensor,
    *,
    q_pos: torch.Tensor,
    window: int,
    k_raw: torch.Tensor | None,
    v_raw: torch.Tensor | None,
    q_norm_weight: torch.Tensor | None,
    k_norm_weight: torch.Tensor | None,
    rope_cos: torch.Tensor,
    rope_sin: torch.Tensor,
    eps: float,
    flags: int,
) -> torch.Tensor:
    """g4_decode_attention with G4DecodePrep: the raw projection rows in, g4_kv_append's work (q / k
    norm + RoPE, v norm, and with k_raw / v_raw the append into ``layer``; a kv-shared layer passes
    its source cache and no k / v) done inside the two-launch attention. q_raw ``[B, Hkv, R, D]`` and
    k_raw / v_raw ``[B, Hkv, D]`` are views of the projection output sharing one batch-row stride;
    rope_cos / rope_sin f32 ``[B, D]``. Returns ``[B, Hkv, R, D]``."""

    B, H, R, D = q_raw.shape
    stride = q_raw.stride(0)
    if q_raw.dtype != layer.key.dtype or q_raw.stride(3) != 1 or q_raw.stride(2) != D or q_raw.stride(1) != R * D:
        raise ValueError("q_raw must hold [Hkv, R, D] contiguous rows in the cache dtype")
    for name, t in (("k_raw", k_raw), ("v_raw", v_raw)):
        if t is not None and (tuple(t.shape) != (B, H, D) or t.stride(0) != stride or t.stride(1) != D
                              or t.stride(2) != 1 or t.dtype != q_raw.dtype):
            raise ValueError(f"{name} must be [B, Hkv, D] rows sharing q_raw's batch stride")
    if (k_raw is None) != (v_raw is None):
        raise ValueError("k_raw and v_raw go together")
    for name, t in (("rope_cos", rope_cos), ("rope_sin", rope_sin)):
        if t.dtype != torch.float32 or t.numel() != B * D or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous f32 [B, D] table")
    if key_mask.dtype != torch.bool or key_mask.dim() != 2 or key_mask.shape[0] != B or key_mask.stride(1) != 1:
        raise ValueError("key_mask must be a [B, C] bool tensor with unit inner stride")
    if q_pos.dtype != torch.int32 or tuple(q_pos.shape) != (B,) or not q_pos.is_contiguous():
        raise ValueError("q_pos must be a contiguous int32 [B] tensor")
    out = torch.empty((B, H, R, D), dtype=q_raw.dtype, device=q_raw.device)
    prep = _lib.G4DecodePrep(q_raw=_ptr(q_raw), k_raw=_ptr(k_raw), v_raw=_ptr(v_raw), in_row_stride=stride,
                             q_norm_weight=_ptr(q_norm_weight), k_norm_weight=_ptr(k_norm_weight),
                             rope_cos=_ptr(rope_cos), rope_sin=_ptr(rope_sin), eps=eps, flags=flags)
    a = _lib.G4DecodeArgs(
        dtype=_code(q_raw), kind=_lib.G4_CACHE_RING if layer.ring else _lib.G4_CACHE_LINEAR, batch=B, kv_heads=H,
        group=R, head_dim=D, capacity=layer.capacity, slot_stride=layer.slot_stride, window=window,
        q_pos_scalar=0, q_pos=_ptr(q_pos), key_mask=_ptr(key_mask), key_mask_stride=key_mask.stride(0),
        q=None, cache_k=_ptr(layer.key), cache_vt=_ptr(layer.value_t), cache_k_w=_ptr(layer.key),
        new_k=None, new_v=None, out=_ptr(out), workspace=None, workspace_bytes=0,
        prep=ctypes.cast(ctypes.pointer(prep), ctypes.c_void_p), num_splits=0,
    )
    need = _lib.lib().g4_decode_workspace_size(ctypes.byref(a))
    ws = torch.empty(need, dtype=torch.uint8, device=q_raw.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), need
    _lib.check(_lib.lib().g4_decode_attention(ctypes.byref(a), _stream()), "g4_decode_attention")
    return out


def prefill_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    vt: torch.Tensor,
    key_mask: torch.Tensor,
    *,
    window: int,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """g4_prefill_attention: q ``[B, S, Hkv, R, D]``, k ``key_shape(B, Hkv, Sp, D)`` and vt
    ``[B, Hkv, Sp / 8, D, 8]`` (the caches' layouts; Sp >= S, multiple of 64); returns
    ``[B, S, Hkv, R, D]``."""

    B, S, H, R, D = q.shape
    Sp = k.shape[2] * 32
    if (not q.is_contiguous() or tuple(k.shape) != key_shape(B, H, Sp, D)
            or tuple(vt.shape) != (B, H, Sp // 8, D, 8)):
        raise ValueError(f"q {tuple(q.shape)} / k {tuple(k.shape)} / vt {tuple(vt.shape)}")
    if not (k.is_contiguous() and vt.is_contiguous()) or k.dtype != q.dtype or vt.dtype != q.dtype:
        raise ValueError("k/vt must be contiguous and in q's dtype")
    if key_mask.dtype != torch.bool or key_mask.dim() != 2 or key_mask.shape[0] != B or key_mask.stride(1) != 1:
        raise ValueError("key_mask must be a [B, >=S] bool tensor with unit inner stride")
    if out is None:
        out = torch.empty_like(q)
    a = _lib.G4PrefillArgs(
        dtype=_code(q), batch=B, seq=S, kv_heads=H, group=R, head_dim=D, window=window, key_mask=_ptr(key_mask),
        key_mask_stride=key_mask.stride(0), q=_ptr(q), k=_ptr(k), vt=_ptr(vt), k_stride=Sp, out=_ptr(out),
    )
    _lib.check(_lib.lib().g4_prefill_attention(ctypes.byref(a), _stream()), "g4_prefill_attention")
    return out


# --- fused decoder-layer glue ------------------------------------------------------------------------


def _rows(x: torch.Tensor) -> tuple[int, int]:
    if not x.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return x.numel() // x.shape[-1], x.shape[-1]


def rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """g4_rms_norm over the last dim: ``cast(x * (mean(x^2) + eps)^-0.5 * w)`` (f32 inside)."""

    rows, cols = _rows(x)
    if weight is not None and (weight.dtype != x.dtype or weight.numel() != cols or not weight.is_contiguous()):
        raise ValueError("weight must be a contiguous [cols] tensor in x's dtype")
    out = torch.empty_like(x) if out is None else out
    _lib.check(_lib.lib().g4_rms_norm(_code(x), rows, cols, _ptr(x), _ptr(weight), eps, _ptr(out), _stream()),
               "g4_rms_norm")
    return out


def residual_norm(branch: torch.Tensor, branch_weight: torch.Tensor | None, residual: torch.Tensor, *,
                  scalar: torch.Tensor | None, next_weight: torch.Tensor | None, eps: float,
                  with_next: bool = True) -> tuple[torch.Tensor, torch.Tensor | None]:
    """g4_residual_norm: ``x = cast(cast(residual + cast(rms(branch) * w)) * scalar)`` and, with
    ``with_next``, ``h = cast(rms(x) * next_weight)``; returns ``(x, h)``. ``scalar`` is a one-
    element f32 tensor (or None)."""

    rows, cols = _rows(branch)
    if residual.shape != branch.shape or residual.dtype != branch.dtype or not residual.is_contiguous():
        raise ValueError("residual must match branch")
    for w in (branch_weight, next_weight):
        if w is not None and (w.dtype != branch.dtype or w.numel() != cols or not w.is_contiguous()):
            raise ValueError("norm weights must be contiguous [cols] tensors in the activation dtype")
    if scalar is not None and (scalar.dtype != torch.float32 or scalar.numel() != 1):
        raise ValueError("scalar must be a one-element f32 tensor")
    x = torch.empty_like(branch)
    h = torch.empty_like(branch) if with_next else None
    _lib.check(_lib.lib().g4_residual_norm(_code(branch), rows, cols, _ptr(branch), _ptr(branch_weight),
                                           _ptr(residual), _ptr(scalar), _ptr(next_weight), eps, _ptr(x), _ptr(h),
                                           _stream()), "g4_residual_norm")
    return x, h


def gelu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """g4_gelu_mul: ``[rows, 2F] -> [rows, F]``, ``cast(gelu_tanh(g) * u)`` in f32."""

    rows, cols2 = _rows(gate_up)
    if cols2 % 2:
        raise ValueError("gate_up must have an even last dim")
    out = torch.empty(gate_up.shape[:-1] + (cols2 // 2,), dtype=gate_up.dtype, device=gate_up.device)
    _lib.check(_lib.lib().g4_gelu_mul(_code(gate_up), rows, cols2 // 2, _ptr(gate_up), _ptr(out), _stream()),
               "g4_gelu_mul")
    return out


# --- sampling ------------------------------------------------------------------------------------------


def sample_tokens(logits: torch.Tensor, *, softcap: float | None, temperature: float, key: torch.Tensor | None,
                  split_key: bool = True, proposal: torch.Tensor | None = None, proposal_index: torch.Tensor | None = None,
                  token_out: torch.Tensor | None = None,
                  logp_out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """g4_sample_tokens on ``[B, V]`` logits (bf16 or f32, rows may be strided): soft-cap (None/0 =
    already capped), then greedy (temperature <= 0) or a categorical draw over ``logits /
    temperature``, or over ``proposal [B, K]`` f32 (truncated scores; column j is vocab id
    ``proposal_index[:, j]``). ``key`` is a 2-word int32 device tensor: with ``split_key`` the
    generation loop's key, split (the draw uses the second half and ``key`` is advanced in place to
    the first), otherwise the sample key itself, left unchanged. Returns ``(token int32 [B], logp f32 [B])`` with logp the
    full-vocab log-softmax of the capped logits at the token."""

    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [B, V] with unit inner stride")
    B, V = logits.shape
    dev = logits.device
    if key is not None and (key.dtype != torch.int32 or key.numel() != 2 or not key.is_contiguous()
                            or key.device != dev):
        raise ValueError("key must be a contiguous 2-element int32 tensor on the logits' device")
    K = 0
    if proposal is not None:
        if proposal.dtype != torch.float32 or proposal.dim() != 2 or proposal.shape[0] != B:
            raise ValueError("proposal must be [B, K] float32")
        proposal = proposal.contiguous()
        K = proposal.shape[1]
        if proposal_index is not None:
            if proposal_index.shape != proposal.shape:
                raise ValueError("proposal_index must match the proposal's shape")
            proposal_index = proposal_index.to(torch.int32).contiguous()
    elif proposal_index is not None:
        raise ValueError("proposal_index needs a proposal")
    token_out = torch.empty(B, dtype=torch.int32, device=dev) if token_out is None else token_out
    logp_out = torch.empty(B, dtype=torch.float32, device=dev) if logp_out is None else logp_out
    a = _lib.G4SampleArgs(
        dtype=_code(logits), batch=B, vocab=V, proposal_width=K, logits=_ptr(logits), row_stride=logits.stride(0),
        softcap=float(softcap or 0.0), temperature=float(temperature), split_key=int(bool(split_key)), key=_ptr(key) if key is not None else None,
        proposal=_ptr(proposal) if proposal is not None else None,
        proposal_index=_ptr(proposal_index) if proposal_index is not None else None,
        token_out=_ptr(token_out), logp_out=_ptr(logp_out),
    )
    _lib.check(_lib.lib().g4_sample_tokens(ctypes.byref(a), _stream()), "g4_sample_tokens")
    return token_out, logp_out


TOP_K_MAX = 256  # the largest top_k g4_sample_top_k takes


def sample_top_k(logits: torch.Tensor, *, softcap: float | None, temperature: float, top_k: int, top_p: float,
                 key: torch.Tensor, split_key: bool = True, token_out: torch.Tensor | None = None,
                 logp_out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """g4_sample_top_k on ``[B, V]`` logits (bf16 or f32, rows may be strided): the top-k (+ top-p)
    categorical draw of sampler.py:162-183 over ``capped logits / temperature`` (0 < top_k < V,
    top_k <= TOP_K_MAX, temperature > 0), scored under the full f32 policy; ``key`` as in
    sample_tokens. Returns ``(token int32 [B], logp f32 [B])``."""

    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [B, V] with unit inner stride")
    B, V = logits.shape
    dev = logits.device
    if key is None or key.dtype != torch.int32 or key.numel() != 2 or not key.is_contiguous() or key.device != dev:
        raise ValueError("key must be a contiguous 2-element int32 tensor on the logits' device")
    token_out = torch.empty(B, dtype=torch.int32, device=dev) if token_out is None else token_out
    logp_out = torch.empty(B, dtype=torch.float32, device=dev) if logp_out is None else logp_out
    a = _lib.G4SampleTopKArgs(
        dtype=_code(logits), batch=B, vocab=V, top_k=int(top_k), logits=_ptr(logits), row_stride=logits.stride(0),
        softcap=float(softcap or 0.0), temperature=float(temperature), top_p=float(top_p),
        split_key=int(bool(split_key)), key=_ptr(key), token_out=_ptr(token_out), logp_out=_ptr(logp_out),
    )
    _lib.check(_lib.lib().g4_sample_top_k(ctypes.byref(a), _stream()), "g4_sample_top_k")
    return token_out, logp_out


def rollout_step(step: int, sampled: torch.Tensor, logp: torch.Tensor, active: torch.Tensor, *,
                 completion_ids: torch.Tensor, completion_mask: torch.Tensor, rollout_logps: torch.Tensor,
                 pad_id: int, eos_ids: torch.Tensor | None, prompt_lengths: torch.Tensor | None = None,
                 next_token: torch.Tensor | None = None, next_pos: torch.Tensor | None = None,
                 next_mask: torch.Tensor | None = None, any_active: torch.Tensor | None = None) -> None:
    """g4_rollout_step: the bookkeeping of one generate step (sampler.py:279-296) in one launch.
    Column ``step`` of ``completion_ids`` (int32/int64) / ``completion_mask`` (bool) /
    ``rollout_logps`` (f32) receives the drawn token and logp of the rows in ``active`` (pad and 0
    elsewhere); ``active`` (bool [B]) is cleared in place for rows whose token is in ``eos_ids``
    (int32 [n]); ``next_token`` / ``next_pos`` / ``next_mask`` (int32 / int32 / bool [B], optional)
    receive the next decode step's inputs (the token, ``prompt_lengths + step``, the mask before the
    update) and ``any_active`` (bool [1], optional) whether a row stays active."""

    B = sampled.shape[0]
    dev = sampled.device
    if B <= 0:
        raise ValueError("rollout_step needs at least one row")
    N = completion_ids.shape[1] if completion_ids.dim() == 2 else -1
    if not 0 <= step < N:
        raise ValueError(f"step {step} outside the completion width {N}")

    def want(t, name, dtype, shape):
        if t is not None and (t.dtype != dtype or tuple(t.shape) != shape or not t.is_contiguous() or t.device != dev):
            raise ValueError(f"{name} must be a contiguous {dtype} tensor of shape {shape} on {dev}")

    want(sampled, "sampled", torch.int32, (B,))
    want(logp, "logp", torch.float32, (B,))
    want(active, "active", torch.bool, (B,))
    if completion_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError("completion_ids must be int32 or int64")
    want(completion_ids, "completion_ids", completion_ids.dtype, (B, N))
    want(completion_mask, "completion_mask", torch.bool, (B, N))
    want(rollout_logps, "rollout_logps", torch.float32, (B, N))
    want(prompt_lengths, "prompt_lengths", torch.int32, (B,))
    want(next_token, "next_token", torch.int32, (B,))
    want(next_pos, "next_pos", torch.int32, (B,))
    want(next_mask, "next_mask", torch.bool, (B,))
    want(any_active, "any_active", torch.bool, (1,))
    n_eos = 0 if eos_ids is None else eos_ids.numel()
    if n_eos:
        want(eos_ids, "eos_ids", torch.int32, (n_eos,))
    if next_pos is not None and prompt_lengths is None:
        raise ValueError("next_pos needs prompt_lengths")
    a = _lib.G4RolloutStepArgs(
        batch=B, max_new=N, step=int(step), pad_id=int(pad_id), n_eos=n_eos, id_bytes=completion_ids.element_size(),
        eos_ids=_ptr(eos_ids) if n_eos else None, sampled=_ptr(sampled), logp=_ptr(logp), active=_ptr(active),
        prompt_lengths=_ptr(prompt_lengths), completion_ids=_ptr(completion_ids),
        completion_mask=_ptr(completion_mask), rollout_logps=_ptr(rollout_logps), next_token=_ptr(next_token),
        next_pos=_ptr(next_pos), next_mask=_ptr(next_mask), any_active=_ptr(any_active),
    )
    _lib.check(_lib.lib().g4_rollout_step(ctypes.byref(a), _stream()), "g4_rollout_step")


def softcap(x: torch.Tensor, cap: float, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """g4_softcap_bf16: ``bf16(tanh(x / cap) * cap)`` elementwise over a contiguous bf16 tensor (the
    f32 division, tanh and multiply of forward_lm_head's soft-cap); ``out`` may be ``x``."""

    if x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError("softcap takes a contiguous bf16 tensor")
    out = torch.empty_like(x) if out is None else out
    if out.dtype != x.dtype or out.shape != x.shape or not out.is_contiguous():
        raise ValueError("out must be a contiguous bf16 tensor of x's shape")
    _lib.check(_lib.lib().g4_softcap_bf16(x.numel(), _ptr(x), float(cap), _ptr(out), _stream()), "g4_softcap_bf16")
    return out


LM_HEAD_MAX_ROWS = 256


def lm_head_supported(x: torch.Tensor, embed: torch.Tensor) -> bool:
    """Whether g4_lm_head_sample takes ``x [B, M] . embed [V, M]^T``: bf16, B <= 256, V % 128 == 0,
    M % 32 == 0 (contiguous operands)."""

    return (x.dtype == torch.bfloat16 and embed.dtype == torch.bfloat16 and x.dim() == 2 and embed.dim() == 2
            and 0 < x.shape[0] <= LM_HEAD_MAX_ROWS and x.shape[1] == embed.shape[1] and embed.shape[0] % 128 == 0
            and x.shape[1] % 32 == 0 and embed.shape[0] * embed.shape[1] * 2 < 2 ** 32)


def _lm_head_call(x: torch.Tensor, embed: torch.Tensor, *, softcap: float | None, temperature: float,
                  key: torch.Tensor | None, split_key: bool, token_out: torch.Tensor | None,
                  logp_out: torch.Tensor | None, logits_out: torch.Tensor | None) -> torch.Tensor | None:
    if not lm_head_supported(x, embed):
        raise ValueError(f"g4_lm_head_sample does not take x {tuple(x.shape)} {x.dtype} / embed "
                         f"{tuple(embed.shape)} {embed.dtype} (bf16, rows <= 256, vocab % 128, hidden % 32)")
    x, embed = x.contiguous(), embed.contiguous()
    B, M = x.shape
    V = embed.shape[0]
    dev = x.device
    if key is not None and (key.dtype != torch.int32 or key.numel() != 2 or not key.is_contiguous()
                            or key.device != dev):
        raise ValueError("key must be a contiguous 2-element int32 tensor on x's device")
    if logits_out is not None and (logits_out.dtype != torch.bfloat16 or tuple(logits_out.shape) != (B, V)
                                   or not logits_out.is_contiguous()):
        raise ValueError(f"logits_out must be a contiguous bf16 [{B}, {V}] tensor")
    a = _lib.G4LmHeadSampleArgs(
        batch=B, vocab=V, hidden=M, x=_ptr(x), embed=_ptr(embed), softcap=float(softcap or 0.0),
        temperature=float(temperature), split_key=int(bool(split_key)), key=_ptr(key),
        token_out=_ptr(token_out), logp_out=_ptr(logp_out), logits_out=_ptr(logits_out), workspace=None,
        workspace_bytes=0)
    need = _lib.lib().g4_lm_head_sample_workspace_size(ctypes.byref(a))
    ws = None
    if need:
        ws = torch.empty(need // 4, dtype=torch.float32, device=dev)
        a.workspace, a.workspace_bytes = ws.data_ptr(), need
    _lib.check(_lib.lib().g4_lm_head_sample(ctypes.byref(a), _stream()), "g4_lm_head_sample")
    return ws


def lm_head(x: torch.Tensor, embed: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """g4_lm_head_sample without sampling: ``bf16(x [B, M] . embed [V, M]^T)`` with f32 accumulation
    (the logits before the soft-cap)."""

    if out is None:
        out = torch.empty((x.shape[0], embed.shape[0]), dtype=torch.bfloat16, device=x.device)
    _lm_head_call(x, embed, softcap=None, temperature=0.0, key=None, split_key=False, token_out=None,
                  logp_out=None, logits_out=out)
    return out


def lm_head_sample(x: torch.Tensor, embed: torch.Tensor, *, softcap: float | None, temperature: float,
                   key: torch.Tensor | None, split_key: bool = True, token_out: torch.Tensor | None = None,
                   logp_out: torch.Tensor | None = None,
                   logits_out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """g4_lm_head_sample: the LM head ``x [B, M] . embed [V, M]^T`` with sample_tokens' draw (no
    proposal) on its bf16 logits in the epilogue, the logits never stored unless ``logits_out`` is
    given. Same key / temperature / soft-cap semantics as sample_tokens; returns ``(token int32 [B],
    logp f32 [B])``."""

    B = x.shape[0]
    token_out = torch.empty(B, dtype=torch.int32, device=x.device) if token_out is None else token_out
    logp_out = torch.empty(B, dtype=torch.float32, device=x.device) if logp_out is None else logp_out
    _lm_head_call(x, embed, softcap=softcap, temperature=temperature, key=key, split_key=split_key,
                  token_out=token_out, logp_out=logp_out, logits_out=logits_out)
    return token_out, logp_out


def decode_prologue(embed: torch.Tensor, tokens: torch.Tensor, positions: torch.Tensor, active: torch.Tensor,
                    slot: torch.Tensor, key_mask: torch.Tensor, *, embed_scale: float,
                    inv_freq: list[torch.Tensor]) -> tuple[torch.Tensor, list[tuple[torch.Tensor, torch.Tensor]]]:
    """g4_decode_prologue: ``x = bf16(embed[tokens] * embed_scale)`` ``[B, M]``, ``key_mask[b, slot[b]] =
    active[b]`` in place, and per ``inv_freq`` table the f32 rotary ``(cos, sin)`` ``[B, D]`` of
    ``positions``. tokens / positions / slot: int32 ``[B]``, active: bool ``[B]``."""

    B = tokens.shape[0]
    if embed.dtype != torch.bfloat16 or embed.dim() != 2 or not embed.is_contiguous():
        raise ValueError("embed must be a contiguous bf16 [vocab, hidden] tensor")
    for name, t, dt in (("tokens", tokens, torch.int32), ("positions", positions, torch.int32),
                        ("slot", slot, torch.int32), ("active", active, torch.bool)):
        if t.dtype != dt or tuple(t.shape) != (B,):
            raise ValueError(f"{name} must be a [{B}] {dt} tensor")
    tokens, positions, slot, active = (t.contiguous() for t in (tokens, positions, slot, active))
    if key_mask.dtype != torch.bool or key_mask.dim() != 2 or key_mask.shape[0] != B or key_mask.stride(1) != 1:
        raise ValueError("key_mask must be a [B, C] bool tensor with unit inner stride")
    if len(inv_freq) > 2 or any(f.dtype != torch.float32 or f.dim() != 1 or not f.is_contiguous() for f in inv_freq):
        raise ValueError("inv_freq: at most two contiguous f32 [D/2] tensors")
    x = torch.empty((B, embed.shape[1]), dtype=embed.dtype, device=embed.device)
    tables = [(torch.empty((B, 2 * f.numel()), dtype=torch.float32, device=embed.device),
               torch.empty((B, 2 * f.numel()), dtype=torch.float32, device=embed.device)) for f in inv_freq]
    a = _lib.G4PrologueArgs(batch=B, hidden=embed.shape[1], vocab=embed.shape[0], key_mask_stride=key_mask.stride(0),
                            tokens=_ptr(tokens), positions=_ptr(positions), active=_ptr(active), slot=_ptr(slot),
                            key_mask=_ptr(key_mask), embed=_ptr(embed), embed_scale=embed_scale,
                            n_tables=len(inv_freq), x_out=_ptr(x))
    for i, (f, (c, sn)) in enumerate(zip(inv_freq, tables)):
        a.rot_dim[i] = 2 * f.numel()
        a.inv_freq[i], a.cos_out[i], a.sin_out[i] = _ptr(f), _ptr(c), _ptr(sn)
    _lib.check(_lib.lib().g4_decode_prologue(ctypes.byref(a), _stream()), "g4_decode_prologue")
    return x, tables


def _linear_call(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None, ksplit: int,
                 epilogue: int = _lib.G4_LINEAR_PLAIN) -> torch.Tensor | None:
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or x.dim() != 2 or w.dim() != 2:
        raise ValueError("linear needs 2-D bf16 x and w")
    if not x.is_contiguous() or not w.is_contiguous() or x.shape[1] != w.shape[1]:
        raise ValueError(f"x {tuple(x.shape)} and w {tuple(w.shape)} must be contiguous with equal k")
    m, k = x.shape
    n = w.shape[0]
    ny = n // 2 if epilogue == _lib.G4_LINEAR_GELU_MUL else n
    if out is not None and (out.dtype != x.dtype or out.dim() != 2 or tuple(out.shape) != (m, ny) or out.stride(1) != 1):
        raise ValueError(f"out must be a bf16 [{m}, {ny}] tensor with unit inner stride")
    a = _lib.G4LinearArgs(x=_ptr(x), w=_ptr(w), y=_ptr(out), m=m, n=n, k=k, ldy=out.stride(0) if out is not None else 0,
                          ksplit=ksplit, workspace=None, workspace_bytes=0, epilogue=epilogue)
    need = _lib.lib().g4_linear_workspace_size(ctypes.byref(a))
    ws = None
    if need:
        ws = torch.empty(need // 4, dtype=torch.float32, device=x.device)
        a.workspace, a.workspace_bytes = ws.data_ptr(), need
    _lib.check(_lib.lib().g4_linear_bf16(ctypes.byref(a), _stream()), "g4_linear_bf16")
    return ws


def linear(x: torch.Tensor, w: torch.Tensor, *, out: torch.Tensor | None = None, ksplit: int = 1) -> torch.Tensor:
    """g4_linear_bf16: ``x [m, k] @ w[n, k]^T`` in bf16 with f32 accumulation (m <= 256, the decode
    batch); ``ksplit`` > 1 splits k across workgroups (partials in a workspace from torch's caching
    allocator, added in split order)."""

    if out is None:
        out = torch.empty((x.shape[0], w.shape[0]), dtype=x.dtype, device=x.device)
    _linear_call(x, w, out, ksplit)
    return out


def linear_gelu(x: torch.Tensor, w_gate_up: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """g4_linear_bf16 with the gated-GELU epilogue: ``w_gate_up [2F, k]`` = gate rows then up rows;
    returns ``bf16(gelu_tanh(g) * u)`` ``[m, F]`` with g / u the bf16 gate / up products."""

    if out is None:
        out = torch.empty((x.shape[0], w_gate_up.shape[0] // 2), dtype=x.dtype, device=x.device)
    _linear_call(x, w_gate_up, out, 1, _lib.G4_LINEAR_GELU_MUL)
    return out


def linear_partials(x: torch.Tensor, w: torch.Tensor, *, ksplit: int) -> torch.Tensor:
    """g4_linear_bf16 without y: the f32 partial sums ``[ksplit, m, n]`` of ``x @ w^T`` over ksplit
    k ranges (for ``residual_norm_splitk``)."""

    if ksplit < 2:
        raise ValueError("linear_partials needs ksplit >= 2")
    ws = _linear_call(x, w, None, ksplit)
    return ws.view(ksplit, x.shape[0], w.shape[0])


def residual_norm_splitk(partials: torch.Tensor, branch_weight: torch.Tensor | None, residual: torch.Tensor, *,
                         scalar: torch.Tensor | None, next_weight: torch.Tensor | None,
                         eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """g4_residual_norm_splitk: ``residual_norm`` whose branch is ``bf16(partials.sum(0))`` (added in
    split order); ``partials`` f32 ``[ksplit, rows, cols]``, residual bf16 ``[..., cols]``."""

    if partials.dtype != torch.float32 or partials.dim() != 3 or not partials.is_contiguous():
        raise ValueError("partials must be a contiguous f32 [ksplit, rows, cols] tensor")
    ks, rows, cols = partials.shape
    if residual.dtype != torch.bfloat16 or residual.numel() != rows * cols or not residual.is_contiguous():
        raise ValueError("residual must be a contiguous bf16 tensor of rows x cols elements")
    for w in (branch_weight, next_weight):
        if w is not None and (w.dtype != residual.dtype or w.numel() != cols or not w.is_contiguous()):
            raise ValueError("norm weights must be contiguous [cols] tensors in the activation dtype")
    if scalar is not None and (scalar.dtype != torch.float32 or scalar.numel() != 1):
        raise ValueError("scalar must be a one-element f32 tensor")
    x = torch.empty_like(residual)
    h = torch.empty_like(residual)
    _lib.check(_lib.lib().g4_residual_norm_splitk(rows, cols, _ptr(partials), ks, _ptr(branch_weight), _ptr(residual),
                                                  _ptr(scalar), _ptr(next_weight), eps, _ptr(x), _ptr(h), _stream()),
               "g4_residual_norm_splitk")
    return x, h


def convert_f32_to_bf16(x: torch.Tensor, *, nonfinite: torch.Tensor | None = None) -> torch.Tensor:
    """g4_convert_f32_to_bf16: the reference's bitwise round-to-nearest-even cast of an f32 tensor
    (any shape) to bf16. ``nonfinite`` (int32 [1] on the device) is set to 1 if an input is inf /
    NaN or a result overflows; it is not cleared."""

    if x.dtype != torch.float32:
        raise TypeError("convert_f32_to_bf16 takes a float32 tensor")
    src = x.contiguous()
    if src.data_ptr() % 16:
        src = src.clone()
    out = torch.empty(src.shape, dtype=torch.bfloat16, device=src.device)
    if nonfinite is not None and (nonfinite.dtype != torch.int32 or nonfinite.device != src.device):
        raise ValueError("nonfinite must be an int32 tensor on the input's device")
    _lib.check(_lib.lib().g4_convert_f32_to_bf16(_ptr(src), _ptr(out), src.numel(),
                                                 _ptr(nonfinite) if nonfinite is not None else None, _stream()),
               "g4_convert_f32_to_bf16")
    return out


def convert_bf16_to_f32(x: torch.Tensor) -> torch.Tensor:
    """g4_convert_bf16_to_f32: exact widening of a bf16 tensor (any shape) to float32."""

    if x.dtype != torch.bfloat16:
        raise TypeError("convert_bf16_to_f32 takes a bfloat16 tensor")
    src = x.contiguous()
    out = torch.empty(src.shape, dtype=torch.float32, device=src.device)
    _lib.check(_lib.lib().g4_convert_bf16_to_f32(_ptr(src), _ptr(out), src.numel(), _stream()),
               "g4_convert_bf16_to_f32")
    return out
