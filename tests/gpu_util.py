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


def k_slots(kt: np.ndarray) -> np.ndarray:
    """The operand-ordered key layout ``[B, H, C, D/32, 2, 16, 32]`` (numpy) -> slot-major
    ``[B, H, 32 C, D]``."""

    B, H, C, NR = kt.shape[:4]
    kr = kt.shape[6]
    return kt.reshape(B, H, C, NR, 2, 4, 4, kr).transpose(0, 1, 2, 5, 4, 6, 3, 7).reshape(B, H, C * 32, NR * kr)


def vt_slots(vt: np.ndarray) -> np.ndarray:
    """The grouped value layout ``[B, H, G, D, 8]`` (numpy) -> slot-major ``[B, H, 8 G, D]``."""

    B, H, G, D, _ = vt.shape
    return vt.transpose(0, 1, 2, 4, 3).reshape(B, H, G * 8, D)


def cache_to_ref(layer) -> tuple[np.ndarray, np.ndarray]:
    """Kernel layout (key [B,H,Cp,D], value_t [B,H,Cp/8,D,8]) -> the reference's [B,C,H,D] pair."""

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


def model_bars(dtype: str, got: np.ndarray, ref: np.ndarray, ref_f64acc: np.ndarray) -> tuple[float, float, float]:
    """Model-level logits bar: max-abs 2e-2 (bf16) / 1e-5 (fp32). Returns (error, bar, spread),
    spread = how far the oracle itself moves when its matmuls accumulate in f64 instead of f32 on
    the same inputs (reported next to the error, not added to the bar)."""

    err = float(np.abs(got - ref).max())
    spread = float(np.abs(ref - ref_f64acc).max())
    return err, TOL[dtype], spread


def attention_rows(got: np.ndarray, ref32: np.ndarray, ref64: np.ndarray, tol: float) -> tuple[float, int, int]:
    """Attention-output parity per row (one query and head: the last axis). A row passes when it
    lies within ``tol`` of the oracle with f32 accumulation or, failing that, of the oracle with
    f64 accumulation (the exactly rounded dot products): a score within f32 rounding of a bf16
    rounding boundary is rounded either way by valid f32 accumulation orders, the reference's XLA
    dot among them, and at scores of ~50 one such flip moves a probability by ~28 %. Returns the
    largest error against the f32 oracle, the number of rows that needed the f64 oracle, and the
    number of rows that match neither."""

    e32 = np.abs(got - ref32).max(axis=-1)
    e64 = np.abs(got - ref64).max(axis=-1)
    ok32 = e32 <= tol
    ok64 = e64 <= tol
    return float(e32.max()), int((~ok32 & ok64).sum()), int((~ok32 & ~ok64).sum())


def bf16_spacing(a: np.ndarray) -> np.ndarray:
    """One bf16 ulp at the magnitude of each element (2^(e - 7) for |a| in [2^e, 2^(e+1)))."""

    mag = np.abs(np.asarray(a, np.float32))
    return np.where(mag > 0, 2.0 ** (np.floor(np.log2(np.maximum(mag, 2.0 ** -126))) - 7), 2.0 ** -133)


def cache_elements(got: np.ndarray, want32: np.ndarray, want64: np.ndarray, tol: float) -> tuple[float, int, int]:
    """Per-element parity of a written cache against the oracle run on the same layer inputs: an
    element passes within ``tol`` of the oracle with f32 accumulation or, failing that, of the
    oracle with f64 accumulation (the exactly rounded projection; a GEMM output within f32
    rounding of a bf16 boundary is rounded either way by valid accumulation orders). Returns the
    largest error against the f32 oracle, the number of elements that needed the f64 oracle, and
    the number that match neither."""

    got = np.asarray(got, np.float32)
    e32 = np.abs(got - want32)
    e64 = np.abs(got - want64)
    ok32 = e32 <= tol
    ok64 = e64 <= tol
    return float(e32.max()), int((~ok32 & ok64).sum()), int((~ok32 & ~ok64).sum())


def ulp_stats(got: np.ndarray, want: np.ndarray, floor_frac: float = 0.125) -> tuple[float, float]:
    """(fraction of bit-equal elements, largest difference in bf16 ulps). An element's ulp is taken
    at its own magnitude, but not below ``floor_frac`` of the array's RMS: a value that results
    from cancellation (a projection output near zero, a rotation of two terms) carries the rounding
    error of its terms, not of itself."""

    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    floor = np.float32(np.sqrt(np.mean(np.square(want.astype(np.float64)))) * floor_frac)
    scale = np.maximum(np.abs(want), floor)
    return float((got == want).mean()), float((np.abs(got - want) / bf16_spacing(scale)).max())


def teacher_forced_layers(oparams, cfg, ids, position_ids, layer_inputs, *, kv_cache, attention_mask,
                          cache_mode: str, dtype: str = O.BF16):
    """The oracle's decoder layers (forward_text's loop, model.py:571-673) run on given inputs:
    layer i reads ``layer_inputs[i]`` (the device's own output of layer i - 1; the embedding for
    layer 0) instead of the oracle's previous layer. Returns (per-layer outputs, updated cache).
    Comparing layer by layer keeps a last-bit difference from one layer from compounding through
    the rest."""

    B, S = ids.shape
    attention_mask = attention_mask.astype(bool)
    key_mask = kv_cache.key_mask.copy()
    key_mask[:, kv_cache.length:kv_cache.length + S] = attention_mask
    if cache_mode == "append":
        masks = O.make_cached_qk_masks(key_mask, cfg.sliding_window, kv_cache.length, S)
    else:
        masks = O.make_qk_masks(attention_mask, cfg.sliding_window, 0, S)
    rots = O.make_rotary(cfg, position_ids)
    shared: dict = {}
    outs, layers = [], []
    for i, lp in enumerate(oparams.layers):
        x, nc = O.forward_decoder_layer(lp, layer_inputs[i], None, masks, rots, layer_index=i, cfg=cfg,
                                        shared_kv=shared, layer_cache=kv_cache.layers[i],
                                        cache_length=kv_cache.length, cache_mode=cache_mode, dtype=dtype)
        outs.append(x)
        layers.append(nc)
    return outs, O.KVCache(tuple(layers), key_mask, kv_cache.length + S)


def oracle_embed(oparams, cfg, ids, dtype: str = O.BF16) -> np.ndarray:
    """forward_text's scaled embedding (model.py:599-600)."""

    x = oparams.embed_tokens[ids]
    return O.cast(x * O.cast(np.float32(np.sqrt(cfg.hidden_size)), dtype), dtype)


def oracle_params(params) -> "O.Params":
    """Device parameters (model.Gemma4TextParams, torch) -> the oracle's float32 numpy pytree."""

    def a(t):
        return None if t is None else t.detach().float().cpu().numpy()

    def nw(p):
        return None if p is None else a(p.weight)

    layers = []
    for lp in params.layers:
        at = lp.attention
        ple = None
        if lp.per_layer_input is not None:
            pi = lp.per_layer_input
            ple = O.PLEParams(a(pi.gate), a(pi.projection), nw(pi.post_norm))
        layers.append(O.LayerParams(nw(lp.input_norm), O.AttnParams(a(at.q_proj), a(at.k_proj), a(at.v_proj),
                                                                    a(at.o_proj), nw(at.q_norm), nw(at.k_norm)),
                                    nw(lp.post_attention_norm), nw(lp.pre_feedforward_norm),
                                    O.MLPParams(a(lp.mlp.gate_proj), a(lp.mlp.up_proj), a(lp.mlp.down_proj)),
                                    nw(lp.post_feedforward_norm), ple, np.float32(lp.layer_scalar.float().item())))
    return O.Params(a(params.embed_tokens), a(params.embed_tokens_per_layer), a(params.per_layer_model_projection),
                    nw(params.per_layer_projection_norm), tuple(layers), nw(params.final_norm))


def oracle_cache_rows(cache, rows) -> "O.KVCache":
    """The device KVCache restricted to batch rows ``rows``, in the oracle's reference layout
    ([r, C, H, D] per layer, None for kv-shared layers), with its key mask and length."""

    idx = torch.as_tensor(list(rows), dtype=torch.long, device=cache.key_mask.device)
    layers = []
    for layer in cache.layers:
        if layer is None:
            layers.append(None)
            continue
        k = layer.key_slots().index_select(0, idx)[:, :, : layer.capacity].permute(0, 2, 1, 3)
        v = layer.value_dmajor().index_select(0, idx)[:, :, :, : layer.capacity].permute(0, 3, 1, 2)
        layers.append(O.LayerKV(to_np(k.contiguous()), to_np(v.contiguous())))
    km = cache.key_mask.index_select(0, idx).cpu().numpy().astype(bool)
    return O.KVCache(tuple(layers), km, int(cache.length))


def ref_to_cache(layer, k_ref: np.ndarray, v_ref: np.ndarray, dtype: str) -> None:
    """Write reference-layout [B,C,H,D] contents into a kernel-layout cache layer in place."""

    dev = layer.key.device
    k = to_dev(k_ref, dtype, dev).permute(0, 2, 1, 3)
    v = to_dev(v_ref, dtype, dev).permute(0, 2, 1, 3)
    layer.set_keys(k)
    layer.set_values(v)
