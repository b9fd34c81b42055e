"""Prefill, one-token decode and rollout generation: the drop-in for
gemma4_posttrain_jax/sampler.py on one MI355X.

Same functions, arguments and semantics as the reference (sampler.py:30-352): left-padded prompts
with logical RoPE positions, cache capacity ``P + N``, full-vocab f32 log-probabilities of the
unmodified policy, EOS masking with early exit, and JAX's random stream: ``PRNGKey(seed)``, one
``split`` per step, ``categorical`` = Gumbel-max over threefry2x32 noise in JAX's partitionable
layout (drawn on the device by g4_sample_tokens). Differences: arrays are torch device tensors, a
key is an int seed or the two uint32 words of ``jax.random.key_data``, and ``mesh`` must be None
(one GPU).
"""

from __future__ import annotations

import math
from typing import Any, NamedTuple, Protocol

import torch

from . import _lib, kernels
from .config import Gemma4TextConfig
from .kvcache import KVCache, init_kv_cache
from .model import Gemma4Output, Gemma4TextParams, _proj, checked_softcap, forward_gemma4_lm, forward_gemma4_text


class SamplerConfig(NamedTuple):
    """sampler.py:30-44: temperature <= 0 is greedy, top_k <= 0 and top_p == 1 disable truncation."""

    max_prompt_len: int
    max_new_tokens: int
    temperature: float = 1.0
    top_k: int = 0
    eos_ids: tuple[int, ...] = ()
    seed: int = 0
    top_p: float = 1.0


class RolloutBatch(NamedTuple):
    """sampler.py:47-52."""

    prompt_ids: torch.Tensor  # [B, P]
    completion_ids: torch.Tensor  # [B, N]
    completion_mask: torch.Tensor  # [B, N] bool; includes the first EOS
    rollout_logps: torch.Tensor  # [B, N] float32; zero outside completion_mask
    lengths: torch.Tensor  # [B] int32


class Rollout(Protocol):
    """sampler.py:55-60."""

    def generate(self, prompt_ids: torch.Tensor, prompt_mask: torch.Tensor, *, key=None) -> RolloutBatch: ...

    def update_params(self, params: Gemma4TextParams) -> None: ...


def _no_mesh(mesh) -> None:
    if mesh is not None:
        raise ValueError("mesh sharding is not supported: the native rollout path runs on one GPU")


def _position_ids(attention_mask: torch.Tensor) -> torch.Tensor:
    """sampler.py:63-67: ``max(cumsum(mask) - 1, 0)``."""

    return torch.clamp(torch.cumsum(attention_mask.to(torch.int32), dim=-1) - 1, min=0).to(torch.int32)


def prefill(
    params: Gemma4TextParams,
    config: Gemma4TextConfig,
    prompt_ids: torch.Tensor,
    prompt_mask: torch.Tensor,
    *,
    max_new_tokens: int,
    cache_dtype: Any | None = None,
    mesh=None,
    lora=None,
) -> Gemma4Output:
    """sampler.py:70-106: encode a left-padded prompt and populate the caches."""

    _no_mesh(mesh)
    if prompt_ids.dim() != 2 or tuple(prompt_mask.shape) != tuple(prompt_ids.shape):
        raise ValueError(
            f"prompt ids/mask must have the same [B, P] shape, got {tuple(prompt_ids.shape)}/{tuple(prompt_mask.shape)}")
    if max_new_tokens < 0:
        raise ValueError(f"max_new_tokens must be non-negative, got {max_new_tokens}")
    B, P = prompt_ids.shape
    dtype = params.embed_tokens.dtype if cache_dtype is None else cache_dtype
    cache = init_kv_cache(config, B, P + max_new_tokens, dtype, prompt_ids.device)
    return forward_gemma4_lm(params, prompt_ids, _position_ids(prompt_mask), config=config,
                             attention_mask=prompt_mask.to(torch.bool), kv_cache=cache, cache_mode="prefill",
                             logits_to_keep=1, lora=lora)


def decode_step(
    params: Gemma4TextParams,
    config: Gemma4TextConfig,
    token_ids: torch.Tensor,
    position_ids: torch.Tensor,
    kv_cache: KVCache,
    *,
    attention_mask: torch.Tensor | None = None,
    mesh=None,
    lora=None,
) -> Gemma4Output:
    """sampler.py:109-142: append one physical token slot per row and return next-token logits."""

    _no_mesh(mesh)
    if token_ids.dim() != 1 or tuple(position_ids.shape) != tuple(token_ids.shape):
        raise ValueError(
            f"token/position must have the same [B] shape, got {tuple(token_ids.shape)}/{tuple(position_ids.shape)}")
    if attention_mask is None:
        attention_mask = torch.ones_like(token_ids, dtype=torch.bool)
    return forward_gemma4_lm(params, token_ids[:, None], position_ids[:, None], config=config,
                             attention_mask=attention_mask[:, None], kv_cache=kv_cache, cache_mode="append",
                             logits_to_keep=1, lora=lora)


class GraphedDecodeStep:
    """One decode step (append forward + LM head, ``decode_step``'s work) captured in a HIP graph
    and replayed once per generated token.

    Inputs live in static device buffers (token ids, logical positions, the active mask) and the
    physical slot is an int32 device counter advanced inside the graph, so a replay launches the
    whole step (every layer's GEMMs, norms, cache append and decode attention, the LM head) with
    one call and no host work per layer. The cache is updated in place.

    With ``temperature`` given, the graph ends in the LM head with the sampler in its epilogue
    (``g4_lm_head_sample``; ``g4_sample_tokens`` after a separate LM head where the shapes are
    outside its limits): the LM head's soft-capping, the full-vocab log-softmax, the split of
    ``key`` (a 2-word int32 device tensor, advanced in place by every replay) and a greedy /
    categorical draw, and
    ``step_sample`` returns the next token and its log-probability; otherwise ``step`` returns the
    logits.

    Capture runs the step once eagerly first (library handles, packed weights); that warm-up
    writes the cache slot ``cache.length``, which the first replay then overwrites.
    """

    def __init__(self, params: Gemma4TextParams, config: Gemma4TextConfig, cache: KVCache, *,
                 temperature: float | None = None, key: torch.Tensor | None = None, top_k: int = 0,
                 top_p: float = 1.0) -> None:
        dev = cache.key_mask.device
        B = cache.key_mask.shape[0]
        self.params, self.config, self.cache = params, config, cache
        self.length = int(cache.length)
        self.tok = torch.zeros(B, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(B, dtype=torch.int32, device=dev)
        self.active = torch.ones(B, dtype=torch.bool, device=dev)
        self.slot = torch.full((B,), self.length, dtype=torch.int32, device=dev)
        if temperature is not None and temperature > 0 and key is None:
            raise ValueError("sampling in the graph needs the device key")
        self.temperature, self.key = temperature, key
        self.top_k, self.top_p = top_k, top_p
        if top_k and not _native_top_k(temperature or 0.0, top_k, top_p, config.vocab_size):
            raise ValueError(f"top_k={top_k} is not a native in-graph draw (0 < top_k <= {kernels.TOP_K_MAX}, T > 0)")
        self.token_out = torch.zeros(B, dtype=torch.int32, device=dev)
        self.logp_out = torch.zeros(B, dtype=torch.float32, device=dev)
        saved_key = None if key is None else key.clone()
        _lib.init_device(dev.index if dev.index is not None else torch.cuda.current_device())
        self._forward()  # eager warm-up: its key split is undone below
        if key is not None:
            key.copy_(saved_key)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side), torch.cuda.graph(self.graph, stream=side):
            self.logits = self._forward()
            self.slot.add_(1)
        torch.cuda.current_stream(dev).wait_stream(side)

    def _forward(self) -> torch.Tensor | None:
        if self.temperature is None:
            out = forward_gemma4_lm(self.params, self.tok[:, None], self.pos[:, None], config=self.config,
                                    attention_mask=self.active[:, None], kv_cache=self.cache, cache_mode="append",
                                    logits_to_keep=1, write_pos=self.slot)
            return out.logits[:, -1].float()
        hidden, _ = forward_gemma4_text(self.params, self.tok[:, None], self.pos[:, None], config=self.config,
                                        attention_mask=self.active[:, None], kv_cache=self.cache,
                                        cache_mode="append", write_pos=self.slot)
        head_in = hidden[:, -1]
        cap = checked_softcap(self.config.final_logit_softcapping)
        if self.top_k:
            # top-k (+ top-p) draw over the raw LM head logits (the kernel applies the soft-cap)
            if kernels.lm_head_supported(head_in, self.params.embed_tokens):
                raw = kernels.lm_head(head_in.contiguous(), self.params.embed_tokens)
            else:
                raw = _proj(head_in, self.params.embed_tokens)
            kernels.sample_top_k(raw, softcap=cap, temperature=self.temperature, top_k=self.top_k, top_p=self.top_p,
                                 key=self.key, split_key=True, token_out=self.token_out, logp_out=self.logp_out)
            return None
        if kernels.lm_head_supported(head_in, self.params.embed_tokens):
            # the LM head with the draw in its epilogue: the [B, V] logits never reach HBM
            kernels.lm_head_sample(head_in, self.params.embed_tokens, softcap=cap, temperature=self.temperature,
                                   key=self.key, split_key=True, token_out=self.token_out, logp_out=self.logp_out)
            return None
        raw = _proj(head_in, self.params.embed_tokens)  # [B, V] before the soft-cap
        kernels.sample_tokens(raw, softcap=cap, temperature=self.temperature, key=self.key, split_key=True,
                              token_out=self.token_out, logp_out=self.logp_out)
        return None

    def _replay(self, token_ids: torch.Tensor, position_ids: torch.Tensor, active: torch.Tensor) -> None:
        self.tok.copy_(token_ids)
        self.pos.copy_(position_ids)
        self.active.copy_(active)
        self.graph.replay()
        self.length += 1

    def step(self, token_ids: torch.Tensor, position_ids: torch.Tensor, active: torch.Tensor) -> torch.Tensor:
        """Append ``token_ids`` at the next slot; returns next-token logits ``[B, V]`` f32 (a static
        buffer, valid until the next call)."""

        if self.temperature is not None:
            raise RuntimeError("this step was captured with fused sampling: use step_sample")
        self._replay(token_ids, position_ids, active)
        return self.logits

    def step_sample(self, token_ids: torch.Tensor, position_ids: torch.Tensor,
                    active: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Append ``token_ids`` and draw the next token: ``(token int32 [B], logp f32 [B])`` (static
        buffers, valid until the next call)."""

        if self.temperature is None:
            raise RuntimeError("this step was captured without sampling: use step")
        self._replay(token_ids, position_ids, active)
        return self.token_out, self.logp_out

    def replay_sample(self) -> tuple[torch.Tensor, torch.Tensor]:
        """``step_sample`` on the inputs already in ``tok`` / ``pos`` / ``active`` (written there by
        the caller's own kernels, e.g. ``g4_rollout_step``)."""

        if self.temperature is None:
            raise RuntimeError("this step was captured without sampling: use replay_logits")
        self.graph.replay()
        self.length += 1
        return self.token_out, self.logp_out

    def replay_logits(self) -> torch.Tensor:
        """``step`` on the inputs already in ``tok`` / ``pos`` / ``active``."""

        if self.temperature is not None:
            raise RuntimeError("this step was captured with fused sampling: use replay_sample")
        self.graph.replay()
        self.length += 1
        return self.logits

    @property
    def kv_cache(self) -> KVCache:
        return self.cache._replace(length=self.length)


# Steps the generation loop may run ahead of the device's any-active flag when EOS ids are set.
EOS_LAG = 4


def _fused_sampling(sc: SamplerConfig, vocab: int) -> bool:
    """Greedy, or no top-k / top-p truncation (the RL configuration): the draw runs over the whole
    row, so it can end the captured decode graph (greedy ignores top-k / top-p, sampler.py:160-161)."""

    return sc.temperature <= 0 or ((sc.top_k <= 0 or sc.top_k >= vocab) and sc.top_p >= 1.0)


def _native_top_k(temperature: float, top_k: int, top_p: float, vocab: int) -> bool:
    """A top-k draw (with or without top-p) that g4_sample_top_k runs on the device: T > 0 and
    0 < top_k <= kernels.TOP_K_MAX below the vocabulary. top-p without top-k (a sort of the whole
    row) stays a host-built proposal."""

    return temperature > 0 and 0 < top_k < vocab and top_k <= kernels.TOP_K_MAX and 0 < top_p <= 1


def _key_words(key, seed: int) -> list[int]:
    """The two uint32 words of a JAX threefry key: ``PRNGKey(seed)`` for None, ``PRNGKey(key)`` for
    an int, else ``key`` itself (``jax.random.key_data``: a sequence, array or tensor of 2 words)."""

    if key is None:
        key = seed
    if isinstance(key, int):
        return [(key >> 32) & 0xFFFFFFFF, key & 0xFFFFFFFF]
    words = [int(w) & 0xFFFFFFFF for w in (key.tolist() if hasattr(key, "tolist") else key)]
    if len(words) != 2:
        raise ValueError(f"a key has two uint32 words, got {len(words)}")
    return words


def key_tensor(key, device: torch.device, seed: int = 0) -> torch.Tensor:
    """A fresh 2-word int32 device tensor holding the key (the native sampler's key format)."""

    return torch.tensor(_key_words(key, seed), dtype=torch.int64).to(torch.int32).to(device)


def _proposal(logits32: torch.Tensor, temperature: float, top_k: int,
              top_p: float) -> tuple[torch.Tensor | None, torch.Tensor | None]:
    """sampler.py:162-178: the truncated proposal the categorical draw runs over, as ``(scores
    [B, K] f32, vocab ids [B, K])``, or ``(None, None)`` without truncation. Ties keep the lower
    vocab id first (lax.top_k and the stable descending argsort do)."""

    V = logits32.shape[-1]
    if not (0 < top_k < V) and top_p >= 1:
        return None, None
    scores, indices = torch.sort(logits32 / temperature, dim=-1, descending=True, stable=True)
    if 0 < top_k < V:
        scores, indices = scores[:, :top_k], indices[:, :top_k]
    if top_p < 1:
        w = torch.exp(scores - scores.max(dim=-1, keepdim=True).values)
        probs = w / w.sum(dim=-1, keepdim=True)
        # mass before each column: 0 followed by the cumulative sum without its last entry, as
        # sampler.py:172-174 forms it (cumsum - probs can round one ulp lower at the boundary)
        previous = torch.cat([torch.zeros_like(probs[:, :1]), torch.cumsum(probs, dim=-1)[:, :-1]], dim=-1)
        keep = (previous < top_p) | (torch.arange(scores.shape[-1], device=scores.device)[None, :] == 0)
        scores = torch.where(keep, scores, torch.full_like(scores, -math.inf))
    return scores.contiguous(), indices.to(torch.int32).contiguous()


def _draw(logits: torch.Tensor, key: torch.Tensor, *, temperature: float, top_k: int, top_p: float,
          split_key: bool) -> tuple[torch.Tensor, torch.Tensor]:
    if logits.is_cuda and _native_top_k(temperature, top_k, top_p, logits.shape[-1]):
        x = logits if logits.dtype in (torch.bfloat16, torch.float32) and logits.stride(-1) == 1 else logits.float()
        return kernels.sample_top_k(x, softcap=None, temperature=temperature, top_k=top_k, top_p=top_p, key=key,
                                    split_key=split_key)
    logits32 = logits.float().contiguous()
    proposal, index = (None, None) if temperature <= 0 else _proposal(logits32, temperature, top_k, top_p)
    return kernels.sample_tokens(logits32, softcap=None, temperature=temperature, key=key, split_key=split_key,
                                 proposal=proposal, proposal_index=index)


def _sample_token(logits: torch.Tensor, key, *, temperature: float, top_k: int,
                  top_p: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    """sampler.py:145-183: sample from the configured proposal (temperature, then top-k, then
    top-p) with ``jax.random.categorical(key, ...)``, score under the full unmodified f32 policy.
    ``key`` is the sample key itself (not split here)."""

    k = key if isinstance(key, torch.Tensor) and key.dtype == torch.int32 else key_tensor(key, logits.device)
    return _draw(logits, k.to(logits.device), temperature=temperature, top_k=top_k, top_p=top_p, split_key=False)


def generate(
    params: Gemma4TextParams,
    config: Gemma4TextConfig,
    prompt_ids: torch.Tensor,
    prompt_mask: torch.Tensor,
    *,
    sampler_config: SamplerConfig,
    key=None,
    mesh=None,
    lora=None,
) -> RolloutBatch:
    """sampler.py:204-322: prefill, then up to ``max_new_tokens`` sample + append steps, stopping
    once every row has emitted an EOS id. Inactive rows emit pad with logp 0; the decode on the
    final step is skipped, so the cache never overflows."""

    _no_mesh(mesh)
    sc = sampler_config
    if prompt_ids.shape[1] != sc.max_prompt_len:
        raise ValueError(f"prompt width {prompt_ids.shape[1]} does not match max_prompt_len={sc.max_prompt_len}")
    if sc.max_prompt_len <= 0 or sc.max_new_tokens <= 0:
        raise ValueError("max_prompt_len and max_new_tokens must both be positive")
    if sc.top_k > config.vocab_size:
        raise ValueError(f"top_k={sc.top_k} exceeds vocab_size={config.vocab_size}")
    if not math.isfinite(sc.temperature):
        raise ValueError("temperature must be finite")
    if not math.isfinite(sc.top_p) or not 0 < sc.top_p <= 1:
        raise ValueError("top_p must be finite and in (0, 1]")
    checked_softcap(config.final_logit_softcapping)

    prompt_mask = prompt_mask.to(torch.bool)
    out = prefill(params, config, prompt_ids, prompt_mask, max_new_tokens=sc.max_new_tokens, mesh=mesh, lora=lora)
    dev = prompt_ids.device
    B, N = prompt_ids.shape[0], sc.max_new_tokens
    key_state = key_tensor(key, dev, sc.seed)  # the loop's key, split once per step on the device
    prompt_lengths = prompt_mask.sum(dim=-1, dtype=torch.int32)
    active = torch.ones(B, dtype=torch.bool, device=dev)
    ids_dtype = prompt_ids.dtype if prompt_ids.dtype in (torch.int32, torch.int64) else torch.int64
    completion_ids = torch.full((B, N), config.pad_token_id, dtype=ids_dtype, device=dev)
    completion_mask = torch.zeros((B, N), dtype=torch.bool, device=dev)
    rollout_logps = torch.zeros((B, N), dtype=torch.float32, device=dev)
    # token ids are int32, so an EOS id outside that range never matches
    eos = torch.tensor([e for e in sc.eos_ids if -2**31 <= e < 2**31], dtype=torch.int32, device=dev)
    any_dev = torch.ones(1, dtype=torch.bool, device=dev)
    logits = out.logits[:, -1].float()
    cache = out.kv_cache
    fused = _fused_sampling(sc, config.vocab_size)
    top_k = sc.top_k if _native_top_k(sc.temperature, sc.top_k, sc.top_p, config.vocab_size) else 0
    if fused or top_k:
        # first token from the prefill logits (already soft-capped), then one graph per step that
        # ends in the draw (the fused LM head sampler, or the LM head and the native top-k draw)
        nxt = _draw(out.logits[:, -1], key_state, temperature=sc.temperature, top_k=top_k, top_p=sc.top_p,
                    split_key=True) if top_k else kernels.sample_tokens(
                        out.logits[:, -1], softcap=None, temperature=sc.temperature, key=key_state)
        graphed = GraphedDecodeStep(params, config, cache, temperature=sc.temperature, key=key_state, top_k=top_k,
                                    top_p=sc.top_p) if N > 1 else None
        fused = True
    else:
        graphed = GraphedDecodeStep(params, config, cache) if N > 1 else None
    # With EOS ids the loop stops once no row is active (while_loop's cond, sampler.py:267-320).
    # The device's any-active flag of each step is copied to pinned host memory behind the step's
    # work, and the host reads the flag of EOS_LAG - 1 steps earlier, waiting only when it runs that
    # far ahead of the device: the device always has queued steps, and the loop may run up to
    # EOS_LAG - 1 steps past the last active one. Those steps change no output: every row is
    # inactive, so g4_rollout_step writes pad / False / 0 into columns that already hold them, and
    # the extra appends land in cache slots that generate never returns.
    watch = eos.numel() > 0
    if watch:
        flags = torch.ones(EOS_LAG, dtype=torch.bool, pin_memory=True)
        events = [torch.cuda.Event() for _ in range(EOS_LAG)]
    step = 0
    while step < N:
        if fused:
            sampled, logp = nxt
        else:
            sampled, logp = _draw(logits, key_state, temperature=sc.temperature, top_k=sc.top_k, top_p=sc.top_p,
                                  split_key=True)
        decode_next = step + 1 < N
        # the masked token / logp into column `step`, the EOS update of `active` and the next decode
        # step's inputs (the token, prompt_lengths + step, this step's mask) written straight into
        # the graph's input buffers
        kernels.rollout_step(step, sampled, logp, active, completion_ids=completion_ids,
                             completion_mask=completion_mask, rollout_logps=rollout_logps,
                             pad_id=config.pad_token_id, eos_ids=eos, prompt_lengths=prompt_lengths,
                             next_token=graphed.tok if decode_next else None,
                             next_pos=graphed.pos if decode_next else None,
                             next_mask=graphed.active if decode_next else None,
                             any_active=any_dev if eos.numel() else None)
        if watch:
            flags[step % EOS_LAG: step % EOS_LAG + 1].copy_(any_dev, non_blocking=True)
            events[step % EOS_LAG].record()
        if decode_next:
            if fused:
                nxt = graphed.replay_sample()
            else:
                logits = graphed.replay_logits()
        step += 1
        if watch and step >= EOS_LAG:
            seen = step % EOS_LAG  # the flag written after step (step - 1) - (EOS_LAG - 1)
            events[seen].synchronize()
            if not bool(flags[seen]):
                break
    lengths = completion_mask.sum(dim=-1, dtype=torch.int32)
    return RolloutBatch(prompt_ids, completion_ids.to(prompt_ids.dtype), completion_mask, rollout_logps, lengths)


class NativeRollout:
    """sampler.py:325-352 (``PureJaxRollout``): host-side parameter holder around ``generate``."""

    def __init__(self, params: Gemma4TextParams, model_config: Gemma4TextConfig, sampler_config: SamplerConfig,
                 mesh=None) -> None:
        _no_mesh(mesh)
        self.params = params
        self.model_config = model_config
        self.sampler_config = sampler_config
        self.mesh = mesh

    def update_params(self, params: Gemma4TextParams) -> None:
        self.params = params

    def generate(self, prompt_ids: torch.Tensor, prompt_mask: torch.Tensor, *, key=None) -> RolloutBatch:
        return generate(self.params, self.model_config, prompt_ids, prompt_mask, sampler_config=self.sampler_config,
                        key=key, mesh=self.mesh)


PureJaxRollout = NativeRollout  # the reference's class name, for drop-in callers
