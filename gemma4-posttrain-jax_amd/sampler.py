"""Prefill, one-token decode and rollout generation: the drop-in for
gemma4_posttrain_jax/sampler.py on one MI355X.

Same functions, arguments and semantics as the reference (sampler.py:30-352): left-padded prompts
with logical RoPE positions, cache capacity ``P + N``, full-vocab f32 log-probabilities of the
unmodified policy, EOS masking with early exit. Differences: arrays are torch device tensors, and
``key`` is an integer seed or a ``torch.Generator`` (the categorical draw is Gumbel-max over
Philox noise rather than JAX's threefry stream). ``mesh`` must be None (one GPU).
"""

from __future__ import annotations

import math
from typing import Any, NamedTuple, Protocol

import torch

from . import kernels
from .config import Gemma4TextConfig
from .kvcache import KVCache, init_kv_cache
from .model import Gemma4Output, Gemma4TextParams, forward_gemma4_lm, forward_gemma4_text


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

    With ``temperature`` given, the graph ends in the fused sampler (``g4_sample_tokens``: the LM
    head's soft-capping, the full-vocab log-softmax and a greedy / Gumbel-max draw, Philox noise
    keyed by ``seed`` and a device step counter starting at ``first_rng_step``) and ``step_sample``
    returns the next token and its log-probability; otherwise ``step`` returns the logits.

    Capture runs the step once eagerly first (library handles, packed weights); that warm-up
    writes the cache slot ``cache.length``, which the first replay then overwrites.
    """

    def __init__(self, params: Gemma4TextParams, config: Gemma4TextConfig, cache: KVCache, *,
                 temperature: float | None = None, seed: int = 0, first_rng_step: int = 1) -> None:
        dev = cache.key_mask.device
        B = cache.key_mask.shape[0]
        self.params, self.config, self.cache = params, config, cache
        self.length = int(cache.length)
        self.tok = torch.zeros(B, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(B, dtype=torch.int32, device=dev)
        self.active = torch.ones(B, dtype=torch.bool, device=dev)
        self.slot = torch.full((B,), self.length, dtype=torch.int32, device=dev)
        self.temperature, self.seed = temperature, seed
        self.rng_step = torch.full((1,), first_rng_step, dtype=torch.int32, device=dev)
        self.token_out = torch.zeros(B, dtype=torch.int32, device=dev)
        self.logp_out = torch.zeros(B, dtype=torch.float32, device=dev)
        self._forward()
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side), torch.cuda.graph(self.graph, stream=side):
            self.logits = self._forward()
            self.slot.add_(1)
            if temperature is not None:
                self.rng_step.add_(1)
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
        raw = hidden[:, -1] @ self.params.embed_tokens.t()  # [B, V] before the soft-cap
        kernels.sample_tokens(raw, softcap=self.config.final_logit_softcapping, temperature=self.temperature,
                              seed=self.seed, step=self.rng_step, token_out=self.token_out, logp_out=self.logp_out)
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

    @property
    def kv_cache(self) -> KVCache:
        return self.cache._replace(length=self.length)


def _fused_sampling(sc: SamplerConfig, vocab: int, device: torch.device) -> bool:
    """The native sampler covers the RL configuration: no top-k / top-p truncation."""

    return device.type == "cuda" and (sc.top_k <= 0 or sc.top_k >= vocab) and sc.top_p >= 1.0


def _seed_from_key(key, seed: int) -> int:
    """64-bit Philox key of the native sampler: the integer ``key`` (or ``seed`` when None), or a
    draw from a ``torch.Generator`` key (one host read)."""

    if isinstance(key, torch.Generator):
        return int(torch.randint(0, 2 ** 62, (1,), generator=key, device=key.device).item())
    return int(seed if key is None else key)


def _generator(key, device, seed: int) -> torch.Generator:
    if isinstance(key, torch.Generator):
        return key
    g = torch.Generator(device=device)
    g.manual_seed(int(seed if key is None else key))
    return g


def _sample_token(logits: torch.Tensor, generator: torch.Generator, *, temperature: float, top_k: int,
                  top_p: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    """sampler.py:145-183: sample from the configured proposal (temperature, then top-k, then
    top-p), score under the full unmodified f32 policy."""

    logits32 = logits.float()
    full_logps = torch.log_softmax(logits32, dim=-1)
    V = logits32.shape[-1]
    if temperature <= 0:
        token = torch.argmax(logits32, dim=-1).to(torch.int32)
    else:
        scores = logits32 / temperature
        indices = None
        if 0 < top_k < V:
            scores, indices = torch.topk(scores, top_k, dim=-1)
        elif top_p < 1:
            scores, indices = torch.sort(scores, dim=-1, descending=True, stable=True)
        if top_p < 1:
            w = torch.exp(scores - scores.max(dim=-1, keepdim=True).values)
            probs = w / w.sum(dim=-1, keepdim=True)
            previous = torch.cumsum(probs, dim=-1) - probs
            keep = (previous < top_p) | (torch.arange(scores.shape[-1], device=scores.device)[None, :] == 0)
            scores = torch.where(keep, scores, torch.full_like(scores, -math.inf))
        u = torch.rand(scores.shape, generator=generator, device=scores.device, dtype=torch.float32)
        gumbel = -torch.log(-torch.log(u))
        selected = torch.argmax(scores + gumbel, dim=-1)
        token = (selected if indices is None else torch.gather(indices, 1, selected[:, None])[:, 0]).to(torch.int32)
    logp = torch.gather(full_logps, 1, token[:, None].long())[:, 0]
    return token, logp


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

    prompt_mask = prompt_mask.to(torch.bool)
    out = prefill(params, config, prompt_ids, prompt_mask, max_new_tokens=sc.max_new_tokens, mesh=mesh, lora=lora)
    dev = prompt_ids.device
    B, N = prompt_ids.shape[0], sc.max_new_tokens
    gen = _generator(key, dev, sc.seed)
    prompt_lengths = prompt_mask.sum(dim=-1, dtype=torch.int32)
    active = torch.ones(B, dtype=torch.bool, device=dev)
    completion_ids = torch.full((B, N), config.pad_token_id, dtype=prompt_ids.dtype, device=dev)
    completion_mask = torch.zeros((B, N), dtype=torch.bool, device=dev)
    rollout_logps = torch.zeros((B, N), dtype=torch.float32, device=dev)
    eos = torch.tensor(list(sc.eos_ids), dtype=torch.int64, device=dev)
    logits = out.logits[:, -1].float()
    cache = out.kv_cache
    fused = _fused_sampling(sc, config.vocab_size, dev)
    if fused:  # first token from the prefill logits (already soft-capped), then one graph per step
        seed = _seed_from_key(key, sc.seed)
        nxt = kernels.sample_tokens(out.logits[:, -1], softcap=None, temperature=sc.temperature, seed=seed, step=0)
        graphed = GraphedDecodeStep(params, config, cache, temperature=sc.temperature, seed=seed,
                                    first_rng_step=1) if N > 1 else None
    else:
        graphed = GraphedDecodeStep(params, config, cache) if dev.type == "cuda" and N > 1 else None
    step = 0
    while step < N:
        if fused:
            sampled, logp = nxt
        else:
            sampled, logp = _sample_token(logits, gen, temperature=sc.temperature, top_k=sc.top_k, top_p=sc.top_p)
        token = torch.where(active, sampled, torch.full_like(sampled, config.pad_token_id)).to(prompt_ids.dtype)
        logp = torch.where(active, logp, torch.zeros_like(logp))
        completion_ids[:, step] = token
        completion_mask[:, step] = active
        rollout_logps[:, step] = logp
        next_active = active & ~torch.isin(token.long(), eos) if len(sc.eos_ids) else active
        any_active = bool(next_active.any())  # the only host sync per step (while_loop's cond)
        if step + 1 < N and any_active:
            pos = (prompt_lengths + step).to(torch.int32)
            if fused:
                nxt = graphed.step_sample(token.to(torch.int32), pos, active)
            elif graphed is not None:
                logits = graphed.step(token.to(torch.int32), pos, active)
            else:
                dec = decode_step(params, config, token.to(torch.int32), pos, cache, attention_mask=active,
                                  lora=lora)
                logits = dec.logits[:, -1].float()
                cache = dec.kv_cache
        active = next_active
        step += 1
        if not any_active:
            break
    lengths = completion_mask.sum(dim=-1, dtype=torch.int32)
    return RolloutBatch(prompt_ids, completion_ids, completion_mask, rollout_logps, lengths)


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
