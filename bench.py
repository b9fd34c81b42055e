"""Benchmark of the Gemma 4 rollout decode hot path on one MI355X.

Headline (BASELINE.json ``configs[1]``): sliding-window decode attention, B=64, Hq=8/Hkv=2,
D=256, W=512 bf16 ring already holding 2048 tokens (per-row write positions U[1536, 2048)); a
step appends one token per row and attends (one launch of the fused append + decode kernel).
``value`` = algorithmic bytes per step / time per step, in GB/s. Steps are replayed from a HIP
graph so the timed region holds only GPU work.

Also reported: ``decode_tok_s_b256`` — full decode steps (30-layer E2B-like model, B=256, T=1
sampling, BASELINE ``configs[4]``) per second x 256, averaged over every step of a 512-token
rollout; ``rollout_tok_s_b256`` — 256 x 512 tokens over prefill + all decode steps (the reference
harness's slot tokens/s); and the oracle's CPU time for the same step.

Also: ``long_context_decode`` (``configs[2]``, split-K decode over a 32768-slot linear cache,
HBM-bound), ``e2b_decode_attention`` (one sliding layer's decode attention at the ``configs[4]``
batch of 256) and ``prefill_attention`` (``configs[3]``, causal / sliding attention on MFMA).

Usage: ``python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-e2b] [--no-cpu] [--no-extra]``.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

# configs[1]
B, HQ, HKV, D, W = 64, 8, 2, 256, 512
R = HQ // HKV
CTX = 2048
NCACHE = 8


def algorithmic_bytes_per_step() -> int:
    """K+V of every valid slot once, Q in, O out, the new token's K/V read and written."""

    kv = B * HKV * W * D * 2 * 2
    q = B * HQ * D * 2
    o = B * HQ * D * 2
    new_kv = B * HKV * D * 2 * 2 * 2
    return kv + q + o + new_kv


def measured_traffic() -> int | None:
    """HBM bytes per launch of the config-2 decode kernel from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the counter's reading on a copy of known
    size); None when the summary is absent."""

    path = ROOT / "profiles" / "decode_attention_config2_traffic.json"
    try:
        return int(json.loads(path.read_text())["hbm_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def prefill_counters() -> dict | None:
    """Counter-based MFMA figures of the config-4 prefill kernel from the committed rocprofv3 --pmc
    summary (MFMA busy fraction, executed bf16 TFLOP per layer); None when it is absent."""

    path = ROOT / "profiles" / "prefill_attention_config4_mfma.json"
    try:
        return json.loads(path.read_text())
    except (OSError, ValueError):
        return None


def cpu_info() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def bench_decode_attention(steps: int, warmup: int, num_splits: int = 0) -> dict:
    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from gemma4_posttrain_jax_amd import kernels
    from gemma4_posttrain_jax_amd.kvcache import new_layer_cache

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    # NCACHE independent config-2 ring caches (64 MiB each), used round-robin: a step reads a
    # cache last touched NCACHE steps earlier, so the 256 MB Infinity Cache cannot serve it from a
    # previous step -- as in the full model, where ~12 GB of other layers' KV and weights stream
    # between two visits of one layer's cache.
    layers = []
    for _ in range(NCACHE):
        layer = new_layer_cache(B, HKV, D, W, True, torch.bfloat16, dev)
        layer.key.normal_(generator=g)
        layer.value_t.normal_(generator=g)
        layers.append(layer)
    rng = np.random.default_rng(0)
    pos0 = rng.integers(1536, 2048, B).astype(np.int32)
    total = warmup + steps
    # per-step query positions, new K/V rows, queries and outputs (separate buffers per step so
    # the graph replays exactly the K distinct steps)
    q_pos = torch.from_numpy(pos0[None, :] + np.arange(total, dtype=np.int32)[:, None]).to(dev).contiguous()
    key_mask = torch.ones((B, CTX + total + 64), dtype=torch.bool, device=dev)
    q = torch.randn((total, B, HKV, R, D), device=dev, generator=g).to(torch.bfloat16)
    nk = torch.randn((total, B, HKV, D), device=dev, generator=g).to(torch.bfloat16)
    nv = torch.randn((total, B, HKV, D), device=dev, generator=g).to(torch.bfloat16)
    out = torch.empty((total, B, HKV, R, D), device=dev, dtype=torch.bfloat16)

    def step(i):
        kernels.decode_attention(layers[i % NCACHE], q[i], key_mask, q_pos=q_pos[i], window=W, out=out[i],
                                 new_k=nk[i], new_v=nv[i], num_splits=num_splits)

    # eager warmup (also compiles nothing: the library is prebuilt)
    for i in range(min(total, 3)):
        step(i)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g_warm, g_timed = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g_warm, stream=s):
            for i in range(warmup):
                step(i)
        with torch.cuda.graph(g_timed, stream=s):
            for i in range(warmup, total):
                step(i)
    torch.cuda.synchronize()
    if warmup:
        g_warm.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    g_timed.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    # second replay, eager launches, for reference (host launch overhead included)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(warmup, total):
        step(i)
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3
    return {"ms_total": ms, "ms_per_step": ms / steps, "eager_ms_per_step": eager_ms / steps}


def _graph_time(step, n_warm: int, n_timed: int) -> float:
    """ms per step of `step(i)` replayed from a HIP graph (steps n_warm .. n_warm + n_timed - 1)."""

    import torch

    for i in range(min(n_warm, 2)):
        step(i)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    gw, gt = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(gw, stream=s):
            for i in range(n_warm):
                step(i)
        with torch.cuda.graph(gt, stream=s):
            for i in range(n_warm, n_warm + n_timed):
                step(i)
    torch.cuda.synchronize()
    gw.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    gt.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n_timed


def bench_long_context_decode(steps: int = 16, warmup: int = 150) -> dict:
    """global-layer decode over a linear cache, B=16, Hq=8/Hkv=2, D=256,
    capacity 32768, per-row lengths U[1024, 32768] growing by one per step (split-K path).
    Algorithmic bytes: K+V of every valid slot once, Q in, O out, the new K/V row. The `warmup`
    graphed steps (~16 ms) bring the GPU to its sustained clock first."""

    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from gemma4_posttrain_jax_amd import kernels
    from gemma4_posttrain_jax_amd.kvcache import new_layer_cache

    Bq, C = 16, 32768
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(3)
    layer = new_layer_cache(Bq, HKV, D, C, False, torch.bfloat16, dev)
    layer.key.normal_(generator=g)
    layer.value_t.normal_(generator=g)
    rng = np.random.default_rng(0)
    total = warmup + steps
    len0 = rng.integers(1024, C - total, Bq).astype(np.int32)
    q_pos = torch.from_numpy(len0[None, :] + np.arange(total, dtype=np.int32)[:, None]).to(dev).contiguous()
    key_mask = torch.ones((Bq, C), dtype=torch.bool, device=dev)
    q = torch.randn((total, Bq, HKV, R, D), device=dev, generator=g).to(torch.bfloat16)
    nk = torch.randn((total, Bq, HKV, D), device=dev, generator=g).to(torch.bfloat16)
    nv = torch.randn((total, Bq, HKV, D), device=dev, generator=g).to(torch.bfloat16)
    out = torch.empty((total, Bq, HKV, R, D), device=dev, dtype=torch.bfloat16)

    def step(i):
        kernels.decode_attention(layer, q[i], key_mask, q_pos=q_pos[i], window=0, out=out[i], new_k=nk[i],
                                 new_v=nv[i])

    ms = _graph_time(step, warmup, steps)
    lens = len0[None, :] + np.arange(warmup, total)[:, None] + 1  # valid slots incl. the appended one
    kv_bytes = float(lens.sum(axis=1).mean()) * HKV * D * 2 * 2
    small = Bq * HQ * D * 2 * 2 + Bq * HKV * D * 2 * 2 * 2
    gbs = (kv_bytes + small) / (ms * 1e-3) / 1e9
    return {"ms_per_step": ms, "gbs": gbs, "bytes_per_step": kv_bytes + small}


def bench_e2b_decode_attention(steps: int = 64, warmup: int = 300, batch: int = 256) -> dict:
    """The decode attention of one sliding layer of the configs[4] model at its rollout batch: B=256,
    Hq=8/Hkv=2, D=256, a full 512-slot ring (positions U[1536, 2048), as configs[1]), one token
    appended and attended per step (the library's automatic choice: the two-launch path). NCACHE
    rotating 256 MiB caches as in the headline; `warmup` graphed steps (~15 ms) first. Algorithmic
    bytes as the headline's: K+V of every valid slot once, Q in, O out, the new K/V row read and
    written."""

    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from gemma4_posttrain_jax_amd import kernels
    from gemma4_posttrain_jax_amd.kvcache import new_layer_cache

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(5)
    layers = []
    for _ in range(NCACHE):
        layer = new_layer_cache(batch, HKV, D, W, True, torch.bfloat16, dev)
        layer.key.normal_(generator=g)
        layer.value_t.normal_(generator=g)
        layers.append(layer)
    rng = np.random.default_rng(5)
    pos0 = rng.integers(1536, 2048, batch).astype(np.int32)
    total = warmup + steps
    q_pos = torch.from_numpy(pos0[None, :] + np.arange(total, dtype=np.int32)[:, None]).to(dev).contiguous()
    key_mask = torch.ones((batch, CTX + total + 64), dtype=torch.bool, device=dev)
    q = torch.randn((total, batch, HKV, R, D), device=dev, generator=g).to(torch.bfloat16)
    nk = torch.randn((total, batch, HKV, D), device=dev, generator=g).to(torch.bfloat16)
    nv = torch.randn((total, batch, HKV, D), device=dev, generator=g).to(torch.bfloat16)
    out = torch.empty((total, batch, HKV, R, D), device=dev, dtype=torch.bfloat16)

    def step(i):
        kernels.decode_attention(layers[i % NCACHE], q[i], key_mask, q_pos=q_pos[i], window=W, out=out[i],
                                 new_k=nk[i], new_v=nv[i])

    ms = _graph_time(step, warmup, steps)
    nbytes = batch * HKV * W * D * 2 * 2 + 2 * batch * HQ * D * 2 + batch * HKV * D * 2 * 2 * 2
    return {"ms_per_step": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "bytes_per_step": nbytes}


def bench_prefill(reps: int = 10, warmup: int = 40) -> dict:
    """chunked-prefill attention, B=8, S=4096, Hq=8/Hkv=2, D=256 bf16, one
    global (causal) and one sliding-window (512) layer. Algorithmic flops = 4 * B * Hq * D *
    (valid (query, key) pairs per (b, h)). Each layer: `warmup` untimed calls (~30 ms of work, as
    the layers before it in a real prefill; after 1-5 the first timed calls still ran 10-15 % slower
    while the GPU settled at its sustained clock), then the mean of `reps` timed calls."""

    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from gemma4_posttrain_jax_amd import kernels

    Bp, S = 8, 4096
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(4)
    q = torch.randn((Bp, S, HKV, R, D), device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn((Bp, HKV, S // 32, D // 32, 2, 16, 32), device=dev, generator=g).to(torch.bfloat16)  # key layout
    vt = torch.randn((Bp, HKV, S // 8, D, 8), device=dev, generator=g).to(torch.bfloat16)  # grouped value layout
    key_mask = torch.ones((Bp, S), dtype=torch.bool, device=dev)
    out = torch.empty_like(q)
    res = {}
    for name, win in (("global", 0), ("sliding", W)):
        pairs = S * (S + 1) // 2 if win == 0 else win * (win + 1) // 2 + (S - win) * win
        flops = 4.0 * Bp * HQ * D * pairs
        for _ in range(warmup):
            kernels.prefill_attention(q, k, vt, key_mask, window=win, out=out)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            kernels.prefill_attention(q, k, vt, key_mask, window=win, out=out)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        res[name] = {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12}
    return res


def cpu_baseline_decode_attention(target_s: float = 12.0) -> dict:
    """The reference's config-2 step on the host: append + dense masked softmax attention over all W
    ring slots (oracle/torch_cpu.py, torch-CPU bf16 on every host core), 1 warm-up step, then the
    median of the timed steps."""

    import torch

    from oracle import torch_cpu as T

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    k = torch.randn((B, HKV, W, D), generator=g).to(torch.bfloat16)  # head-major ring (oracle/torch_cpu.py)
    v = torch.randn((B, HKV, W, D), generator=g).to(torch.bfloat16)
    key_mask = torch.ones((B, CTX + 4096), dtype=torch.bool)
    pos = torch.from_numpy(np.random.default_rng(0).integers(1536, 2048, B).astype(np.int32))
    times = []
    t_begin = time.perf_counter()
    n = 0
    while True:
        q = torch.randn((B, R, HKV, D), generator=g).to(torch.bfloat16)
        nk = torch.randn((B, HKV, D), generator=g).to(torch.bfloat16)
        nv = torch.randn((B, HKV, D), generator=g).to(torch.bfloat16)
        t0 = time.perf_counter()
        # positions advance by one per step and repeat every 2048 steps (inside the key mask)
        T.ring_decode_attention(q, k, v, nk, nv, pos + (n % 2048), key_mask, W)
        times.append(time.perf_counter() - t0)
        n += 1
        if (time.perf_counter() - t_begin > target_s and n >= 4) or n >= 100000:
            break
    sec = float(np.median(times[1:]))  # the first step is the warm-up
    return {
        "value": algorithmic_bytes_per_step() / sec / 1e9,
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{n - 1} timed config-2 steps after 1 warm-up (append + dense masked attention over the 512-slot "
                  f"ring, the reference's algorithm restated in torch-CPU bf16, oracle/torch_cpu.py); median "
                  f"{sec * 1e3:.2f} ms/step on {cpu_info()}",
        "s_per_step": sec,
    }


E2B = dict(
    vocab_size=262144, hidden_size=2048, intermediate_size=8192, num_hidden_layers=30, num_attention_heads=8,
    num_key_value_heads=2, head_dim=256, global_head_dim=256,
    layer_types=(["sliding_attention"] * 4 + ["full_attention"]) * 6, sliding_window=512, num_kv_shared_layers=10,
    hidden_size_per_layer_input=0, final_logit_softcapping=30.0,
)


# q / k norm weights of the E2B-like model in the parity test (tests/test_gpu_e2b.py). With norm
# weights 1 (the benchmarked model, as configs[4] fixes the norms) the normed q and k of dimension
# 256 give scale-1.0 scores up to ~50 (one bf16 ulp 0.25) and the random model is chaotic: the
# oracle run with f32 and with f64 accumulation disagrees by up to 3.8 on the logits. At 0.25 the
# scores are O(1) and the model's outputs are determined well enough to test. The runtime does not
# depend on the values.
E2B_QK_NORM = 0.25


def random_params(cfg, dev, seed=0, qk_norm: float = 1.0):
    """Random-init E2B-like bf16 weights ~N(0, 0.02), q / k norm weights ``qk_norm``, other norms 1,
    layer_scalar 1 (on the GPU)."""

    import torch

    from gemma4_posttrain_jax_amd import model as M
    from gemma4_posttrain_jax_amd.config import (
        is_kv_shared, layer_has_v_proj, layer_head_dim, layer_intermediate_size, layer_kv_heads)

    g = torch.Generator(device=dev).manual_seed(seed)

    def w(*shape):
        return (torch.randn(shape, device=dev, generator=g) * 0.02).to(torch.bfloat16)

    def n(dim, value=1.0):
        return M.RMSNormParams(torch.full((dim,), value, device=dev, dtype=torch.bfloat16))

    Mh = cfg.hidden_size
    layers = []
    for i in range(cfg.num_hidden_layers):
        Dh, H = layer_head_dim(cfg, i), layer_kv_heads(cfg, i)
        Rr = cfg.num_attention_heads // H
        sh = is_kv_shared(cfg, i)
        att = M.AttentionParams(w(Mh, Rr, H, Dh), None if sh else w(Mh, H, Dh),
                                None if sh or not layer_has_v_proj(cfg, i) else w(Mh, H, Dh), w(Rr, H, Dh, Mh),
                                n(Dh, qk_norm), None if sh else n(Dh, qk_norm))
        F = layer_intermediate_size(cfg, i)
        layers.append(M.DecoderLayerParams(n(Mh), att, n(Mh), n(Mh), M.MLPParams(w(Mh, F), w(Mh, F), w(F, Mh)), n(Mh),
                                           None, torch.ones((), device=dev, dtype=torch.bfloat16)))
    return M.Gemma4TextParams(w(cfg.vocab_size, Mh), None, None, None, tuple(layers), n(Mh))


def bench_e2b_decode(steps: int, warmup: int, batch: int = 256, prompt: int = 256, new_tokens: int = 512) -> dict:
    """A whole rollout at B=256: prefill of the 256-token prompts, then the
    ``new_tokens - 1`` decode steps that generate() runs, each its loop body: the bookkeeping launch
    (g4_rollout_step) and one graph replay (one-token forward of all 30 layers + LM head with the
    T=1 draw in its epilogue); the last sampled token is not decoded, sampler.py:287-300.

    ``steps`` = 0 times every decode step after ``warmup`` (the caches fill from 256 to 767
    positions over the rollout, so the average covers short and full rows alike); ``steps`` > 0
    times only that many steps right after the prefill. The prefill is run twice and the second
    call is timed (the first pays one-time library and allocator set-up, as the reference's
    harness excludes compilation and warms up before timing, benchmark_rollout.py:296-311)."""

    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from gemma4_posttrain_jax_amd import config as C
    from gemma4_posttrain_jax_amd import kernels
    from gemma4_posttrain_jax_amd import sampler as SMP

    dev = torch.device("cuda:0")
    cfg = C.config_from_hf(E2B)
    params = random_params(cfg, dev)
    g = torch.Generator(device=dev).manual_seed(1)
    ids = torch.randint(0, cfg.vocab_size, (batch, prompt), device=dev, generator=g, dtype=torch.int32)
    mask = torch.ones_like(ids, dtype=torch.bool)
    SMP.prefill(params, cfg, ids, mask, max_new_tokens=new_tokens)  # set-up run, discarded
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = SMP.prefill(params, cfg, ids, mask, max_new_tokens=new_tokens)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    cache = out.kv_cache
    lengths = torch.full((batch,), prompt, dtype=torch.int32, device=dev)
    active = torch.ones(batch, dtype=torch.bool, device=dev)
    # what generate() does per token at T=1 without EOS ids (sampler.generate's loop body): the
    # bookkeeping launch (g4_rollout_step: the drawn token and logp into the completion columns, the
    # next step's token / position / mask written into the graph's input buffers), then one graph
    # replay = forward of all layers + LM head + fused soft-cap / log-softmax / Gumbel-max draw
    key = SMP.key_tensor(2, dev)  # PRNGKey(2), split once per step on the device
    tok, logp = kernels.sample_tokens(out.logits[:, -1], softcap=None, temperature=1.0, key=key)
    engine = SMP.GraphedDecodeStep(params, cfg, cache, temperature=1.0, key=key)
    completion_ids = torch.full((batch, new_tokens), cfg.pad_token_id, dtype=torch.int32, device=dev)
    completion_mask = torch.zeros((batch, new_tokens), dtype=torch.bool, device=dev)
    rollout_logps = torch.zeros((batch, new_tokens), dtype=torch.float32, device=dev)

    def step(i, tok, logp):
        kernels.rollout_step(i, tok, logp, active, completion_ids=completion_ids, completion_mask=completion_mask,
                             rollout_logps=rollout_logps, pad_id=cfg.pad_token_id, eos_ids=None,
                             prompt_lengths=lengths, next_token=engine.tok, next_pos=engine.pos,
                             next_mask=engine.active)
        return engine.replay_sample()

    n_decode = new_tokens - 1
    timed = n_decode - warmup if steps <= 0 else min(steps, n_decode - warmup)
    torch.cuda.synchronize()
    for i in range(warmup):
        tok, logp = step(i, tok, logp)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(warmup, warmup + timed):
        tok, logp = step(i, tok, logp)
    torch.cuda.synchronize()
    s = (time.perf_counter() - t0) / timed
    rollout_s = prefill_s + n_decode * s
    logits = out.logits[:, -1]
    return {"decode_s_per_step": s, "decode_tok_s": batch / s, "prefill_s": prefill_s, "steps_timed": timed,
            "rollout_s": rollout_s, "rollout_tok_s": batch * new_tokens / rollout_s, "params": params, "cfg": cfg,
            "cache": engine.kv_cache, "logits": logits}


def lm_head_passes(n: int = 3) -> None:
    """g4_lm_head_sample at configs[4]'s LM head, n launches: B = 256 rows of N(0, 1) hidden states
    against the [262144, 2048] bf16 embedding ~N(0, 0.02), soft-cap 30, T = 1 with the key split.
    The launches the LM head's rocprofv3 counter passes read (profiles/)."""

    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from gemma4_posttrain_jax_amd import config as C
    from gemma4_posttrain_jax_amd import kernels
    from gemma4_posttrain_jax_amd import sampler as SMP

    dev = torch.device("cuda:0")
    cfg = C.config_from_hf(E2B)
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(256, cfg.hidden_size, device=dev, generator=g).to(torch.bfloat16)
    embed = (0.02 * torch.randn(cfg.vocab_size, cfg.hidden_size, device=dev, generator=g)).to(torch.bfloat16)
    tok = torch.zeros(256, dtype=torch.int32, device=dev)
    logp = torch.zeros(256, dtype=torch.float32, device=dev)
    key = SMP.key_tensor(123, dev)
    for _ in range(n):
        kernels.lm_head_sample(x, embed, softcap=cfg.final_logit_softcapping, temperature=1.0, key=key,
                               split_key=True, token_out=tok, logp_out=logp)
    torch.cuda.synchronize()


def bench_e2b_generate(params, cfg, batch: int = 256, prompt: int = 256, new_tokens: int = 512,
                       eos_ids: tuple = (), top_k: int = 0, top_p: float = 1.0) -> dict:
    """sampler.generate itself at configs[4] (B=256, P=256, N=512, T=1 full-vocab sampling), timed
    as the reference's harness times its compiled generate (scripts/benchmark_rollout.py:296-357):
    one untimed call, then one timed call from prompt ids to RolloutBatch (prefill, the HIP-graph
    capture of the decode step, the graphed decode steps with fused sampling, the per-step
    bookkeeping). Reports the harness's figures: decode steps = the longest completion, slot
    tokens = batch x decode steps, actual tokens = the sum of the lengths, and its output-semantics
    check (the mask is each row's prefix of its length, pad ids and zero log-probabilities outside
    it, finite ones inside). With ``eos_ids`` rows finish at different steps and the loop exits
    once none is active."""

    import torch

    from gemma4_posttrain_jax_amd import sampler as SMP

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(11)
    ids = torch.randint(0, cfg.vocab_size, (batch, prompt), device=dev, generator=g, dtype=torch.int32)
    mask = torch.ones_like(ids, dtype=torch.bool)
    sc = SMP.SamplerConfig(max_prompt_len=prompt, max_new_tokens=new_tokens, temperature=1.0, seed=3,
                           eos_ids=tuple(eos_ids), top_k=top_k, top_p=top_p)
    SMP.generate(params, cfg, ids, mask, sampler_config=sc, key=1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    rb = SMP.generate(params, cfg, ids, mask, sampler_config=sc, key=2)
    torch.cuda.synchronize()
    s = time.perf_counter() - t0
    lengths = rb.lengths.cpu().numpy().astype(np.int64)
    cm = rb.completion_mask.cpu().numpy()
    ok = bool(np.array_equal(cm, np.arange(new_tokens)[None, :] < lengths[:, None])
              and (rb.completion_ids.cpu().numpy()[~cm] == cfg.pad_token_id).all()
              and (rb.rollout_logps.cpu().numpy()[~cm] == 0).all()
              and np.isfinite(rb.rollout_logps.cpu().numpy()[cm]).all())
    steps = int(lengths.max())
    return {"generate_s": s, "decode_steps": steps, "slot_tok_s": batch * steps / s,
            "actual_tok_s": float(lengths.sum()) / s, "amortized_step_ms": s * 1e3 / steps,
            "mean_length": float(lengths.mean()), "min_length": int(lengths.min()), "output_semantics_ok": ok}


def cpu_baseline_e2b_decode(gpu: dict, steps: int = 3) -> dict:
    """The reference's full decode step at B=256 on the host (oracle/torch_cpu.py: torch-CPU bf16 on
    every host core, dense attention over the whole 768-slot capacity, full-vocab log-softmax),
    weights copied from the GPU: 1 warm-up step, then the median of ``steps`` timed steps."""

    import torch

    from oracle import g4_oracle as O
    from oracle import torch_cpu as T

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cfg, params = gpu["cfg"], gpu["params"]

    def a(t):
        return None if t is None else t.float().cpu().numpy()

    def nw(p):
        return None if p is None else a(p.weight)

    layers = []
    for lp in params.layers:
        at = lp.attention
        layers.append(O.LayerParams(nw(lp.input_norm), O.AttnParams(a(at.q_proj), a(at.k_proj), a(at.v_proj),
                                                                    a(at.o_proj), nw(at.q_norm), nw(at.k_norm)),
                                    nw(lp.post_attention_norm), nw(lp.pre_feedforward_norm),
                                    O.MLPParams(a(lp.mlp.gate_proj), a(lp.mlp.up_proj), a(lp.mlp.down_proj)),
                                    nw(lp.post_feedforward_norm), None, np.float32(1.0)))
    op = O.Params(a(params.embed_tokens), None, None, None, tuple(layers), nw(params.final_norm))
    model = T.TorchCPUModel(op, O.config_from_hf(E2B))
    del op, layers
    Bsz = gpu["logits"].shape[0]
    cap = gpu["cache"].key_mask.shape[1]
    length = min(gpu["cache"].length, cap - steps - 2)  # room for the timed steps' appends
    cache = model.init_cache(Bsz, cap)
    cache["key_mask"][:, :length] = True
    cache["length"] = length
    torch.cuda.empty_cache()
    tok = torch.zeros(Bsz, dtype=torch.int32)
    times = []
    with torch.no_grad():
        for i in range(steps + 1):
            t0 = time.perf_counter()
            T.decode_step(model, tok, torch.full((Bsz,), length + i, dtype=torch.int32), cache)
            times.append(time.perf_counter() - t0)
    return {"s_per_step": float(np.median(times[1:])), "steps": steps, "cores": cores}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    # 1000 untimed steps (~15 ms of the same launch): after only 8 the timed steps ran 1-2 % slower
    # while the GPU settled at its sustained clock
    ap.add_argument("--warmup", type=int, default=1000)
    ap.add_argument("--e2b-steps", type=int, default=0,
                    help="E2B decode steps to time (0: every step of the 512-token rollout)")
    ap.add_argument("--no-e2b", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the configs[2]/[3] lines")
    ap.add_argument("--pmc-calibration", action="store_true",
                    help="first copy 256 MiB device-to-device once: the reference kernel whose FETCH_SIZE / "
                         "WRITE_SIZE counters scale the decode kernel's (see profiles/)")
    ap.add_argument("--lm-head-only", action="store_true",
                    help="only run g4_lm_head_sample at configs[4]'s shape three times (after the calibration "
                         "copy, if asked for), for the LM head's counter passes; prints no bench line")
    ap.add_argument("--e2b-only", action="store_true",
                    help="only the configs[4] decode (prefill, then --e2b-steps graphed steps, default 4), for the "
                         "decode step's counter passes; prints the step time, not the bench line")
    ap.add_argument("--num-splits", type=int, default=0,
                    help="workgroups per (b, kv head) for decode attention (0: library default)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (every box here has one GPU)",
              file=sys.stderr)
        return 2

    if args.pmc_calibration:
        import torch
        src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.lm_head_only:
        lm_head_passes()
        print("lm head passes done")
        return 0
    if args.e2b_only:
        e2b = bench_e2b_decode(args.e2b_steps if args.e2b_steps > 0 else 4, 2)
        print(json.dumps({"e2b_decode_ms_per_step": round(e2b["decode_s_per_step"] * 1e3, 3),
                          "steps_timed": e2b["steps_timed"]}))
        return 0
    # The configs[2]-[4] lines run first, so that the headline's timed steps find the GPU at the
    # sustained clock it holds inside a model step (on a cold GPU the first milliseconds of work ran
    # 1-2 % slower).
    extra: dict = {}
    if not args.no_extra:
        lc = bench_long_context_decode()
        extra["long_context_decode"] = {"workload": "configs[2]: B16 Hq8/Hkv2 D256, linear cache 32768, ragged "
                                       "lengths U[1024,32768], split-K", "ms_per_step": round(lc["ms_per_step"], 4),
                                       "GB/s": round(lc["gbs"], 1), "frac_hbm_peak": round(lc["gbs"] / HBM_PEAK_GBS, 4)}
        ea = bench_e2b_decode_attention()
        extra["e2b_decode_attention"] = {"workload": "configs[4] shape: one sliding layer's decode attention at B256 "
                                        "Hq8/Hkv2 D256, full 512-slot ring, 1-token append + attend, two-launch path",
                                        "ms_per_step": round(ea["ms_per_step"], 4), "GB/s": round(ea["gbs"], 1),
                                        "frac_hbm_peak": round(ea["gbs"] / HBM_PEAK_GBS, 4)}
        pf = bench_prefill()
        extra["prefill_attention"] = {
            "workload": "configs[3]: B8 S4096 Hq8/Hkv2 D256 bf16 attention, per layer",
            **{f"{k}_ms": round(v["ms"], 3) for k, v in pf.items()},
            **{f"{k}_TFLOP/s": round(v["tflops"], 1) for k, v in pf.items()},
            **{f"{k}_frac_mfma_peak": round(v["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4) for k, v in pf.items()}}
        pc = prefill_counters()
        if pc is not None:  # rocprofv3 PMC: SQ_VALU_MFMA_BUSY_CYCLES, SQ_INSTS_VALU_MFMA_MOPS_BF16
            for k in ("global", "sliding"):
                extra["prefill_attention"][f"{k}_mfma_busy_counter"] = pc[k]["mfma_busy_frac"]
                extra["prefill_attention"][f"{k}_executed_TFLOP_counter"] = pc[k]["executed_bf16_tflop"]
            extra["prefill_attention"]["counters"] = pc["source"]
    res = bench_decode_attention(args.steps, args.warmup, args.num_splits)
    bytes_step = algorithmic_bytes_per_step()
    gbs = bytes_step / (res["ms_per_step"] * 1e-3) / 1e9
    line = {
        "metric": "decode-attn HBM GB/s (% of peak) + decode tokens/sec at batch 256, 1 GPU",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "configs[1]: sliding-window decode attention, 1-token append + attend per step",
                   "batch": B, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "window": W, "ring_context": CTX,
                   "bytes_per_step": bytes_step, "caches_round_robin": NCACHE, "num_splits": args.num_splits},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic()},
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
        "eager_ms_per_step": round(res["eager_ms_per_step"], 4),
    }
    line.update(extra)
    if not args.no_e2b:
        e2b = bench_e2b_decode(args.e2b_steps, 2)
        line["decode_tok_s_b256"] = round(e2b["decode_tok_s"], 1)
        line["decode_ms_per_step_b256"] = round(e2b["decode_s_per_step"] * 1e3, 3)
        line["decode_steps_timed_b256"] = e2b["steps_timed"]
        line["prefill_s_b256_p256"] = round(e2b["prefill_s"], 3)
        # the reference harness's slot tokens/s: batch x new tokens / (prefill + every decode step)
        line["rollout_tok_s_b256"] = round(e2b["rollout_tok_s"], 1)
        gen = bench_e2b_generate(e2b["params"], e2b["cfg"])
        assert gen["min_length"] == 512 and gen["output_semantics_ok"]
        line["generate_s_b256"] = round(gen["generate_s"], 3)
        line["generate_tok_s_b256"] = round(gen["slot_tok_s"], 1)
        # with EOS ids (every 64th vocab id: at T = 1 a row stops after ~64 tokens on average, the
        # longest after a few hundred), the GRPO caller's configuration (train_grpo.py:854-856)
        eos = bench_e2b_generate(e2b["params"], e2b["cfg"], eos_ids=tuple(range(1, e2b["cfg"].vocab_size, 64)))
        tk = bench_e2b_generate(e2b["params"], e2b["cfg"], top_k=50)
        assert tk["min_length"] == 512 and tk["output_semantics_ok"]
        line["generate_top_k50_b256"] = {
            "workload": "configs[4] generate at the reference harness's default draw: T = 1, top_k = 50 "
                        "(scripts/benchmark_rollout.py:62-67), native top-k draw in the decode graph",
            "s": round(tk["generate_s"], 3), "slot_tok_s": round(tk["slot_tok_s"], 1),
            "amortized_step_ms": round(tk["amortized_step_ms"], 3)}
        line["generate_eos_b256"] = {
            "workload": "configs[4] generate with 4096 EOS ids (every 64th id), rows finishing at varied steps",
            "s": round(eos["generate_s"], 3), "decode_steps": eos["decode_steps"],
            "mean_length": round(eos["mean_length"], 1), "slot_tok_s": round(eos["slot_tok_s"], 1),
            "actual_tok_s": round(eos["actual_tok_s"], 1), "amortized_step_ms": round(eos["amortized_step_ms"], 3),
            "output_semantics_ok": eos["output_semantics_ok"]}
        if not args.no_cpu:
            cpu5 = cpu_baseline_e2b_decode(e2b)
            line["cpu_decode_s_per_step_b256"] = round(cpu5["s_per_step"], 3)
            line["cpu_decode_b256"] = (f"torch-CPU bf16 restatement of the reference's decode step (oracle/torch_cpu.py), "
                                      f"{cpu5['cores']} cores, 1 warm-up + median of {cpu5['steps']} steps at B=256")
            line["decode_speedup_vs_cpu"] = round(cpu5["s_per_step"] / e2b["decode_s_per_step"], 1)
        del e2b
    if not args.no_cpu:
        cpu = cpu_baseline_decode_attention()
        line["cpu_baseline"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in cpu.items()
                                if k != "s_per_step"}
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
