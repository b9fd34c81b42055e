"""BASELINE config 5 end to end: the 30-layer E2B-like model (M 2048, F 8192, 8 q / 2 kv heads,
head dim 256, sliding window 512 in a 4:1 pattern, last 10 layers kv-shared, V 262144, bf16
N(0, 0.02); q / k norm weights bench.E2B_QK_NORM) at the rollout batch B = 256 with 256-token
prompts, against the oracle.

The GPU runs the production path at full size: the prefill (hipBLASLt projections, the fused
append, the LDS prefill attention), then graphed decode steps with fused sampling (the native
prologue, the q/k/v preparation inside the two-launch decode attention, the gated-GELU gate/up
GEMM, the split-K down projection into the residual norm, the LM head and the fused sampler)
until the 512-slot rings have wrapped.

Parity is checked kernel by kernel (tests/kernel_trace.py): every step of the forward is recorded
for a few rows and recomputed by the oracle from the recorded inputs, so each kernel is held to
one bf16 rounding (attention rows to 2e-2) however the model amplifies last-bit differences
between steps. The end-to-end difference of the logits (the oracle run free from the embedding)
is printed beside the oracle's own f32-vs-f64 spread, which measures that amplification. The
token the fused sampler draws for every row must equal the oracle's categorical draw over all
262,144 columns under the same key.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import model_bars, oracle_cache_rows, oracle_params, to_np, ulp_stats
from kernel_trace import KernelTrace, check_trace, clear_weight_cache
from oracle import g4_oracle as O
from oracle import jax_random as JR

import bench
from gemma4_posttrain_jax_amd import config as C
from gemma4_posttrain_jax_amd import kernels
from gemma4_posttrain_jax_amd import model as M
from gemma4_posttrain_jax_amd import sampler as SMP
from gemma4_posttrain_jax_amd.kvcache import init_kv_cache

pytestmark = pytest.mark.gpu

B, P, N = 256, 256, 512
ROWS = (0, 77, 200, 255)  # rows the oracle follows; row 77 is left-padded by 40 tokens
PAD_ROW, PAD = 77, 40
LOGP_ATOL = 2e-6


def _say(msg):
    print(f"[e2b] {msg}", flush=True)


def _summary(name, results):
    worst = max((r for r in results if isinstance(r[2], float)), key=lambda r: r[2], default=None)
    _say(f"{name}: {len(results)} kernel comparisons passed; largest ulp difference {worst}")


@pytest.fixture(scope="module")
def e2b(device):
    torch.set_grad_enabled(False)
    cfg = C.config_from_hf(bench.E2B)
    ocfg = O.config_from_hf(bench.E2B)
    params = bench.random_params(cfg, device, seed=0, qk_norm=bench.E2B_QK_NORM)
    g = torch.Generator(device=device).manual_seed(5)
    ids = torch.randint(0, cfg.vocab_size, (B, P), device=device, generator=g, dtype=torch.int32)
    mask = torch.ones_like(ids, dtype=torch.bool)
    mask[PAD_ROW, :PAD] = False
    ids[PAD_ROW, :PAD] = cfg.pad_token_id
    _say("prefill B=256 P=256")
    out = SMP.prefill(params, cfg, ids, mask, max_new_tokens=N)
    torch.cuda.synchronize()
    yield dict(cfg=cfg, ocfg=ocfg, params=params, ids=ids, mask=mask, out=out)
    clear_weight_cache()


def test_e2b_prefill_kernels_match_oracle(e2b, device):
    """sampler.prefill (sampler.py:70-106) at B=256, P=256: the same forward recorded step by step
    gives bitwise the logits of sampler.prefill, and every recorded step for two rows (one
    left-padded) matches the oracle on its inputs: projections, the q/k/v norms + RoPE and the
    ring / linear cache writes, the prefill attention, the norms and residuals, the gated GELU, the
    LM head."""

    cfg, params, ids, mask = e2b["cfg"], e2b["params"], e2b["ids"], e2b["mask"]
    cache = init_kv_cache(cfg, B, P + N, torch.bfloat16, device)
    with KernelTrace([0, PAD_ROW], B) as trace:
        out = M.forward_gemma4_lm(params, ids, SMP._position_ids(mask), config=cfg, attention_mask=mask,
                                  kv_cache=cache, cache_mode="prefill", logits_to_keep=1)
    assert torch.equal(out.logits, e2b["out"].logits)
    kinds = [k for k, _ in trace.calls]
    assert kinds.count("prefill_attention") == 30 and kinds.count("proj") == 30 * 4 + 1
    results = check_trace(trace, window=cfg.sliding_window)
    got = to_np(out.logits.index_select(0, torch.tensor([0, PAD_ROW], device=device)))
    raw = trace.calls[-1][1]["y"].reshape(got.shape)  # the LM head's bf16 logits before the soft-cap
    cap = np.float32(cfg.final_logit_softcapping)
    exact, ulps = ulp_stats(got, O.cast(np.tanh(raw / cap) * cap, O.BF16))
    assert exact >= 0.999 and ulps <= 1.0, f"soft-cap: {exact} {ulps}"
    _summary("prefill", results)


def _clone_cache(cache):
    return [None if l is None else (l.key.clone(), l.value_t.clone()) for l in cache.layers], cache.key_mask.clone()


def _restore_cache(cache, snap):
    layers, km = snap
    for l, s in zip(cache.layers, layers):
        if l is not None:
            l.key.copy_(s[0])
            l.value_t.copy_(s[1])
    cache.key_mask.copy_(km)


def test_e2b_graphed_decode_after_ring_wrap_matches_oracle(e2b, device):
    """generate's loop body (sampler.py:262-312) at B=256 after 260 graphed steps (positions up to
    516: the 512-slot rings have wrapped). One more step then runs three times from the same
    state: the sampling graph (tokens, logp), the logits graph, and the same forward eagerly,
    recorded step by step (bitwise the logits graph's logits and caches). Checks: every row's
    drawn token equals the oracle's categorical draw (oracle/jax_random.py) over the logits
    graph's 262,144 logits under the same key, logp within 2e-6; every recorded kernel for four
    rows matches the oracle on its inputs (the prologue, the q/k/v preparation and cache append
    inside the decode attention, the attention over the wrapped ring and the 768-slot linear
    cache, the gate/up GEMM with its GELU epilogue, the split-K down projection with the residual
    norm, the LM head)."""

    cfg, ocfg, params, out = e2b["cfg"], e2b["ocfg"], e2b["params"], e2b["out"]
    key = SMP.key_tensor(9, device)
    tok, _ = kernels.sample_tokens(out.logits[:, -1], softcap=None, temperature=1.0, key=key)
    engine = SMP.GraphedDecodeStep(params, cfg, out.kv_cache, temperature=1.0, key=key)
    plen = e2b["mask"].sum(-1, dtype=torch.int32)
    active = torch.ones(B, dtype=torch.bool, device=device)
    steps = 260
    _say(f"{steps} graphed sampling steps")
    for i in range(steps):
        tok, _ = engine.step_sample(tok.clone(), plen + i, active)
    torch.cuda.synchronize()
    tok = tok.clone()
    pos = plen + steps
    cache = engine.kv_cache
    assert cache.length == P + steps
    snap = _clone_cache(cache)
    key_before = [int(w) & 0xFFFFFFFF for w in key.cpu().tolist()]
    s_tok, s_logp = (x.cpu().numpy().copy() for x in engine.step_sample(tok, pos, active))
    _restore_cache(cache, snap)
    rows = list(ROWS)
    ocache = oracle_cache_rows(cache, rows)
    logits_engine = SMP.GraphedDecodeStep(params, cfg, cache)
    logits = logits_engine.step(tok, pos, active).clone()
    after = _clone_cache(logits_engine.kv_cache)
    lg = to_np(logits)

    # the fused sampler's draw: the oracle's categorical over the same logits and key
    _, sample_key = JR.split(np.asarray(key_before, np.uint32))
    want_tok, want_logp = O.sample_token(lg, temperature=1.0, key=sample_key)
    _say(f"sampled tokens: {int((want_tok != s_tok).sum())} of {B} rows differ from the oracle's draw")
    np.testing.assert_array_equal(s_tok, want_tok)
    np.testing.assert_allclose(s_logp, want_logp, rtol=0, atol=LOGP_ATOL)

    # the same step eagerly, recorded kernel by kernel (the graph captures this call)
    _restore_cache(cache, snap)
    slot = torch.full((B,), int(cache.length), dtype=torch.int32, device=device)
    with KernelTrace(rows, B) as trace:
        step = M.forward_gemma4_lm(params, tok[:, None], pos[:, None], config=cfg, attention_mask=active[:, None],
                                   kv_cache=cache, cache_mode="append", logits_to_keep=1, write_pos=slot)
    assert torch.equal(step.logits[:, -1].float(), logits)
    for (k1, v1), l2 in zip((s for s in after[0] if s is not None), (l for l in step.kv_cache.layers if l is not None)):
        assert torch.equal(k1, l2.key) and torch.equal(v1, l2.value_t)
    kinds = [k for k, _ in trace.calls]
    assert kinds.count("decode_attention_fused") == 30 and kinds.count("linear_gelu") == 30
    assert kinds.count("residual_norm_splitk") == 30 and kinds[0] == "decode_prologue"
    results = check_trace(trace, window=cfg.sliding_window)
    _summary("decode step", results)

    # end to end: the oracle's decode step from the embedding on (reported: the random model
    # amplifies last-bit differences over 30 layers; see the oracle's own f32-vs-f64 spread)
    t, p = tok.cpu().numpy()[rows], pos.cpu().numpy()[rows]
    oparams = oracle_params(params)
    ref, _, _ = O.decode_step(oparams, ocfg, t, p, ocache, dtype=O.BF16)
    with O.accumulate_f64():
        ref64, _, _ = O.decode_step(oparams, ocfg, t, p, ocache, dtype=O.BF16)
    err, _, spread = model_bars(O.BF16, lg[rows], ref[:, -1], ref64[:, -1])
    _say(f"end-to-end decode logits: max|err| {err:.4g} (oracle f32/f64 spread {spread:.4g}; |logits| <= "
         f"{np.abs(ref).max():.3g}; one bf16 ulp at 4 is 0.031)")
