"""Kernel-by-kernel parity of a model forward at full size: every native / library step the
forward makes is recorded (inputs and outputs, restricted to a few batch rows) and the oracle
recomputes that step from the recorded inputs.

A random bf16 model amplifies a last-bit difference from one step through the steps after it (an
attention score that rounds the other way, then a norm), so comparing layer outputs or logits at
depth measures the model's conditioning as much as the kernels. Feeding each step its own
recorded inputs isolates the kernels: every step must then agree with the oracle to one bf16
rounding (attention rows to the 2e-2 bar, against the f32- or the f64-accumulated oracle).
"""

from __future__ import annotations


import numpy as np
import torch

from gpu_util import TOL, attention_rows, k_slots, to_np, ulp_stats, vt_slots
from oracle import g4_oracle as O

from gemma4_posttrain_jax_amd import kernels
from gemma4_posttrain_jax_amd import model as M

# bars per recorded step: (minimum bit-equal fraction, largest difference in bf16 ulps, ulp floor as a
# fraction of the array's RMS)
GEMM_BAR = (0.99, 1.0, 0.125)  # one rounding of an f32 sum accumulated in another order
NORM_BAR = (0.999, 1.0, 0.125)  # f32 statistics summed in another order, then one rounding
# RMSNorm then RoPE: a flipped norm rounding moves a rotated value by one ulp of its terms, whose
# magnitude is the row's (RMS 1), also where the rotation cancels to a small result
PREP_BAR = (0.999, 2.0, 1.0)
# residual + RMSNorm(branch) (+ the down projection for the split-K variant): a branch element one
# rounding off moves the sum by one ulp of the branch, which may exceed the sum's own where they cancel
RESIDUAL_BAR = (0.999, 2.0, 1.0)
RESIDUAL_SPLITK_BAR = (0.99, 2.0, 1.0)
# gelu(g) * u of two GEMM outputs that may each be one rounding off
GELU_GEMM_BAR = (0.99, 2.0, 0.125)


class KernelTrace:
    """Context manager recording the model's calls (in order) for batch rows ``rows`` of a forward
    over ``batch`` rows (2-D GEMM inputs are [batch * S, K])."""

    def __init__(self, rows, batch: int):
        self.rows = list(rows)
        self.batch = batch
        self.calls: list[tuple[str, dict]] = []
        self._saved: list = []

    def _sel(self, t):
        if t is None:
            return None
        idx = torch.as_tensor(self.rows, device=t.device)
        if t.shape[0] == self.batch:
            return to_np(t.index_select(0, idx))
        n = t.shape[0] // self.batch
        return to_np(t.reshape(self.batch, n, *t.shape[1:]).index_select(0, idx))

    def _layer(self, layer):
        idx = torch.as_tensor(self.rows, device=layer.key.device)
        return (to_np(layer.key_slots().index_select(0, idx)), to_np(layer.value_dmajor().index_select(0, idx)),
                layer.capacity,
                layer.ring)

    def _patch(self, mod, name, make):
        orig = getattr(mod, name)
        self._saved.append((mod, name, orig))
        setattr(mod, name, make(orig))

    def __enter__(self):
        sel, rec = self._sel, self.calls.append

        def proj(orig):
            def f(x, w_t):
                y = orig(x, w_t)
                rec(("proj", dict(x=sel(x), y=sel(y), w=w_t)))
                return y
            return f

        def lm_head(orig):
            def f(x, embed, *, out=None):
                y = orig(x, embed, out=out)
                rec(("proj", dict(x=sel(x), y=sel(y), w=embed)))
                return y
            return f

        def rms(orig):
            def f(x, weight, eps, out=None):
                y = orig(x, weight, eps, out)
                rec(("rms_norm", dict(x=sel(x), y=sel(y), w=weight, eps=eps)))
                return y
            return f

        def resnorm(orig):
            def f(branch, branch_weight, residual, *, scalar, next_weight, eps, with_next=True):
                x, h = orig(branch, branch_weight, residual, scalar=scalar, next_weight=next_weight, eps=eps,
                            with_next=with_next)
                rec(("residual_norm", dict(branch=sel(branch), residual=sel(residual), x=sel(x), h=sel(h),
                                           bw=branch_weight, nw=next_weight, scalar=scalar, eps=eps)))
                return x, h
            return f

        def gelu(orig):
            def f(gu):
                y = orig(gu)
                rec(("gelu_mul", dict(gu=sel(gu), y=sel(y))))
                return y
            return f

        def linear_gelu(orig):
            def f(x, w, *, out=None):
                y = orig(x, w, out=out)
                rec(("linear_gelu", dict(x=sel(x), y=sel(y), w=w)))
                return y
            return f

        def partials(orig):
            def f(x, w, *, ksplit):
                p = orig(x, w, ksplit=ksplit)
                rec(("linear_partials", dict(x=sel(x), w=w)))
                return p
            return f

        def resnorm_splitk(orig):
            def f(partials, branch_weight, residual, *, scalar, next_weight, eps):
                x, h = orig(partials, branch_weight, residual, scalar=scalar, next_weight=next_weight, eps=eps)
                rec(("residual_norm_splitk", dict(residual=sel(residual), x=sel(x), h=sel(h), bw=branch_weight,
                                                  nw=next_weight, scalar=scalar, eps=eps)))
                return x, h
            return f

        def append(orig):
            def f(layer, k, v, **kw):
                r = orig(layer, k, v, **kw)
                rec(("kv_append", dict(k=sel(k), v=sel(v), q=sel(kw.get("q")), q_out=sel(kw.get("q_out")),
                                       k_out=sel(kw.get("k_out")), vt_out=sel(kw.get("vt_out")),
                                       cos=sel(kw.get("rope_cos")), sin=sel(kw.get("rope_sin")),
                                       qn=kw.get("q_norm_weight"), kn=kw.get("k_norm_weight"), eps=kw.get("eps"),
                                       flags=kw.get("flags", 0), layer=self._layer(layer), write_pos=kw.get("write_pos"))))
                return r
            return f

        def prep_q(orig):
            def f(q, q_out, **kw):
                r = orig(q, q_out, **kw)
                rec(("kv_append", dict(k=None, v=None, q=sel(q), q_out=sel(q_out), k_out=None, vt_out=None,
                                       cos=sel(kw.get("rope_cos")), sin=sel(kw.get("rope_sin")),
                                       qn=kw.get("q_norm_weight"), kn=None, eps=kw.get("eps"),
                                       flags=kw.get("flags", 0), layer=None, write_pos=None)))
                return r
            return f

        def prefill_attn(orig):
            def f(q, k, vt, key_mask, *, window, out=None):
                o = orig(q, k, vt, key_mask, window=window, out=out)
                rec(("prefill_attention", dict(q=sel(q), k=sel(k), vt=sel(vt), km=sel(key_mask), window=window,
                                               out=sel(o))))
                return o
            return f

        def fused(orig):
            def f(layer, q_raw, key_mask, **kw):
                before = self._layer(layer)
                o = orig(layer, q_raw, key_mask, **kw)
                rec(("decode_attention_fused", dict(
                    before=before, after=self._layer(layer), q=sel(q_raw), k=sel(kw["k_raw"]), v=sel(kw["v_raw"]),
                    km=sel(key_mask), q_pos=sel(kw["q_pos"]), window=kw["window"], cos=sel(kw["rope_cos"]),
                    sin=sel(kw["rope_sin"]), qn=kw["q_norm_weight"], kn=kw["k_norm_weight"], eps=kw["eps"],
                    flags=kw["flags"], out=sel(o))))
                return o
            return f

        def prologue(orig):
            def f(embed, tokens, positions, active, slot, key_mask, *, embed_scale, inv_freq):
                x, tables = orig(embed, tokens, positions, active, slot, key_mask, embed_scale=embed_scale,
                                 inv_freq=inv_freq)
                rec(("decode_prologue", dict(x=sel(x), tokens=sel(tokens), positions=sel(positions),
                                             tables=[(sel(c), sel(s)) for c, s in tables], inv_freq=inv_freq,
                                             embed=embed, embed_scale=embed_scale)))
                return x, tables
            return f

        self._patch(M, "_proj", proj)
        for name, make in (("rms_norm", rms), ("residual_norm", resnorm), ("gelu_mul", gelu),
                           ("linear_gelu", linear_gelu), ("linear_partials", partials),
                           ("residual_norm_splitk", resnorm_splitk), ("kv_append", append), ("prepare_q", prep_q),
                           ("prefill_attention", prefill_attn), ("decode_attention_fused", fused),
                           ("decode_prologue", prologue), ("lm_head", lm_head)):
            self._patch(kernels, name, make)
        return self

    def __exit__(self, *exc):
        for mod, name, orig in reversed(self._saved):
            setattr(mod, name, orig)
        self._saved.clear()


_WEIGHTS: dict = {}


def w_np(t: torch.Tensor | None):
    """Device weight -> float32 numpy (cached per tensor for the trace's lifetime)."""

    if t is None:
        return None
    key = (t.data_ptr(), tuple(t.shape))
    if key not in _WEIGHTS:
        _WEIGHTS[key] = to_np(t)
    return _WEIGHTS[key]


def clear_weight_cache() -> None:
    _WEIGHTS.clear()


def _bar(name, got, want, bar, results):
    exact, ulps = ulp_stats(got, want, bar[2] if len(bar) > 2 else 0.125)
    results.append((name, exact, ulps))
    assert exact >= bar[0] and ulps <= bar[1], f"{name}: bit-equal {exact:.5f}, max {ulps:.2f} ulp (bar {bar})"


def _rows_ok(name, got, r32, r64, results, max_f64_rows=1):
    err, n64, bad = attention_rows(got, r32, r64, TOL[O.BF16])
    results.append((name, err, n64))
    assert bad == 0 and n64 <= max_f64_rows, f"{name}: max {err}, {n64} rows only near the f64 oracle, {bad} neither"


def _prep_qkv(d, R, D, dtype=O.BF16):
    """g4_kv_append's / G4DecodePrep's preparation (model.py:463-482) on recorded raw rows."""

    rope = lambda x, c, s: O.rope(x, c, s, dtype)  # noqa: E731
    flags = d["flags"]
    q = d["q"]
    q = O.rms_norm(w_np(d["qn"]), q, d["eps"], dtype) if flags & 8 else q
    q = rope(q, d["cos"], d["sin"]) if flags & 16 else q
    k = v = None
    if d.get("k") is not None:
        k = O.rms_norm(w_np(d["kn"]), d["k"], d["eps"], dtype) if flags & 1 else d["k"]
        k = rope(k, d["cos"], d["sin"]) if flags & 4 else k
        v = O.rms_norm(None, d["v"], d["eps"], dtype) if flags & 2 else d["v"]
    return q, k, v


def check_trace(trace: KernelTrace, *, window: int) -> list:
    """Recompute every recorded step with the oracle on its recorded inputs and assert the bars.
    Returns (step, bit-equal fraction or max error, max ulps or f64 rows) per comparison."""

    results: list = []
    pending_partials = None
    for i, (kind, d) in enumerate(trace.calls):
        tag = f"call {i} {kind}"
        if kind == "proj":
            want = O.matmul(d["x"], w_np(d["w"]).T, O.BF16)
            _bar(tag, d["y"], want, GEMM_BAR, results)
        elif kind == "rms_norm":
            _bar(tag, d["y"], O.rms_norm(w_np(d["w"]), d["x"], d["eps"], O.BF16), NORM_BAR, results)
        elif kind in ("residual_norm", "residual_norm_splitk"):
            if kind == "residual_norm":
                branch = d["branch"]
            else:
                xp, wp = pending_partials
                # the down projection's bf16 output, shaped like the residual
                branch = O.matmul(xp, w_np(wp).T, O.BF16).reshape(d["residual"].shape)
            x = O.cast(d["residual"] + O.rms_norm(w_np(d["bw"]), branch, d["eps"], O.BF16), O.BF16)
            if d["scalar"] is not None:
                x = O.cast(x * np.float32(d["scalar"].item()), O.BF16)
            bar = RESIDUAL_SPLITK_BAR if kind == "residual_norm_splitk" else RESIDUAL_BAR
            _bar(tag + " x", d["x"], x, bar, results)
            if d["h"] is not None:
                _bar(tag + " h", d["h"], O.rms_norm(w_np(d["nw"]), d["x"], d["eps"], O.BF16), NORM_BAR, results)
        elif kind == "gelu_mul":
            F = d["gu"].shape[-1] // 2
            want = O.cast(O.gelu_tanh(d["gu"][..., :F]) * d["gu"][..., F:], O.BF16)
            _bar(tag, d["y"], want, NORM_BAR, results)
        elif kind == "linear_gelu":
            w = w_np(d["w"])
            F = w.shape[0] // 2
            g = O.matmul(d["x"], w[:F].T, O.BF16)
            u = O.matmul(d["x"], w[F:].T, O.BF16)
            _bar(tag, d["y"], O.cast(O.gelu_tanh(g) * u, O.BF16), GELU_GEMM_BAR, results)
        elif kind == "linear_partials":
            pending_partials = (d["x"], d["w"])
        elif kind == "kv_append":
            q_out = d["q_out"]
            R, D = q_out.shape[-2], q_out.shape[-1]
            q, k, v = _prep_qkv(d, R, D)
            _bar(tag + " q", q_out, q, PREP_BAR, results)
            if d["k_out"] is not None:
                S = d["k"].shape[1]
                _bar(tag + " k", k_slots(d["k_out"])[:, :, :S].transpose(0, 2, 1, 3), k, PREP_BAR, results)
                _bar(tag + " v", vt_slots(d["vt_out"])[:, :, :S].transpose(0, 2, 1, 3), v, NORM_BAR, results)
            if k is not None:
                ck, cvt, cap, ring = d["layer"]
                assert isinstance(d["write_pos"], int) and d["write_pos"] == 0, "traced appends start at 0"
                S = k.shape[1]
                keep = min(S, cap) if ring else S
                slots = (np.arange(S - keep, S) % cap) if ring else np.arange(S)  # prefill: start 0
                _bar(tag + " cache k", ck[:, :, slots].transpose(0, 2, 1, 3), k[:, S - keep:], PREP_BAR, results)
                _bar(tag + " cache v", cvt[:, :, :, slots].transpose(0, 3, 1, 2), v[:, S - keep:], NORM_BAR, results)
        elif kind == "prefill_attention":
            q = d["q"]  # [r, S, H, R, D]
            S = q.shape[1]
            k = k_slots(d["k"])[:, :, :S].transpose(0, 2, 1, 3)
            v = vt_slots(d["vt"])[:, :, :S].transpose(0, 2, 1, 3)
            mask = O.make_qk_masks(d["km"][:, :S], d["window"] if d["window"] else 1 << 30, 0, S)[O.SLIDING]
            qr = q.transpose(0, 1, 3, 2, 4)
            r32 = O.attention_core(qr, k, v, mask, O.BF16).transpose(0, 1, 3, 2, 4)
            with O.accumulate_f64():
                r64 = O.attention_core(qr, k, v, mask, O.BF16).transpose(0, 1, 3, 2, 4)
            _rows_ok(tag, d["out"], r32, r64, results, max_f64_rows=max(1, r32[..., 0].size // 1000))
        elif kind == "decode_attention_fused":
            ck, cvt, cap, ring = d["before"]
            ak, avt, _, _ = d["after"]
            q_raw = d["q"]  # [r, H, R, D]
            R, D = q_raw.shape[-2], q_raw.shape[-1]
            cos, sin = d["cos"][:, None], d["sin"][:, None]  # [r, 1, D]
            dd = dict(d, q=q_raw[:, None], k=None if d["k"] is None else d["k"][:, None],
                      v=None if d["v"] is None else d["v"][:, None], cos=cos, sin=sin)
            q, k, v = _prep_qkv(dd, R, D)
            keys = ck[:, :, :cap].transpose(0, 2, 1, 3).copy()  # [r, cap, H, D]
            vals = cvt[:, :, :, :cap].transpose(0, 3, 1, 2).copy()
            qpos = d["q_pos"].astype(np.int64)
            if k is not None:
                with O.inplace_cache_updates():
                    O.update_layer_cache(O.LayerKV(keys, vals), k, v, qpos, ring, O.BF16)
                got_k = ak[:, :, :cap].transpose(0, 2, 1, 3)
                got_v = avt[:, :, :, :cap].transpose(0, 3, 1, 2)
                _bar(tag + " cache k", got_k, keys, PREP_BAR, results)
                _bar(tag + " cache v", got_v, vals, NORM_BAR, results)
            masks = O.make_cached_qk_masks(d["km"], window, qpos, 1)
            mask = masks[O.SLIDING] if ring else masks[O.FULL]
            qr = q.transpose(0, 1, 3, 2, 4)  # [r, 1, R, H, D]
            r32 = O.attention_core(qr, keys, vals, mask, O.BF16)[:, 0].transpose(0, 2, 1, 3)
            with O.accumulate_f64():
                r64 = O.attention_core(qr, keys, vals, mask, O.BF16)[:, 0].transpose(0, 2, 1, 3)
            _rows_ok(tag, d["out"], r32, r64, results)
        elif kind == "decode_prologue":
            embed = w_np(d["embed"])
            x = O.cast(embed[d["tokens"].astype(np.int64)] * np.float32(d["embed_scale"]), O.BF16)
            _bar(tag + " embedding", d["x"], x, (1.0, 0.0, 0.125), results)
            for f, (c, sn) in zip(d["inv_freq"], d["tables"]):
                rc, rs = O.rotary_values(to_np(f), d["positions"][:, None])  # [r, 1, D]
                np.testing.assert_allclose(c, rc[:, 0], rtol=0, atol=2.0 ** -22, err_msg=tag + " cos")
                np.testing.assert_allclose(sn, rs[:, 0], rtol=0, atol=2.0 ** -22, err_msg=tag + " sin")
        else:
            raise AssertionError(f"unhandled step {kind}")
    return results
