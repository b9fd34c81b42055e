"""The C-ABI library on the CPU: it loads, exports every symbol include/g4_rollout.h declares,
its host-side functions match the oracle, and invalid arguments are rejected with an error
code and message before any launch (no GPU needed: validation precedes every HIP call)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import hf_util as H
from oracle import g4_oracle as O

from gemma4_posttrain_jax_amd import _lib
from gemma4_posttrain_jax_amd import config as C

HEADER = Path(__file__).resolve().parents[1] / "include" / "g4_rollout.h"


def declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(g4_\w+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    assert names == set(_lib.PROTOTYPES), "ctypes prototypes and header declarations differ"
    for name in names:
        assert hasattr(lib, name), name
    assert lib.g4_version().startswith(b"g4rollout")


def test_ctypes_structs_match_the_compiled_header(tmp_path):
    """Size and every field offset of the ctypes mirrors equal what a C compiler lays out."""

    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for st in (_lib.G4AppendArgs, _lib.G4DecodeArgs, _lib.G4PrefillArgs, _lib.G4SampleArgs, _lib.G4SampleTopKArgs,
               _lib.G4LmHeadSampleArgs, _lib.G4LinearArgs, _lib.G4PrologueArgs, _lib.G4RolloutStepArgs):
        lines.append(f'printf("{st.__name__} size %zu\\n", sizeof({st.__name__}));')
        for f, _ in st._fields_:
            lines.append(f'printf("{st.__name__} {f} %zu\\n", offsetof({st.__name__}, {f}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([cc, str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    for line in filter(None, out):
        name, field, value = line.split()
        st = getattr(_lib, name)
        got = ctypes.sizeof(st) if field == "size" else getattr(st, field).offset
        assert got == int(value), f"{name}.{field}: ctypes {got} != C {value}"


@pytest.mark.parametrize("name", ["TINY_A", "TINY_B", "CFG1"])
def test_native_kv_source_layers_match_oracle(name):
    kw = getattr(H, name)
    ocfg, cfg = O.config_from_hf(kw), C.config_from_hf(kw)
    assert C.kv_source_layers(cfg) == [O.kv_source_layer(ocfg, i) for i in range(ocfg.num_hidden_layers)]


def test_native_kv_source_layers_e2b_like():
    types = [0, 0, 0, 0, 1] * 6
    got = _lib.kv_source_layers(types, 10)
    assert got[:20] == list(range(20))
    assert got[20:] == [18, 18, 18, 18, 19, 18, 18, 18, 18, 19]


def test_native_kv_source_layers_rejects_missing_source():
    with pytest.raises(_lib.G4Error, match="no non-shared layer"):
        _lib.kv_source_layers([1, 0, 0], 2)


@pytest.mark.parametrize("wc", [1, 7, 16, 512])
def test_native_ring_slot_positions_match_oracle(wc):
    for last in [-3, 0, 5, wc - 1, wc, 3 * wc + 1, 2047]:
        np.testing.assert_array_equal(_lib.ring_slot_positions(last, wc), O.ring_slot_positions(last, wc))


def _decode_args(**kw):
    base = dict(dtype=_lib.G4_DTYPE_BF16, kind=_lib.G4_CACHE_RING, batch=2, kv_heads=2, group=4, head_dim=256,
                capacity=512, slot_stride=512, window=512, q_pos_scalar=0, q_pos=None, key_mask=1,
                key_mask_stride=2048, q=1, cache_k=1, cache_vt=1, cache_k_w=1, new_k=None, new_v=None, out=1,
                workspace=None, workspace_bytes=0, prep=None, num_splits=0)
    base.update(kw)
    return _lib.G4DecodeArgs(**base)


@pytest.mark.parametrize("override,match", [
    (dict(dtype=7), "dtype"),
    (dict(kind=5), "kind"),
    (dict(group=17), "group"),
    (dict(head_dim=96), "head_dim"),
    (dict(slot_stride=500), "slot_stride"),
    (dict(window=0), "window"),
    (dict(q=None), "NULL"),
    (dict(new_k=1), "together"),
    (dict(kind=_lib.G4_CACHE_LINEAR, key_mask_stride=100), "key_mask_stride"),
    (dict(capacity=32768, slot_stride=32768, kind=_lib.G4_CACHE_LINEAR, key_mask_stride=32768,
          dtype=_lib.G4_DTYPE_F32), "too large"),
    (dict(num_splits=3), "num_splits"),
    (dict(num_splits=_lib.G4_DECODE_SPLIT_KEYS), "split-K needs"),
    (dict(num_splits=2, head_dim=128), "num_splits 2 with head_dim 128"),
    (dict(num_splits=-3), "num_splits"),
    (dict(num_splits=_lib.G4_DECODE_TWO_PASS, capacity=1040, slot_stride=1088, kind=_lib.G4_CACHE_LINEAR),
     "two-pass needs bf16"),
    (dict(num_splits=_lib.G4_DECODE_TWO_PASS, head_dim=64), "two-pass needs bf16"),
    (dict(num_splits=_lib.G4_DECODE_TWO_PASS, dtype=_lib.G4_DTYPE_F32), "two-pass needs bf16"),
])
def test_decode_rejects_invalid_arguments(override, match):
    a = _decode_args(**override)
    rc = _lib.lib().g4_decode_attention(ctypes.byref(a), None)
    assert rc in (-1, -2)
    assert re.search(match, _lib.lib().g4_last_error().decode())


def test_decode_split_keys_workspace():
    """Long rows over few pairs take the split-K path: the library reports its workspace and
    refuses to run without it."""

    L = _lib.lib()
    long_rows = dict(capacity=32768, slot_stride=32768, kind=_lib.G4_CACHE_LINEAR, key_mask_stride=32768, batch=16)
    a = _decode_args(**long_rows)
    need = L.g4_decode_workspace_size(ctypes.byref(a))
    n_splits = 32768 // 512
    assert need == 32 * 4 * 32768 * 2 + 32 * n_splits * 4 * 2 * 4 + 32 * n_splits * 4 * 256 * 4
    assert L.g4_decode_attention(ctypes.byref(a), None) == _lib.G4_ERR_WORKSPACE
    assert re.search("workspace", L.g4_last_error().decode())
    a = _decode_args(**long_rows, workspace=1, workspace_bytes=need - 1)
    assert L.g4_decode_attention(ctypes.byref(a), None) == _lib.G4_ERR_WORKSPACE
    # ring rows of 512 slots and one-pass choices need none
    assert L.g4_decode_workspace_size(ctypes.byref(_decode_args())) == 0
    assert L.g4_decode_workspace_size(ctypes.byref(_decode_args(**long_rows, num_splits=1))) == 0


def test_decode_prep_rejections():
    """The fused preparation runs only on the two-launch path and needs its inputs."""

    L = _lib.lib()
    prep = _lib.G4DecodePrep(q_raw=16, k_raw=16, v_raw=16, in_row_stride=12 * 256, q_norm_weight=16,
                             k_norm_weight=16, rope_cos=16, rope_sin=16, eps=1e-6, flags=0)
    pp = ctypes.cast(ctypes.pointer(prep), ctypes.c_void_p)
    cases = [
        (dict(prep=pp, head_dim=64), "two-launch path"),
        (dict(prep=pp, num_splits=2), "two-launch path"),
        (dict(prep=pp, new_k=16, new_v=16), "replaces new_k"),
    ]
    for kw, match in cases:
        a = _decode_args(**kw)
        assert L.g4_decode_attention(ctypes.byref(a), None) in (_lib.G4_ERR_INVALID, _lib.G4_ERR_UNSUPPORTED)
        assert re.search(match, L.g4_last_error().decode()), L.g4_last_error().decode()
    prep.in_row_stride = 100
    a = _decode_args(prep=pp)
    assert L.g4_decode_attention(ctypes.byref(a), None) == _lib.G4_ERR_INVALID
    assert re.search("in_row_stride", L.g4_last_error().decode())
    prep.in_row_stride, prep.flags, prep.q_norm_weight = 12 * 256, _lib.G4_APPEND_NORM_Q, None
    a = _decode_args(prep=pp)
    assert L.g4_decode_attention(ctypes.byref(a), None) == _lib.G4_ERR_INVALID
    assert re.search("flags", L.g4_last_error().decode())
    # with the preparation the library always asks for the two-launch workspace, also below 256 pairs
    prep.flags, prep.q_norm_weight = 0, 16
    assert L.g4_decode_workspace_size(ctypes.byref(_decode_args(prep=pp))) == 2 * 2 * 4 * 512 * 2


def test_decode_two_pass_workspace():
    """The two-launch path keeps bf16 scores [B * Hkv][R][512] in the workspace and refuses to run
    without enough of it."""

    L = _lib.lib()
    a = _decode_args(num_splits=_lib.G4_DECODE_TWO_PASS, batch=64)
    need = L.g4_decode_workspace_size(ctypes.byref(a))
    assert need == 64 * 2 * 4 * 512 * 2
    # rows of 513..1024 slots keep 1024-slot score rows; the automatic choice takes the path for
    # >= 256 (b, kv head) pairs and leaves fewer to the one-launch kernels (no workspace)
    linear = dict(kind=_lib.G4_CACHE_LINEAR, capacity=768, slot_stride=768, key_mask_stride=768)
    assert L.g4_decode_workspace_size(ctypes.byref(_decode_args(**linear, batch=128))) == 128 * 2 * 4 * 1024 * 2
    assert L.g4_decode_workspace_size(ctypes.byref(_decode_args(batch=127))) == 0
    assert L.g4_decode_workspace_size(ctypes.byref(_decode_args(batch=127, num_splits=1))) == 0
    assert L.g4_decode_attention(ctypes.byref(a), None) == _lib.G4_ERR_WORKSPACE
    assert re.search("two-pass needs .* workspace", L.g4_last_error().decode())
    a = _decode_args(num_splits=_lib.G4_DECODE_TWO_PASS, batch=64, workspace=1, workspace_bytes=need - 1)
    assert L.g4_decode_attention(ctypes.byref(a), None) == _lib.G4_ERR_WORKSPACE



def test_decode_head_dim_512_paths():
    """bf16 head dim 512 (the reference's default global head dim, model.py:66) has no one-launch
    kernel: rows of up to 1024 slots take the two-launch path at any pair count, longer rows the
    split-K path, and a one-pass split count is refused."""

    L = _lib.lib()
    a = _decode_args(head_dim=512, batch=1)  # 2 pairs, 512-slot ring
    assert L.g4_decode_workspace_size(ctypes.byref(a)) == 2 * 4 * 512 * 2
    linear = dict(kind=_lib.G4_CACHE_LINEAR, capacity=1000, slot_stride=1024, key_mask_stride=1024)
    assert L.g4_decode_workspace_size(ctypes.byref(_decode_args(head_dim=512, batch=1, **linear))) == 2 * 4 * 1024 * 2
    # 1040 slots: 3 splits of 512, scores + statistics + f32 partials of the 512 value dims
    long_rows = dict(kind=_lib.G4_CACHE_LINEAR, capacity=1040, slot_stride=1088, key_mask_stride=1088)
    splits = 3
    want = 2 * 4 * splits * 512 * 2 + 2 * splits * 4 * 2 * 4 + 2 * splits * 4 * 512 * 4
    assert L.g4_decode_workspace_size(ctypes.byref(_decode_args(head_dim=512, batch=1, **long_rows))) == want
    for n in (1, 2):
        assert L.g4_decode_attention(ctypes.byref(_decode_args(head_dim=512, num_splits=n)), None) == \
            _lib.G4_ERR_UNSUPPORTED
        assert re.search("head_dim 512 takes num_splits", L.g4_last_error().decode())


def _linear_args(**kw):
    base = dict(x=16, w=16, y=16, m=256, n=2048, k=8192, ldy=2048, ksplit=1, workspace=None, workspace_bytes=0,
                epilogue=_lib.G4_LINEAR_PLAIN)
    base.update(kw)
    return _lib.G4LinearArgs(**base)


@pytest.mark.parametrize("override,match", [
    (dict(x=None), "NULL"),
    (dict(m=257), "m 257"),
    (dict(m=0), "m 0"),
    (dict(n=100, ldy=100), "n 100"),
    (dict(k=8192 + 32), "k 8224"),
    (dict(ksplit=3), "k 8192 .* ksplit 3"),
    (dict(ksplit=0), "ksplit 0"),
    (dict(ldy=1024), "ldy"),
    (dict(y=18), "alignment"),
    (dict(ksplit=8), "workspace"),
    (dict(epilogue=2), "epilogue 2"),
    (dict(epilogue=_lib.G4_LINEAR_GELU_MUL, ksplit=2, workspace=16, workspace_bytes=1 << 30), "gated-GELU"),
    (dict(epilogue=_lib.G4_LINEAR_GELU_MUL, ldy=1020), "ldy 1020"),
])
def test_linear_rejects_invalid_arguments(override, match):
    a = _linear_args(**override)
    rc = _lib.lib().g4_linear_bf16(ctypes.byref(a), None)
    assert rc in (_lib.G4_ERR_INVALID, _lib.G4_ERR_UNSUPPORTED, _lib.G4_ERR_WORKSPACE)
    assert re.search(match, _lib.lib().g4_last_error().decode())


@pytest.mark.parametrize("override,match", [
    (dict(ksplit=9), "ksplit 9"),
    (dict(ksplit=0), "ksplit 0"),
    (dict(partials=None), "NULL"),
    (dict(partials=8), "aligned"),
    (dict(cols=4104), "cols 4104"),
    (dict(cols=12), "cols 12"),
])
def test_residual_norm_splitk_rejects_invalid_arguments(override, match):
    a = dict(rows=4, cols=2048, partials=16, ksplit=8, branch_weight=16, residual=16, scalar=None, next_weight=16,
             eps=1e-6, residual_out=16, next_out=16, stream=None)
    a.update(override)
    rc = _lib.lib().g4_residual_norm_splitk(*a.values())
    assert rc in (_lib.G4_ERR_INVALID, _lib.G4_ERR_UNSUPPORTED)
    assert re.search(match, _lib.lib().g4_last_error().decode())


def test_decode_prologue_rejects_invalid_arguments():
    L = _lib.lib()

    def args(**kw):
        base = dict(batch=2, hidden=64, vocab=10, key_mask_stride=8, tokens=16, positions=16, active=16, slot=16,
                    key_mask=16, embed=16, embed_scale=8.0, n_tables=1, x_out=16)
        base.update(kw)
        a = _lib.G4PrologueArgs(**base)
        a.rot_dim[0], a.inv_freq[0], a.cos_out[0], a.sin_out[0] = 64, 16, 16, 16
        return a

    for kw, match in [(dict(hidden=60), "hidden 60"), (dict(tokens=None), "NULL"), (dict(embed=8), "alignment"),
                      (dict(n_tables=3), "n_tables 3"), (dict(key_mask_stride=0), "key_mask_stride")]:
        assert L.g4_decode_prologue(ctypes.byref(args(**kw)), None) == _lib.G4_ERR_INVALID
        assert re.search(match, L.g4_last_error().decode())
    a = args()
    a.rot_dim[0] = 63
    assert L.g4_decode_prologue(ctypes.byref(a), None) == _lib.G4_ERR_INVALID
    assert re.search("rotary table 0", L.g4_last_error().decode())


def test_linear_workspace_size():
    L = _lib.lib()
    assert L.g4_linear_workspace_size(ctypes.byref(_linear_args())) == 0
    assert L.g4_linear_workspace_size(ctypes.byref(_linear_args(ksplit=8))) == 8 * 256 * 2048 * 4


def test_append_and_prefill_reject_invalid_arguments():
    L = _lib.lib()
    a = _lib.G4AppendArgs(dtype=_lib.G4_DTYPE_BF16, kind=_lib.G4_CACHE_LINEAR, batch=1, seq=10, kv_heads=1, group=0,
                          head_dim=64, capacity=8, slot_stride=64, k=1, v=1, cache_k=1, cache_vt=1, in_row_stride=64)
    assert L.g4_kv_append(ctypes.byref(a), None) == -1
    assert b"do not fit" in L.g4_last_error()
    a.seq, a.flags = 1, _lib.G4_APPEND_ROPE_K
    assert L.g4_kv_append(ctypes.byref(a), None) == -1
    assert b"RoPE" in L.g4_last_error()
    assert L.g4_kv_append(None, None) == -1
    p = _lib.G4PrefillArgs(dtype=_lib.G4_DTYPE_BF16, batch=1, seq=100, kv_heads=1, group=4, head_dim=64, window=0,
                           key_mask=1, key_mask_stride=100, q=1, k=1, vt=1, k_stride=100, out=1)
    assert L.g4_prefill_attention(ctypes.byref(p), None) == -1
    assert b"k_stride" in L.g4_last_error()
    p.k_stride, p.group = 128, 3
    assert L.g4_prefill_attention(ctypes.byref(p), None) == -2
    assert b"group" in L.g4_last_error()


def test_python_wrappers_fail_loudly_without_the_library(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "missing.so")
    with pytest.raises(_lib.G4Error, match="missing"):
        _lib.lib()


def _sample_args(**kw):
    base = dict(dtype=_lib.G4_DTYPE_BF16, batch=4, vocab=1000, proposal_width=0, logits=1, row_stride=1000,
                softcap=30.0, temperature=1.0, split_key=1, key=1, proposal=None, proposal_index=None,
                token_out=1, logp_out=1)
    base.update(kw)
    return _lib.G4SampleArgs(**base)


@pytest.mark.parametrize("override,match", [
    (dict(dtype=3), "dtype"),
    (dict(row_stride=999), "row_stride"),
    (dict(batch=0), "batch"),
    (dict(logits=None), "NULL"),
    (dict(softcap=-1.0), "softcap"),
    (dict(key=None), "key"),
    (dict(split_key=2), "split_key"),
    (dict(proposal=1, proposal_width=0), "proposal_width"),
    (dict(proposal=1, proposal_width=1001), "without proposal_index"),
    (dict(proposal_width=5), "without a proposal"),
])
def test_sample_rejects_invalid_arguments(override, match):
    a = _sample_args(**override)
    rc = _lib.lib().g4_sample_tokens(ctypes.byref(a), None)
    assert rc == _lib.G4_ERR_INVALID
    assert re.search(match, _lib.lib().g4_last_error().decode())


def _lm_head_args(**kw):
    base = dict(batch=256, vocab=262144, hidden=1536, x=16, embed=16, softcap=30.0, temperature=1.0, split_key=1,
                key=16, token_out=16, logp_out=16, logits_out=None, workspace=None, workspace_bytes=0)
    base.update(kw)
    return _lib.G4LmHeadSampleArgs(**base)


@pytest.mark.parametrize("override,match", [
    (dict(batch=0), "batch 0"),
    (dict(batch=257), "batch 257"),
    (dict(vocab=1000), "vocab 1000"),
    (dict(hidden=1540), "hidden 1540"),
    (dict(vocab=262144 * 8, hidden=1536), "4 GiB"),
    (dict(x=None), "NULL"),
    (dict(embed=8), "alignment"),
    (dict(logits_out=4), "alignment"),
    (dict(token_out=None), "neither"),
    (dict(logp_out=None), "logp_out"),
    (dict(softcap=-1.0), "softcap"),
    (dict(key=None), "key"),
    (dict(split_key=2), "split_key"),
])
def test_lm_head_sample_rejects_invalid_arguments(override, match):
    a = _lm_head_args(**override)
    rc = _lib.lib().g4_lm_head_sample(ctypes.byref(a), None)
    assert rc in (_lib.G4_ERR_INVALID, _lib.G4_ERR_UNSUPPORTED)
    assert re.search(match, _lib.lib().g4_last_error().decode())


def test_softcap_rejects_invalid_arguments():
    L = _lib.lib()
    for args, match in [((-1, 16, 30.0, 16), "n -1"), ((8, 16, 0.0, 16), "cap"), ((8, 16, float("inf"), 16), "cap"),
                        ((8, None, 30.0, 16), "NULL"), ((8, 18, 30.0, 16), "alignment")]:
        assert L.g4_softcap_bf16(*args, None) == _lib.G4_ERR_INVALID
        assert re.search(match, L.g4_last_error().decode())
    assert L.g4_softcap_bf16(0, None, 30.0, None, None) == 0


def test_convert_rejects_invalid_arguments():
    L = _lib.lib()
    assert L.g4_convert_f32_to_bf16(1, 1, -1, None, None) == _lib.G4_ERR_INVALID
    assert L.g4_convert_f32_to_bf16(None, 16, 8, None, None) == _lib.G4_ERR_INVALID
    assert L.g4_convert_f32_to_bf16(4, 16, 8, None, None) == _lib.G4_ERR_INVALID
    assert re.search("16-byte aligned", L.g4_last_error().decode())
    assert L.g4_convert_f32_to_bf16(None, None, 0, None, None) == _lib.G4_OK  # nothing to do
    assert L.g4_convert_bf16_to_f32(None, 16, 8, None) == _lib.G4_ERR_INVALID


def _rollout_step_args(**kw):
    base = dict(batch=4, max_new=8, step=0, pad_id=0, n_eos=1, id_bytes=4, eos_ids=16, sampled=16, logp=16,
                active=16, prompt_lengths=16, completion_ids=16, completion_mask=16, rollout_logps=16,
                next_token=16, next_pos=16, next_mask=16, any_active=16)
    base.update(kw)
    return _lib.G4RolloutStepArgs(**base)


@pytest.mark.parametrize("override,match", [
    (dict(batch=0), "batch 0"),
    (dict(step=8), "step 8"),
    (dict(step=-1), "step -1"),
    (dict(max_new=0), "max_new = 0"),
    (dict(id_bytes=2), "id_bytes 2"),
    (dict(eos_ids=None), "eos_ids"),
    (dict(n_eos=-1), "eos_ids"),
    (dict(sampled=None), "NULL"),
    (dict(prompt_lengths=None), "NULL"),
    (dict(id_bytes=8, completion_ids=20), "8-byte aligned"),
])
def test_rollout_step_rejects_invalid_arguments(override, match):
    a = _rollout_step_args(**override)
    rc = _lib.lib().g4_rollout_step(ctypes.byref(a), None)
    assert rc == _lib.G4_ERR_INVALID
    assert re.search(match, _lib.lib().g4_last_error().decode())


def _top_k_args(**kw):
    base = dict(dtype=_lib.G4_DTYPE_BF16, batch=4, vocab=1000, top_k=50, logits=16, row_stride=1000, softcap=30.0,
                temperature=1.0, top_p=0.9, split_key=1, key=16, token_out=16, logp_out=16)
    base.update(kw)
    return _lib.G4SampleTopKArgs(**base)


@pytest.mark.parametrize("override,match", [
    (dict(dtype=3), "dtype"),
    (dict(row_stride=999), "row_stride"),
    (dict(batch=0), "batch"),
    (dict(top_k=0), "top_k"),
    (dict(top_k=1000), "top_k"),
    (dict(top_k=257, vocab=4096, row_stride=4096), "top_k"),
    (dict(temperature=0.0), "temperature"),
    (dict(temperature=float("inf")), "temperature"),
    (dict(top_p=0.0), "top_p"),
    (dict(top_p=1.5), "top_p"),
    (dict(softcap=-1.0), "softcap"),
    (dict(key=None), "NULL"),
    (dict(logits=None), "NULL"),
    (dict(split_key=2), "split_key"),
])
def test_sample_top_k_rejects_invalid_arguments(override, match):
    a = _top_k_args(**override)
    rc = _lib.lib().g4_sample_top_k(ctypes.byref(a), None)
    assert rc in (_lib.G4_ERR_INVALID, _lib.G4_ERR_UNSUPPORTED)
    assert re.search(match, _lib.lib().g4_last_error().decode())
