"""Write ``tests/golden/cfg1_hf.npz``: Hugging Face transformers' Gemma4ForCausalLM outputs for
BASELINE config 1, the independent implementation the reference itself is pinned to
(tests/test_model_ops.py and tests/conftest.py of the reference).

Config 1: 4 layers (0-2 sliding W=16, 3 global), M=256, Hq=4, Hkv=1, D=64, V=1024, F=1024, no PLE,
no KV sharing, softcap 30, norms 1, layer_scalar 1. Weights: ``oracle.init_params(cfg, seed=0,
float32, std=0.02)`` (numpy PCG64, regenerated identically by the tests). Prompt: batch 2 x 24 ids
U[0, 1024) from ``default_rng(1)``. HF runs eager fp32 attention and recomputes the full sequence
each step (no cache), greedy for 32 steps; the ring of the sliding layers wraps (24 + 32 > 2*16).

Stored: ``prompt_ids [2, 24]``, ``tokens [2, 32]`` (greedy), ``logits [32, 2, 1024]`` (the
distribution each token was chosen from; step 0 = prefill's last position).
Run: ``python tests/golden/make_golden.py`` (CPU, a few seconds).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, str(HERE.parent))

from oracle import g4_oracle as O  # noqa: E402
import hf_util as H  # noqa: E402

STEPS = 32


def cfg1_params():
    cfg = O.config_from_hf(H.CFG1)
    return cfg, O.init_params(cfg, seed=0, dtype=O.F32, std=0.02)


def cfg1_prompt() -> np.ndarray:
    return np.random.default_rng(1).integers(0, 1024, (2, 24)).astype(np.int32)


def main() -> None:
    torch.set_grad_enabled(False)
    cfg, params = cfg1_params()
    model = H.build_hf_model(H.CFG1, seed=0)
    H.params_to_hf(model, params, cfg)
    ids = cfg1_prompt()
    seq = ids.copy()
    logits_all, tokens = [], []
    for _ in range(STEPS):
        pos = np.tile(np.arange(seq.shape[1]), (seq.shape[0], 1))
        lg = H.hf_logits(model, seq, pos=pos)[:, -1]
        tok = lg.argmax(-1).astype(np.int32)
        logits_all.append(lg)
        tokens.append(tok)
        seq = np.concatenate([seq, tok[:, None]], axis=1)
    np.savez_compressed(HERE / "cfg1_hf.npz", prompt_ids=ids, tokens=np.stack(tokens, 1),
                        logits=np.stack(logits_all).astype(np.float32))
    print("wrote", HERE / "cfg1_hf.npz")


if __name__ == "__main__":
    main()
