#!/usr/bin/env python3
"""Writes the full-size oracle fixtures of tests/golden/ (run from the repository root; each
configuration takes several minutes of CPU time).

Both fixtures run the oracle (oracle/oracle.c) on the 28-layer q4 group-64 decoder that the
decode benchmark builds (synth tag "bench-q4"), pinned by the sha256 of its .icua image:

oracle_c3_28layer.npz
    text context: 1024 random token ids (synth tag "c3-prompt"), prefill at slot 0, then 256
    greedy tokens (the first from the prefill), text-only M-RoPE.
oracle_c4_28layer.npz
    vision-shaped context (the benchmark's prompt, synth tag "bench-vis"): 16 text tokens, a
    32 x 32 grid of fp16 N(0, 1) visual rows with 3D M-RoPE and three DeepStack sets added after
    layers 0-2, then 3056 text tokens (4096 in all); then 128 greedy tokens.

Each holds the prompt, the greedy tokens with the oracle's top-1 logit and top-1 minus top-2 margin
per step, the first-token logits (float32, the whole vocabulary) and K / V rows of layers 0 and 27 at a few
cache slots (fp16 bit patterns [2][8][len(slots)][128]).

usage: python tests/golden/make_golden_28.py [c3] [c4]
"""
import hashlib
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

from instantcua_amd import synth  # noqa: E402
from instantcua_amd.modelfile import WeightFormat  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))

MODEL_TAG = "bench-q4"
LAYERS = 28
C3_PROMPT, C3_STEPS = 1024, 256
C4_PROMPT, C4_STEPS = 4096, 128
C4_VIS_OFFSET, C4_GRID = 16, (32, 32)
KV_LAYERS = (0, 27)


def c3_prompt() -> np.ndarray:
    return synth.random_tokens(C3_PROMPT, "c3-prompt")


def c4_prompt() -> synth.VisualPrompt:
    return synth.visual_prompt(C4_PROMPT, C4_VIS_OFFSET, C4_GRID[0], C4_GRID[1], tag="bench-vis")


def kv_slots(n_prompt: int, steps: int) -> np.ndarray:
    """Cache slots whose K/V rows the fixtures keep: prompt start, middle and end, the first
    decode slot and the last one a `steps`-token generation writes (slot n_prompt + steps - 2)."""
    last = n_prompt + steps - 2
    return np.array(sorted({0, 1, n_prompt // 2, n_prompt - 1, n_prompt, (n_prompt + last) // 2, last}),
                    dtype=np.int32)


def model_image() -> np.ndarray:
    return synth.build_model_image(WeightFormat.Q4, n_layers=LAYERS, tag=MODEL_TAG)


def _kv_rows(om, slots):
    out = np.empty((len(KV_LAYERS), 2, 8, len(slots), 128), dtype=np.uint16)
    for i, l in enumerate(KV_LAYERS):
        for kind in (0, 1):
            out[i, kind] = om.kv(l, kind)[:, slots, :].view(np.uint16)
    return out


def run(which: str, img: np.ndarray, sha: bytes) -> None:
    import oracle

    t0 = time.time()
    if which == "c3":
        toks, steps = c3_prompt(), C3_STEPS
        om = oracle.OracleModel(img, C3_PROMPT + steps + 8)
        out, margins, first, top1 = om.generate(toks, steps, with_top1=True)
        extra = {}
    else:
        vp, steps = c4_prompt(), C4_STEPS
        toks = vp.tokens
        om = oracle.OracleModel(img, C4_PROMPT + steps + 8)
        om.prepare_mrope(vp.vis_offset, vp.llm_h, vp.llm_w)
        out, margins, first, top1 = om.generate(toks, steps, pooler=vp.pooler.astype(np.float32),
                                                vis_offset=vp.vis_offset,
                                                deepstack=[d.astype(np.float32) for d in vp.deepstack],
                                                with_top1=True)
        extra = {"vis_offset": np.int32(vp.vis_offset), "grid": np.array([vp.llm_h, vp.llm_w], np.int32)}
    slots = kv_slots(toks.size, steps)
    np.savez_compressed(os.path.join(HERE, f"oracle_{which}_28layer.npz"),
                        image_sha256=np.frombuffer(sha, dtype=np.uint8), prompt=toks.astype(np.int32),
                        greedy=out, margins=margins, top1=top1, first_logits=first, kv_layers=np.array(KV_LAYERS, np.int32),
                        kv_slots=slots, kv=_kv_rows(om, slots), **extra)
    om.close()
    print(f"{which}: {steps} tokens in {time.time() - t0:.0f}s; first {list(out[:8])}", flush=True)


def main(argv):
    import oracle

    oracle.build()
    which = [a for a in argv if a in ("c3", "c4")] or ["c3", "c4"]
    t0 = time.time()
    img = model_image()
    sha = hashlib.sha256(img.tobytes()).digest()
    print(f"model image {img.nbytes / 1e6:.0f} MB in {time.time() - t0:.0f}s, sha256 {sha.hex()[:16]}", flush=True)
    for w in which:
        run(w, img, sha)


if __name__ == "__main__":
    main(sys.argv[1:])
