#!/usr/bin/env python3
"""Writes tests/golden/oracle_pairs_28layer.npz: the reference's token loop with grammar pairs
(or_generate_commit, Shaders.swift:1531-1561) on the 28-layer q4 decoder of the decode benchmark
(synth tag "bench-q4", pinned by the sha256 of its .icua image) whose embedding rows of tokens 11
and 3678 are scaled by 8 (synth.scale_embedding_rows), so that forced pairs fire.

Two prompts (synth.random_tokens(n, "gram", 3)): n = 9 (short context: the pair's two rows fall
in different attention splits) and n = 600 (one split holds both rows and ~18 cached rows).
Each runs 24 tokens with grammar pairs on and no EOS.  Run from the repository root; a few
minutes of CPU time.

usage: python tests/golden/make_golden_pairs.py
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
SCALES = {11: 8.0, 3678: 8.0}
PROMPTS = (9, 600)
STEPS = 24


def main():
    import oracle

    oracle.build()
    t0 = time.time()
    base = synth.build_model_image(WeightFormat.Q4, n_layers=28, tag="bench-q4")
    sha = hashlib.sha256(base.tobytes()).digest()
    img = synth.scale_embedding_rows(base, SCALES)
    out = {"image_sha256": np.frombuffer(sha, dtype=np.uint8),
           "scales": np.array(list(SCALES.items()), dtype=np.float32)}
    for n in PROMPTS:
        toks = synth.random_tokens(n, "gram", 3)
        om = oracle.OracleModel(img, n + STEPS + 8)
        ref = np.array(om.generate_commit(toks, STEPS, grammar=True), dtype=np.int32)
        om.close()
        pairs = int(sum(1 for a, b in zip(ref, ref[1:]) if (a, b) == (11, 220)))
        print(f"prompt {n}: {ref.size} tokens, {pairs} pairs after 11, {time.time() - t0:.0f}s: {list(ref)}", flush=True)
        out[f"prompt_{n}"] = toks.astype(np.int32)
        out[f"tokens_{n}"] = ref
    np.savez_compressed(os.path.join(HERE, "oracle_pairs_28layer.npz"), **out)


if __name__ == "__main__":
    main()
