#!/usr/bin/env python3
"""Writes the committed fixtures of tests/golden/ (run from the repository root).

codec_kat.npz   hand-built codec known answers: packed q4/q8 bytes, scales and the expected
                fp32 weights, computed here from the codec definitions (Convert.swift:215-262),
                not by the oracle.
oracle_1layer.npz
                outputs of the oracle on a seeded 1-layer q4 model: a fingerprint of the model
                image, the top-32 first-token logits (ids and values) and 8 greedy tokens with
                their top-2 margins.  Pins the oracle (and the synthetic generator) against drift.
"""
import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

from instantcua_amd import synth  # noqa: E402
from instantcua_amd.modelfile import WeightFormat  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def codec_kat():
    rng = np.random.default_rng(1234)
    # q4: 4 rows x K=128 (two groups per row)
    q = rng.integers(0, 16, size=(4, 128))
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    s = np.abs(rng.standard_normal((4, 2)) * 0.01).astype(np.float16)
    z = rng.integers(0, 16, size=(4, 2)).astype(np.float32)
    b = (-(s.astype(np.float32) * z)).astype(np.float16)
    sb = np.stack([s, b], axis=-1)  # [4][2 groups][scale, bias]
    w4 = (np.repeat(s.astype(np.float32), 64, 1) * q.astype(np.float32)
          + np.repeat(b.astype(np.float32), 64, 1)).astype(np.float32)
    # q8: 3 rows x K=64
    c8 = rng.integers(-127, 128, size=(3, 64)).astype(np.int8)
    s8 = (np.abs(rng.standard_normal((3, 2)) * 0.02) / 127).astype(np.float16)
    w8 = (np.repeat(s8.astype(np.float32), 32, 1) * c8.astype(np.float32)).astype(np.float32)
    np.savez(os.path.join(HERE, "codec_kat.npz"), q4_packed=packed, q4_sb=sb.reshape(-1).view(np.uint8),
             q4_w=w4, q8_codes=c8.view(np.uint8), q8_scales=s8.reshape(-1).view(np.uint8), q8_w=w8)


def oracle_1layer():
    import oracle

    oracle.build()
    img = synth.build_model_image(WeightFormat.Q4, n_layers=1, tag="golden-1layer")
    toks = synth.random_tokens(10, "golden-1layer")
    om = oracle.OracleModel(img, 64)
    out, margins, first = om.generate(toks, 8)
    top = np.argsort(first)[::-1][:32].astype(np.int32)
    np.savez(os.path.join(HERE, "oracle_1layer.npz"), image_sha256=np.frombuffer(
        hashlib.sha256(img.tobytes()).digest(), dtype=np.uint8), tokens=toks, top_ids=top,
        top_logits=first[top], greedy=out, margins=margins)


if __name__ == "__main__":
    codec_kat()
    oracle_1layer()
    print("wrote", os.listdir(HERE))
