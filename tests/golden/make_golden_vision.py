#!/usr/bin/env python3
"""Writes tests/golden/oracle_vision_24x40.npz: the oracle vision tower (oracle/vision.c) on the
reference's default 640 x 384 frame (a 24 x 40 patch grid: 960 patches, 240 merged visual rows)
of the synthetic q4 vision model (synth tag "q4-vision", one decoder layer), pinned by the sha256
of its .icua image and of the frame (synth.random_rgb(24, 40, "tower-24x40")).

The full outputs (pooler and three DeepStack sets, 240 x 2048 float32 each) would be 7.9 MB, so
the fixture keeps every 15th visual row of each set (16 rows, fp16) and, for all 240 rows of each
set, the float32 sum and sum of squares.  About a minute of CPU time.

usage: python tests/golden/make_golden_vision.py
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
GH, GW = 24, 40
ROW_STEP = 15


def main():
    import oracle

    oracle.build()
    oracle.set_threads(os.cpu_count() or 1)
    img = synth.build_model_image(WeightFormat.Q4, n_layers=1, tag="q4-vision", vision=True)
    rgb = synth.random_rgb(GH, GW, "tower-24x40")
    t0 = time.time()
    pooler, ds = oracle.vision(img, rgb)
    print(f"oracle tower {GH}x{GW}: {time.time() - t0:.1f}s", flush=True)
    sets = np.stack([pooler] + list(ds)).astype(np.float32)  # [4][240][2048]
    rows = np.arange(0, sets.shape[1], ROW_STEP)
    np.savez_compressed(
        os.path.join(HERE, "oracle_vision_24x40.npz"),
        image_sha256=np.frombuffer(hashlib.sha256(img.tobytes()).digest(), np.uint8),
        rgb_sha256=np.frombuffer(hashlib.sha256(np.ascontiguousarray(rgb).tobytes()).digest(), np.uint8),
        grid=np.array([GH, GW], np.int32), rows=rows.astype(np.int32),
        row_values=sets[:, rows].astype(np.float16),
        row_sum=sets.sum(axis=2, dtype=np.float64).astype(np.float32),
        row_sumsq=(sets.astype(np.float64) ** 2).sum(axis=2).astype(np.float32),
        max_abs=np.abs(sets).reshape(4, -1).max(axis=1).astype(np.float32))


if __name__ == "__main__":
    main()
