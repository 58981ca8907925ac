"""Seeded synthetic models and inputs for the Qwen3-VL-2B-shaped decoder workloads.

No real checkpoint is available offline, so every workload runs on random-init
weights with the decoder's exact shapes, written in the ``.icua`` layout
(Sources/Engine/ModelFile.swift:62-111, 168-195) with the reference codecs
(Sources/Engine/Convert.swift:157-171, 215-270):

* q4 affine group-64: codes uniform in 0..15, packed ``pk[j] = q[2j] | q[2j+1] << 4``
  (Convert.swift:262); per group an fp16 pair ``(scale, bias)`` interleaved
  ``[row][K/64]`` (Convert.swift:260-261).  Scales are ``fp16(|N(0, 0.01)|)``,
  zero-points ``z`` uniform in 0..15, stored as the reference's bias
  ``b = fp16(-scale * z)`` so that ``w = scale * q + b``.
* q8 symmetric group-32: codes uniform in -127..127, scales
  ``fp16(|N(0, 0.02)| / 127)`` stored ``[row][K/32]`` (Convert.swift:215-241).
* f16: ``fp16(N(0, 0.05))``.

Norm weights (input/post-attention/final RMSNorm and per-head q/k norms) are
``fp32(1 + 0.1 N(0, 1))``; the workloads leave them unspecified and non-unit
values make every norm multiply observable in parity tests.

Every tensor has its own PCG64 stream seeded by ``(workload tag, layer, tensor id)``.
Because two independent uniform nibbles form a uniform byte, the q4 code bytes
are drawn directly as uniform bytes.
"""
from __future__ import annotations

import zlib
from dataclasses import dataclass
from typing import Optional

import numpy as np

from .modelfile import (ALIGN, HEADER_SIZE, MAGIC, PAGE_SIZE, VERSION, Dims, TensorID,
                        WeightFormat, matrix_bytes)

IMAGE_PAD_ID = 151655


def _rng(tag: str, layer: int, tid: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([zlib.crc32(tag.encode()), layer + 1, tid])))


def _layer_mats():
    """(slot, scale slot, rows, K) of the four fused matrices of one layer (Convert.swift:185-197)."""
    H, F = Dims.hidden, Dims.ff
    return [
        (TensorID.wqkv, TensorID.wqkv_sb, Dims.qkv_rows, H),
        (TensorID.wo, TensorID.wo_sb, H, H),
        (TensorID.wgu, TensorID.wgu_sb, Dims.gu_rows, H),
        (TensorID.wd, TensorID.wd_sb, H, F),
    ]


def model_tensor_sizes(fmt: int, n_layers: int) -> dict:
    """Byte size of every language-backbone tensor of an ``n_layers`` model."""
    H, V = Dims.hidden, Dims.vocab
    sizes = {}
    c, s = matrix_bytes(fmt, V, H)
    sizes[TensorID.embed] = c
    sizes[TensorID.embed_sb] = s
    sizes[TensorID.final_norm] = H * 4
    for l in range(n_layers):
        L = lambda k: TensorID.llm_layer(l, k)
        sizes[L(TensorID.attn_norm)] = H * 4
        sizes[L(TensorID.q_norm)] = Dims.head_dim * 4
        sizes[L(TensorID.k_norm)] = Dims.head_dim * 4
        sizes[L(TensorID.mlp_norm)] = H * 4
        for wid, sid, rows, cols in _layer_mats():
            c, s = matrix_bytes(fmt, rows, cols)
            sizes[L(wid)] = c
            sizes[L(sid)] = s
    return sizes


def _layout(sizes: dict):
    table = np.zeros((TensorID.count, 2), dtype="<u8")
    cursor = HEADER_SIZE
    for tid in sorted(sizes):
        cursor = (cursor + ALIGN - 1) & ~(ALIGN - 1)
        table[tid] = (cursor, sizes[tid])
        cursor += sizes[tid]
    total = (cursor + PAGE_SIZE - 1) // PAGE_SIZE * PAGE_SIZE
    return table, total


def fill_matrix(fmt: int, rows: int, cols: int, codes: np.ndarray, sb: np.ndarray, rng: np.random.Generator) -> None:
    """Fill code bytes and scale bytes (uint8 views) of one quantised matrix in place."""
    if fmt == WeightFormat.Q4:
        codes[:] = rng.integers(0, 256, size=codes.size, dtype=np.uint8)
        g = rows * (cols // 64)
        s = np.abs(rng.standard_normal(g, dtype=np.float32) * np.float32(0.01)).astype(np.float16)
        z = rng.integers(0, 16, size=g).astype(np.float32)
        b = (-(s.astype(np.float32) * z)).astype(np.float16)
        pair = sb.view(np.float16).reshape(g, 2)
        pair[:, 0] = s
        pair[:, 1] = b
    elif fmt == WeightFormat.Q8:
        codes.view(np.int8)[:] = rng.integers(-127, 128, size=codes.size, dtype=np.int8)
        g = rows * (cols // 32)
        s = (np.abs(rng.standard_normal(g, dtype=np.float32) * np.float32(0.02)) / np.float32(127)).astype(np.float16)
        sb.view(np.float16)[:] = s
    else:
        codes.view(np.float16)[:] = (rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(0.05)).astype(np.float16)


def _norm_weights(rng: np.random.Generator, n: int) -> np.ndarray:
    return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)


def build_model_image(fmt: int, n_layers: int = Dims.layers, tag: str = "model") -> np.ndarray:
    """Return a complete in-memory ``.icua`` image (uint8 array) of a synthetic decoder."""
    sizes = model_tensor_sizes(fmt, n_layers)
    table, total = _layout(sizes)
    img = np.zeros(total, dtype=np.uint8)
    hdr = np.array([MAGIC, VERSION, fmt, TensorID.count], dtype="<u4")
    img[:16] = hdr.view(np.uint8)
    img[16:16 + table.nbytes] = table.reshape(-1).view(np.uint8)

    def view(tid):
        off, n = int(table[tid, 0]), int(table[tid, 1])
        return img[off:off + n]

    H, V = Dims.hidden, Dims.vocab
    fill_matrix(fmt, V, H, view(TensorID.embed), view(TensorID.embed_sb), _rng(tag, -1, TensorID.embed))
    view(TensorID.final_norm).view(np.float32)[:] = _norm_weights(_rng(tag, -1, TensorID.final_norm), H)
    for l in range(n_layers):
        L = lambda k: TensorID.llm_layer(l, k)
        for slot, n in ((TensorID.attn_norm, H), (TensorID.q_norm, Dims.head_dim),
                        (TensorID.k_norm, Dims.head_dim), (TensorID.mlp_norm, H)):
            view(L(slot)).view(np.float32)[:] = _norm_weights(_rng(tag, l, L(slot)), n)
        for wid, sid, rows, cols in _layer_mats():
            fill_matrix(fmt, rows, cols, view(L(wid)), view(L(sid)), _rng(tag, l, L(wid)))
    return img


def save_image(img: np.ndarray, path: str) -> None:
    img.tofile(path)


# ---------------------------------------------------------------------------------------------
# Standalone quantised matrices (isolated dequant-GEMV sweep)

@dataclass
class QMatrix:
    fmt: int
    rows: int
    cols: int
    codes: np.ndarray  # uint8, codes bytes
    sb: np.ndarray  # uint8, scale bytes (may be empty for f16)


def make_matrix(fmt: int, rows: int, cols: int, tag: str = "gemv", index: int = 0) -> QMatrix:
    c, s = matrix_bytes(fmt, rows, cols)
    codes = np.empty(c, dtype=np.uint8)
    sb = np.empty(s, dtype=np.uint8)
    fill_matrix(fmt, rows, cols, codes, sb, _rng(tag, index, rows * 131071 + cols))
    return QMatrix(fmt, rows, cols, codes, sb)


def fp16_normal(shape, tag: str, index: int = 0) -> np.ndarray:
    """fp16 N(0, 1) activations / cache contents."""
    rng = _rng(tag, index, 7)
    return rng.standard_normal(shape, dtype=np.float32).astype(np.float16)


def random_tokens(n: int, tag: str, index: int = 0, vocab: int = Dims.vocab) -> np.ndarray:
    return _rng(tag, index, 11).integers(0, vocab, size=n).astype(np.int32)


# ---------------------------------------------------------------------------------------------
# Multimodal prompt shape (vision-context prefill)

@dataclass
class VisualPrompt:
    tokens: np.ndarray  # int32 [n], IMAGE_PAD_ID at the visual rows
    vis_offset: int
    llm_h: int
    llm_w: int
    pooler: np.ndarray  # fp16 [n_vis, H] visual embeddings
    deepstack: list  # 3 x fp16 [n_vis, H]


def visual_prompt(n_total: int, vis_offset: int, llm_h: int, llm_w: int, tag: str) -> VisualPrompt:
    """Text prefix, ``llm_h * llm_w`` image-pad rows, then random text to ``n_total`` tokens."""
    n_vis = llm_h * llm_w
    assert vis_offset + n_vis <= n_total
    toks = random_tokens(n_total, tag, 0)
    toks = np.where(toks == IMAGE_PAD_ID, 0, toks).astype(np.int32)
    toks[vis_offset:vis_offset + n_vis] = IMAGE_PAD_ID
    pooler = fp16_normal((n_vis, Dims.hidden), tag, 1)
    ds = [fp16_normal((n_vis, Dims.hidden), tag, 2 + i) for i in range(3)]
    return VisualPrompt(toks, vis_offset, llm_h, llm_w, pooler, ds)
