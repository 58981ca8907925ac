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


def vision_tensor_specs():
    """(slot, dtype, shape) of every vision-tower tensor (Convert.swift:97-152): fp16 matrices,
    float32 biases, norms and the position table."""
    VH, VF, MH = Dims.vit_hidden, Dims.vit_ff, Dims.merger_hidden
    specs = [(TensorID.vit_patch_w, np.float16, (VH, Dims.vit_patch_dim)),
             (TensorID.vit_patch_b, np.float32, (VH,)),
             (TensorID.vit_pos_emb, np.float32, (Dims.vit_pos_grid ** 2, VH))]
    for l in range(Dims.vit_layers):
        V = lambda k: TensorID.vit_layer(l, k)
        specs += [(V(TensorID.v_norm1_w), np.float32, (VH,)), (V(TensorID.v_norm1_b), np.float32, (VH,)),
                  (V(TensorID.v_qkv_w), np.float16, (Dims.vit_qkv_rows, VH)),
                  (V(TensorID.v_qkv_b), np.float32, (Dims.vit_qkv_rows,)),
                  (V(TensorID.v_proj_w), np.float16, (VH, VH)), (V(TensorID.v_proj_b), np.float32, (VH,)),
                  (V(TensorID.v_norm2_w), np.float32, (VH,)), (V(TensorID.v_norm2_b), np.float32, (VH,)),
                  (V(TensorID.v_fc1_w), np.float16, (VF, VH)), (V(TensorID.v_fc1_b), np.float32, (VF,)),
                  (V(TensorID.v_fc2_w), np.float16, (VH, VF)), (V(TensorID.v_fc2_b), np.float32, (VH,))]
    for i in range(Dims.num_deepstack + 1):
        M = lambda k: TensorID.merger(i, k)
        nn = MH if i < Dims.num_deepstack else VH  # DeepStack mergers normalise 4096 columns
        specs += [(M(TensorID.m_norm_w), np.float32, (nn,)), (M(TensorID.m_norm_b), np.float32, (nn,)),
                  (M(TensorID.m_fc1_w), np.float16, (MH, MH)), (M(TensorID.m_fc1_b), np.float32, (MH,)),
                  (M(TensorID.m_fc2_w), np.float16, (Dims.hidden, MH)),
                  (M(TensorID.m_fc2_b), np.float32, (Dims.hidden,))]
    return specs


def _fill_vision(view, tag: str, zero_blocks: bool = False) -> None:
    """Random vision weights: matrices fp16(N(0, 0.02)) (QKV 0.05, so that attention is peaked),
    biases N(0, 0.02), norm weights 1 + 0.1 N(0, 1), norm biases 0.1 N(0, 1), position table
    N(0, 0.2).  zero_blocks zeroes every block tensor (each block is then the identity)."""
    norm_w = {TensorID.v_norm1_w, TensorID.v_norm2_w}
    norm_b = {TensorID.v_norm1_b, TensorID.v_norm2_b}
    for tid, dt, shape in vision_tensor_specs():
        rng = _rng(tag + "-vision", 0, tid)
        n = int(np.prod(shape))
        in_block = TensorID.vit_base <= tid < TensorID.merger_base
        k = (tid - TensorID.vit_base) % TensorID.vit_per_layer if in_block else \
            (tid - TensorID.merger_base) % TensorID.merger_per_unit
        if in_block and zero_blocks:
            continue  # the image is zero-initialised
        if in_block and k in norm_w or not in_block and tid >= TensorID.merger_base and k == TensorID.m_norm_w:
            v = 1.0 + 0.1 * rng.standard_normal(n, dtype=np.float32)
        elif in_block and k in norm_b or not in_block and tid >= TensorID.merger_base and k == TensorID.m_norm_b:
            v = 0.1 * rng.standard_normal(n, dtype=np.float32)
        elif tid == TensorID.vit_pos_emb:
            v = 0.2 * rng.standard_normal(n, dtype=np.float32)
        elif dt == np.float16:
            sd = 0.05 if in_block and k == TensorID.v_qkv_w else 0.02
            v = sd * rng.standard_normal(n, dtype=np.float32)
        else:
            v = 0.02 * rng.standard_normal(n, dtype=np.float32)
        view(tid).view(dt)[:] = v.astype(dt)


def _layout(sizes: dict):
    table = np.zeros((TensorID.count, 2), dtype="<u8")
    cursor = HEADER_SIZE
    for tid in sorted(sizes):
        cursor = (cursor + ALIGN - 1) & ~(ALIGN - 1)
        table[tid] = (cursor, sizes[tid])
        cursor += sizes[tid]
    total = (cursor + PAGE_SIZE - 1) // PAGE_SIZE * PAGE_SIZE
    return table, total


def fill_matrix(fmt: int, rows: int, cols: int, codes: np.ndarray, sb: np.ndarray, rng: np.random.Generator,
                f16_bits: bool = False) -> None:
    """Fill code bytes and scale bytes (uint8 views) of one quantised matrix in place.  With
    f16_bits, f16 weights are random bit patterns of magnitude 2^-7 .. 2^-3 with a random sign and
    mantissa, the matrix tiled from one random 4 MiB block (an order of magnitude faster than
    normal values; for timing runs, where the values do not matter)."""
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
    elif f16_bits:
        bits = codes.view(np.uint16)
        block = np.frombuffer(rng.bytes(2 * min(bits.size, 1 << 21)), dtype=np.uint16) & np.uint16(0x8FFF)
        block |= np.uint16(0x2000)  # sign, exponent 8 .. 11 (2^-7 <= |w| < 2^-3), mantissa
        for i in range(0, bits.size, block.size):
            bits[i:i + block.size] = block[:bits.size - i]
    else:
        codes.view(np.float16)[:] = (rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(0.05)).astype(np.float16)


def _norm_weights(rng: np.random.Generator, n: int) -> np.ndarray:
    return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)


def tensor_view(img: np.ndarray, tid: int) -> np.ndarray:
    """Writable uint8 view of tensor `tid` of an in-memory ``.icua`` image."""
    table = img[16:16 + TensorID.count * 16].view("<u8").reshape(TensorID.count, 2)
    off, n = int(table[tid, 0]), int(table[tid, 1])
    return img[off:off + n]


def copy_embedding_row(img: np.ndarray, src: int, dst: int) -> None:
    """Gives token dst the codes and scales of token src in the tied embedding, so the lm_head
    logits of the two are bit-identical (an exact argmax tie)."""
    codes = tensor_view(img, TensorID.embed).reshape(Dims.vocab, -1)
    sb = tensor_view(img, TensorID.embed_sb).reshape(Dims.vocab, -1)
    codes[dst] = codes[src]
    sb[dst] = sb[src]


def build_model_image(fmt: int, n_layers: int = Dims.layers, tag: str = "model", vision: bool = False,
                      zero_vision_blocks: bool = False, f16_bits: bool = False) -> np.ndarray:
    """Return a complete in-memory ``.icua`` image (uint8 array) of a synthetic decoder, with the
    vision tower and its mergers when ``vision`` is set (f16_bits: see fill_matrix)."""
    sizes = model_tensor_sizes(fmt, n_layers)
    if vision:
        for tid, dt, shape in vision_tensor_specs():
            sizes[tid] = int(np.prod(shape)) * np.dtype(dt).itemsize
    table, total = _layout(sizes)
    img = np.zeros(total, dtype=np.uint8)
    hdr = np.array([MAGIC, VERSION, fmt, TensorID.count], dtype="<u4")
    img[:16] = hdr.view(np.uint8)
    img[16:16 + table.nbytes] = table.reshape(-1).view(np.uint8)

    def view(tid):
        off, n = int(table[tid, 0]), int(table[tid, 1])
        return img[off:off + n]

    H, V = Dims.hidden, Dims.vocab
    fill_matrix(fmt, V, H, view(TensorID.embed), view(TensorID.embed_sb), _rng(tag, -1, TensorID.embed), f16_bits)
    view(TensorID.final_norm).view(np.float32)[:] = _norm_weights(_rng(tag, -1, TensorID.final_norm), H)
    for l in range(n_layers):
        L = lambda k: TensorID.llm_layer(l, k)
        for slot, n in ((TensorID.attn_norm, H), (TensorID.q_norm, Dims.head_dim),
                        (TensorID.k_norm, Dims.head_dim), (TensorID.mlp_norm, H)):
            view(L(slot)).view(np.float32)[:] = _norm_weights(_rng(tag, l, L(slot)), n)
        for wid, sid, rows, cols in _layer_mats():
            fill_matrix(fmt, rows, cols, view(L(wid)), view(L(sid)), _rng(tag, l, L(wid)), f16_bits)
    if vision:
        _fill_vision(view, tag, zero_vision_blocks)
    return img


def random_rgb(gh: int, gw: int, tag: str, index: int = 0) -> np.ndarray:
    """RGB8 image [16 gh][16 gw][3]: smooth gradients plus uniform noise."""
    rng = _rng(tag, index, 13)
    y, x = np.mgrid[0:16 * gh, 0:16 * gw].astype(np.float32)
    base = np.stack([x / (16 * gw), y / (16 * gh), (x + y) / (16 * (gh + gw))], axis=-1) * 160.0
    return np.clip(base + rng.uniform(0, 96, base.shape), 0, 255).astype(np.uint8)


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


def scale_embedding_rows(img: np.ndarray, scales: dict) -> np.ndarray:
    """Copy of an image whose tied-embedding rows `tok` are multiplied by `c` (q4: their fp16
    (scale, bias) words; q8: their scales; f16: the values), so that those tokens win the argmax
    often: the grammar-pair workloads use it to make the forced pairs (Shaders.swift:1537-1561)
    fire on a random-init model."""
    img = img.copy()
    fmt = int(img[8:12].view("<u4")[0])
    table = np.frombuffer(img[16:16 + 16 * TensorID.count].tobytes(), dtype="<u8").reshape(-1, 2)
    if fmt == WeightFormat.F16:
        off = int(table[TensorID.embed, 0])
        rows = img[off:off + Dims.vocab * Dims.hidden * 2].view(np.float16).reshape(Dims.vocab, Dims.hidden)
    else:
        off = int(table[TensorID.embed_sb, 0])
        per_row = (Dims.hidden // 64) * 4 if fmt == WeightFormat.Q4 else (Dims.hidden // 32) * 2
        rows = img[off:off + Dims.vocab * per_row].view(np.float16).reshape(Dims.vocab, -1)
    for tok, c in scales.items():
        rows[tok] = (rows[tok].astype(np.float32) * c).astype(np.float16)
    return img
