"""The ``.icua`` model file: layout constants, tensor ids, reader and writer.

Restates the reference container format (Sources/Engine/ModelFile.swift:6-196):

* a 16 KiB header: u32 magic ``0x31554349`` ("ICU1"), u32 version 1, u32 weight
  format (0 f16, 1 q8, 2 q4), u32 tensor count (710), then a table of
  ``(u64 offset, u64 size)`` pairs, one per tensor id (ModelFile.swift:113-115,
  139-148, 168-187);
* tensors in id order, each 256-byte aligned (ModelFile.swift:172-177);
* the file padded to a multiple of 16 KiB (ModelFile.swift:179).

Tensor ids follow ``TensorID`` (ModelFile.swift:62-111).  Only the language
backbone ids are read by the decoder; the vision ids stay empty in synthetic
files.  Quantised matrices are stored row-major ``[rows][K]`` with the codecs of
Sources/Engine/Convert.swift:157-171 (q8: 215-241, q4: 246-270).
"""
from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np

MAGIC = 0x31554349  # "ICU1", ModelFile.swift:113
VERSION = 1
HEADER_SIZE = 16384  # ModelFile.swift:114
PAGE_SIZE = 16384  # ModelFile.swift:115
ALIGN = 256  # ModelFile.swift:173


class WeightFormat:
    """ModelFile.swift:6-27."""

    F16 = 0
    Q8 = 1
    Q4 = 2
    NAMES = {0: "f16", 1: "q8", 2: "q4"}
    BY_NAME = {"f16": 0, "q8": 1, "q4": 2}


class Dims:
    """Language-backbone dimensions (ModelFile.swift:47-59)."""

    layers = 28
    hidden = 2048
    ff = 6144
    heads = 16
    kv_heads = 8
    head_dim = 128
    q_rows = 2048
    kv_rows = 1024
    qkv_rows = 4096
    gu_rows = 12288
    vocab = 151936
    rope_theta = 5_000_000.0
    eps = 1e-6
    vit_layers = 24
    num_deepstack = 3
    # Vision encoder (ModelFile.swift:31-45).
    vit_hidden = 1024
    vit_ff = 4096
    vit_heads = 16
    vit_head_dim = 64
    vit_qkv_rows = 3072
    vit_patch = 16
    vit_patch_dim = 768  # 3 x 16 x 16 (the temporal pair folded into the patch embedding)
    vit_pos_grid = 48
    deepstack_layers = (5, 11, 17)
    merger_hidden = 4096
    npatch_max = 1024


class TensorID:
    """Tensor-table indices (ModelFile.swift:62-111)."""

    vit_patch_w = 0  # [1024][768] f16
    vit_patch_b = 1  # [1024] f32
    vit_pos_emb = 2  # [2304][1024] f32
    vit_base = 3
    vit_per_layer = 12
    v_norm1_w, v_norm1_b, v_qkv_w, v_qkv_b, v_proj_w, v_proj_b = 0, 1, 2, 3, 4, 5
    v_norm2_w, v_norm2_b, v_fc1_w, v_fc1_b, v_fc2_w, v_fc2_b = 6, 7, 8, 9, 10, 11
    m_norm_w, m_norm_b, m_fc1_w, m_fc1_b, m_fc2_w, m_fc2_b = 0, 1, 2, 3, 4, 5
    merger_base = vit_base + Dims.vit_layers * vit_per_layer  # 291
    merger_per_unit = 6
    llm_base = merger_base + (Dims.num_deepstack + 1) * merger_per_unit  # 315
    embed = llm_base + 0
    embed_sb = llm_base + 1
    final_norm = llm_base + 2
    llm_layer_base = llm_base + 3  # 318
    llm_per_layer = 14
    attn_norm = 0
    wqkv, wqkv_sb = 1, 2
    q_norm, k_norm = 3, 4
    wo, wo_sb = 5, 6
    mlp_norm = 7
    wgu, wgu_sb = 8, 9
    wd, wd_sb = 10, 11
    count = llm_layer_base + Dims.layers * llm_per_layer  # 710

    @staticmethod
    def vit_layer(l: int, k: int) -> int:
        return TensorID.vit_base + l * TensorID.vit_per_layer + k

    @staticmethod
    def merger(i: int, k: int) -> int:
        """DeepStack mergers 0..2 and the final merger 3."""
        return TensorID.merger_base + i * TensorID.merger_per_unit + k

    @staticmethod
    def llm_layer(l: int, k: int) -> int:
        return TensorID.llm_layer_base + l * TensorID.llm_per_layer + k


def matrix_bytes(fmt: int, rows: int, cols: int) -> tuple[int, int]:
    """(code bytes, scale bytes) of one matrix (Convert.swift:157-171)."""
    if fmt == WeightFormat.Q4:
        return rows * cols // 2, rows * (cols // 64) * 4
    if fmt == WeightFormat.Q8:
        return rows * cols, rows * (cols // 32) * 2
    return rows * cols * 2, 0


def write_icua(path: str, fmt: int, tensors: Dict[int, bytes | np.ndarray]) -> int:
    """Write an ``.icua`` file; returns its length.

    Follows ``ModelWriter.write`` (ModelFile.swift:168-195): tensors in ascending
    id order, each placed at the next 256-byte boundary after the 16 KiB header,
    the total rounded up to 16 KiB.  Ids that are absent keep ``(0, 0)``.
    """
    table = [0] * (2 * TensorID.count)
    layout = []
    cursor = HEADER_SIZE
    for tid in sorted(tensors):
        blob = tensors[tid]
        nbytes = blob.nbytes if isinstance(blob, np.ndarray) else len(blob)
        cursor = (cursor + ALIGN - 1) & ~(ALIGN - 1)
        table[2 * tid] = cursor
        table[2 * tid + 1] = nbytes
        layout.append((cursor, blob))
        cursor += nbytes
    total = (cursor + PAGE_SIZE - 1) // PAGE_SIZE * PAGE_SIZE
    with open(path, "wb") as f:
        f.truncate(total)
        hdr = struct.pack("<IIII", MAGIC, VERSION, fmt, TensorID.count)
        hdr += struct.pack("<%dQ" % len(table), *table)
        f.seek(0)
        f.write(hdr)
        for off, blob in layout:
            f.seek(off)
            if isinstance(blob, np.ndarray):
                f.write(np.ascontiguousarray(blob).view(np.uint8).reshape(-1).data)
            else:
                f.write(blob)
    return total


@dataclass
class ModelFile:
    """Read-only mmap of an ``.icua`` file (ModelFile.swift:117-156)."""

    path: str
    fmt: int
    length: int
    _mm: mmap.mmap
    _table: np.ndarray

    @classmethod
    def open(cls, path: str) -> "ModelFile":
        size = os.path.getsize(path)
        if size < HEADER_SIZE or size % PAGE_SIZE:
            raise ValueError(f"{path}: bad size {size}")
        with open(path, "rb") as f:
            mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        magic, ver, fmt, count = struct.unpack_from("<IIII", mm, 0)
        if magic != MAGIC:
            raise ValueError(f"{path}: not an instantcua model")
        if ver != VERSION:
            raise ValueError(f"{path}: unsupported version")
        if fmt not in WeightFormat.NAMES:
            raise ValueError(f"{path}: unknown weight format")
        if count != TensorID.count:
            raise ValueError(f"{path}: tensor table mismatch")
        table = np.frombuffer(mm, dtype="<u8", count=2 * count, offset=16).reshape(count, 2)
        return cls(path, fmt, size, mm, table)

    def offset(self, tid: int) -> int:
        return int(self._table[tid, 0])

    def size(self, tid: int) -> int:
        return int(self._table[tid, 1])

    def array(self, tid: int, dtype) -> np.ndarray:
        dt = np.dtype(dtype)
        return np.frombuffer(self._mm, dtype=dt, count=self.size(tid) // dt.itemsize, offset=self.offset(tid))

    def num_layers(self) -> int:
        """Layers present: the first layer whose fused QKV tensor is empty ends the stack."""
        n = 0
        while n < Dims.layers and self.size(TensorID.llm_layer(n, TensorID.wqkv)) > 0:
            n += 1
        return n

    def close(self) -> None:
        """Unmaps the file; arrays returned by ``array`` must be released first."""
        self._table = None
        self._mm.close()
