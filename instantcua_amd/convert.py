"""Hugging Face safetensors -> ``.icua`` converter for the language backbone.

Mirrors ``Converter`` of Sources/Engine/Convert.swift:

* ``SafeTensors`` (Convert.swift:8-68): a u64 header length, the JSON header, then raw tensors;
  BF16, F16 and F32 tensors are read as float32 (BF16 by a 16-bit shift, exact).
* ``quantize_q8`` / ``quantize_q4_raw`` (Convert.swift:214-320, ``quantizeQ8`` /
  ``quantizeQ4Raw``): run on the GPU by the engine library's ``icua_quantize`` kernels, bit-exact
  with the reference's float32 arithmetic.
* ``convert`` (Convert.swift:156-206): the language-backbone part of ``Converter.convert`` --
  embed_tokens, the final norm and, per layer, the four norm vectors and the fused q|k|v, o,
  gate|up and down matrices, in the given weight format.
* ``vision_tensors`` (Convert.swift:93-154): the vision tower and its four mergers, when the
  checkpoint holds them -- fp16 matrices, float32 biases, norms and position table, and the
  patch embedding with its two temporal slices summed in float32 (the image is one frame).
"""
from __future__ import annotations

import json
import os
import struct
from typing import Dict, Optional

import numpy as np

from . import engine as eng
from .modelfile import Dims, TensorID, WeightFormat, matrix_bytes, write_icua


class SafeTensors:
    """Read-only view of one ``.safetensors`` file (Convert.swift:8-68)."""

    def __init__(self, path: str):
        self.path = path
        self._mm = np.memmap(path, dtype=np.uint8, mode="r")
        if self._mm.size < 8:
            raise ValueError(f"{path}: not a safetensors file")
        n = struct.unpack("<Q", bytes(self._mm[:8]))[0]
        if 8 + n > self._mm.size:
            raise ValueError(f"{path}: header length {n} past the end of the file")
        header = json.loads(bytes(self._mm[8:8 + n]).decode("utf-8"))
        self.data_start = 8 + n
        self.entries: Dict[str, tuple] = {}
        for k, v in header.items():
            if k == "__metadata__":
                continue
            s, e = v["data_offsets"]
            self.entries[k] = (v["dtype"], tuple(v["shape"]), int(s), int(e))

    def floats(self, name: str) -> tuple[tuple, np.ndarray]:
        """(shape, float32 data) of tensor ``name`` (Convert.swift:43-67)."""
        if name not in self.entries:
            raise KeyError(f"missing tensor {name}")
        dtype, shape, s, e = self.entries[name]
        raw = self._mm[self.data_start + s:self.data_start + e]
        if dtype == "BF16":
            out = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        elif dtype == "F16":
            out = raw.view(np.float16).astype(np.float32)
        elif dtype == "F32":
            out = np.array(raw.view(np.float32))
        else:
            raise ValueError(f"{name}: unsupported dtype {dtype}")
        return shape, out


def write_safetensors(path: str, tensors: Dict[str, np.ndarray], dtype: str = "BF16") -> None:
    """Writes float32 arrays as one safetensors file, BF16 (truncated to the upper 16 bits after
    round-to-nearest-even), F16 or F32.  For building test inputs of the converter."""
    header, blobs, off = {}, [], 0
    for name, a in tensors.items():
        a = np.ascontiguousarray(a, dtype=np.float32)
        if dtype == "BF16":
            u = a.view(np.uint32).astype(np.uint64)
            b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        elif dtype == "F16":
            b = a.astype(np.float16)
        else:
            b = a
        blob = b.tobytes()
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + len(blob)]}
        blobs.append(blob)
        off += len(blob)
    hj = json.dumps(header).encode()
    hj += b" " * (-len(hj) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for blob in blobs:
            f.write(blob)


def _quantize(fmt: int, m: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    m = np.ascontiguousarray(m, dtype=np.float32)
    rows, cols = m.shape
    cb, sbb = matrix_bytes(fmt, rows, cols)
    dm = eng.DeviceBuffer.from_array(m)
    dc, ds = eng.DeviceBuffer(cb), eng.DeviceBuffer(sbb)
    try:
        eng._check(eng.lib().icua_quantize(fmt, dm.ptr, rows, cols, dc.ptr, ds.ptr))
        return dc.to_array(np.uint8, (cb,)), ds.to_array(np.uint8, (sbb,))
    finally:
        for b in (dm, dc, ds):
            b.free()


def quantize_q8(m: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """quantizeQ8 (Convert.swift:215-241): int8 codes [rows][cols], fp16 scales [rows][cols/32]."""
    rows, cols = m.shape
    c, s = _quantize(WeightFormat.Q8, m)
    return c.view(np.int8).reshape(rows, cols), s.view(np.uint16).reshape(rows, cols // 32)


def quantize_q4_raw(m: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """quantizeQ4Raw (Convert.swift:243-320): packed codes [rows][cols/2], fp16 (scale, bias)
    [rows][cols/64][2]."""
    rows, cols = m.shape
    c, s = _quantize(WeightFormat.Q4, m)
    return c.reshape(rows, cols // 2), s.view(np.uint16).reshape(rows, cols // 64, 2)


def _emit(fmt: int, m: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """emitMat (Convert.swift:157-171): (codes, scales) bytes of one matrix."""
    if fmt == WeightFormat.F16:
        return np.ascontiguousarray(m, dtype=np.float32).astype(np.float16).view(np.uint8).reshape(-1), \
            np.zeros(0, np.uint8)
    c, s = _quantize(fmt, m)
    return c, s


def vision_tensors(st: "SafeTensors") -> Dict[int, np.ndarray]:
    """The vision tower and mergers of Converter.convert (Convert.swift:93-154), by tensor id."""
    VH, VF, MH = Dims.vit_hidden, Dims.vit_ff, Dims.merger_hidden
    out: Dict[int, np.ndarray] = {}

    def f32(name, n):
        v = st.floats(name)[1]
        if v.size != n:
            raise ValueError(f"{name}: {v.size} values, expected {n}")
        return np.ascontiguousarray(v, dtype=np.float32)

    f16 = lambda name, n: f32(name, n).astype(np.float16)  # noqa: E731  Float16(x), nearest even
    pw = f32("model.visual.patch_embed.proj.weight", VH * 3 * 2 * 256).reshape(VH, 3, 2, 256)
    out[TensorID.vit_patch_w] = (pw[:, :, 0] + pw[:, :, 1]).astype(np.float16).reshape(-1)  # Convert.swift:97-112
    out[TensorID.vit_patch_b] = f32("model.visual.patch_embed.proj.bias", VH)
    out[TensorID.vit_pos_emb] = f32("model.visual.pos_embed.weight", Dims.vit_pos_grid ** 2 * VH)
    for l in range(Dims.vit_layers):
        p = f"model.visual.blocks.{l}."
        V = lambda k: TensorID.vit_layer(l, k)  # noqa: E731
        out[V(TensorID.v_norm1_w)] = f32(p + "norm1.weight", VH)
        out[V(TensorID.v_norm1_b)] = f32(p + "norm1.bias", VH)
        out[V(TensorID.v_qkv_w)] = f16(p + "attn.qkv.weight", Dims.vit_qkv_rows * VH)
        out[V(TensorID.v_qkv_b)] = f32(p + "attn.qkv.bias", Dims.vit_qkv_rows)
        out[V(TensorID.v_proj_w)] = f16(p + "attn.proj.weight", VH * VH)
        out[V(TensorID.v_proj_b)] = f32(p + "attn.proj.bias", VH)
        out[V(TensorID.v_norm2_w)] = f32(p + "norm2.weight", VH)
        out[V(TensorID.v_norm2_b)] = f32(p + "norm2.bias", VH)
        out[V(TensorID.v_fc1_w)] = f16(p + "mlp.linear_fc1.weight", VF * VH)
        out[V(TensorID.v_fc1_b)] = f32(p + "mlp.linear_fc1.bias", VF)
        out[V(TensorID.v_fc2_w)] = f16(p + "mlp.linear_fc2.weight", VH * VF)
        out[V(TensorID.v_fc2_b)] = f32(p + "mlp.linear_fc2.bias", VH)
    for i in range(Dims.num_deepstack + 1):
        p = f"model.visual.deepstack_merger_list.{i}." if i < Dims.num_deepstack else "model.visual.merger."
        nn = MH if i < Dims.num_deepstack else VH  # post-shuffle norm over 4096, final merger over 1024
        M = lambda k: TensorID.merger(i, k)  # noqa: E731
        out[M(TensorID.m_norm_w)] = f32(p + "norm.weight", nn)
        out[M(TensorID.m_norm_b)] = f32(p + "norm.bias", nn)
        out[M(TensorID.m_fc1_w)] = f16(p + "linear_fc1.weight", MH * MH)
        out[M(TensorID.m_fc1_b)] = f32(p + "linear_fc1.bias", MH)
        out[M(TensorID.m_fc2_w)] = f16(p + "linear_fc2.weight", Dims.hidden * MH)
        out[M(TensorID.m_fc2_b)] = f32(p + "linear_fc2.bias", Dims.hidden)
    return out


def convert(hf_dir: str, output: str, fmt: int, layers: Optional[int] = None, log=print) -> int:
    """Converter.convert (Convert.swift:83-206) for the language backbone; returns the file size.

    ``hf_dir`` holds ``model.safetensors``; ``layers`` defaults to the 28 of the model (fewer
    only for reduced test models)."""
    st = SafeTensors(os.path.join(hf_dir, "model.safetensors"))
    n_layers = Dims.layers if layers is None else int(layers)
    H, F, V = Dims.hidden, Dims.ff, Dims.vocab
    out: Dict[int, np.ndarray] = {}
    if "model.visual.patch_embed.proj.weight" in st.entries:
        out.update(vision_tensors(st))
        log("vision encoder & mergers done")

    def f32(name):
        return st.floats(name)[1]

    def mat(tid, tsb, data, rows, cols):
        if data.size != rows * cols:
            raise ValueError(f"tensor {tid}: {data.size} values, expected {rows} x {cols}")
        out[tid], out[tsb] = _emit(fmt, data.reshape(rows, cols))

    mat(TensorID.embed, TensorID.embed_sb, f32("model.language_model.embed_tokens.weight"), V, H)
    out[TensorID.final_norm] = f32("model.language_model.norm.weight")
    log("language embeddings done")
    for l in range(n_layers):
        p = f"model.language_model.layers.{l}."
        L = lambda k: TensorID.llm_layer(l, k)  # noqa: E731
        out[L(TensorID.attn_norm)] = f32(p + "input_layernorm.weight")
        out[L(TensorID.q_norm)] = f32(p + "self_attn.q_norm.weight")
        out[L(TensorID.k_norm)] = f32(p + "self_attn.k_norm.weight")
        out[L(TensorID.mlp_norm)] = f32(p + "post_attention_layernorm.weight")
        qkv = np.concatenate([f32(p + "self_attn.q_proj.weight"), f32(p + "self_attn.k_proj.weight"),
                              f32(p + "self_attn.v_proj.weight")])
        mat(L(TensorID.wqkv), L(TensorID.wqkv_sb), qkv, Dims.qkv_rows, H)
        mat(L(TensorID.wo), L(TensorID.wo_sb), f32(p + "self_attn.o_proj.weight"), H, H)
        gu = np.concatenate([f32(p + "mlp.gate_proj.weight"), f32(p + "mlp.up_proj.weight")])
        mat(L(TensorID.wgu), L(TensorID.wgu_sb), gu, Dims.gu_rows, H)
        mat(L(TensorID.wd), L(TensorID.wd_sb), f32(p + "mlp.down_proj.weight"), H, F)
        if (l + 1) % 7 == 0 or l == n_layers - 1:
            log(f"llm layer {l + 1}/{n_layers} done")
    size = write_icua(output, fmt, out)
    log(f"wrote {output} ({size} bytes)")
    return size
