"""The converter's safetensors reader and writer (Convert.swift:8-68) -- CPU only."""
import json
import struct

import numpy as np
import pytest

from instantcua_amd.convert import SafeTensors, write_safetensors


def test_safetensors_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    a = rng.standard_normal((3, 64)).astype(np.float32)
    bf = (a.view(np.uint32) & 0xFFFF0000).view(np.float32)  # representable in bf16
    for dtype, src, want in (("BF16", bf, bf), ("F16", a, a.astype(np.float16).astype(np.float32)),
                             ("F32", a, a)):
        p = tmp_path / f"m_{dtype}.safetensors"
        write_safetensors(str(p), {"w": src, "v": src[0]}, dtype)
        st = SafeTensors(str(p))
        shape, got = st.floats("w")
        assert shape == (3, 64) and np.array_equal(got.reshape(3, 64), want)
        assert np.array_equal(st.floats("v")[1], want[0])


def test_bf16_writer_rounds_to_nearest_even(tmp_path):
    # 1 + 2^-8 is halfway between bf16 neighbours 1 and 1 + 2^-7: ties to the even one (1).
    v = np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(1.0 + 2.0 ** -9)], np.float32)
    p = tmp_path / "r.safetensors"
    write_safetensors(str(p), {"x": v}, "BF16")
    got = SafeTensors(str(p)).floats("x")[1]
    assert list(got) == [1.0, 1.0 + 2.0 ** -6, -1.0]


def test_reader_reads_the_reference_layout_and_rejects_unknown_dtypes(tmp_path):
    """Hand-built file: u64 header length, JSON with __metadata__, raw little-endian data."""
    data = np.array([1.5, -2.0], np.float32).tobytes() + np.array([7], np.int32).tobytes()
    hdr = {"__metadata__": {"format": "pt"},
           "a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
           "i": {"dtype": "I32", "shape": [1], "data_offsets": [8, 12]}}
    hj = json.dumps(hdr).encode()
    p = tmp_path / "h.safetensors"
    p.write_bytes(struct.pack("<Q", len(hj)) + hj + data)
    st = SafeTensors(str(p))
    assert list(st.floats("a")[1]) == [1.5, -2.0]
    with pytest.raises(ValueError, match="unsupported dtype I32"):
        st.floats("i")
    with pytest.raises(KeyError, match="missing tensor"):
        st.floats("nope")


def _hf_vision_sizes():
    """Element counts of the checkpoint's vision tensors (HF names of Convert.swift:97-152)."""
    sz = {"model.visual.patch_embed.proj.weight": 1024 * 3 * 2 * 256, "model.visual.patch_embed.proj.bias": 1024,
          "model.visual.pos_embed.weight": 2304 * 1024}
    for l in range(24):
        p = f"model.visual.blocks.{l}."
        sz.update({p + "norm1.weight": 1024, p + "norm1.bias": 1024, p + "attn.qkv.weight": 3072 * 1024,
                   p + "attn.qkv.bias": 3072, p + "attn.proj.weight": 1024 * 1024, p + "attn.proj.bias": 1024,
                   p + "norm2.weight": 1024, p + "norm2.bias": 1024, p + "mlp.linear_fc1.weight": 4096 * 1024,
                   p + "mlp.linear_fc1.bias": 4096, p + "mlp.linear_fc2.weight": 1024 * 4096,
                   p + "mlp.linear_fc2.bias": 1024})
    for i in range(4):
        p = f"model.visual.deepstack_merger_list.{i}." if i < 3 else "model.visual.merger."
        n = 4096 if i < 3 else 1024
        sz.update({p + "norm.weight": n, p + "norm.bias": n, p + "linear_fc1.weight": 4096 * 4096,
                   p + "linear_fc1.bias": 4096, p + "linear_fc2.weight": 2048 * 4096, p + "linear_fc2.bias": 2048})
    return sz


def test_vision_tensors_fold_and_types():
    """Convert.swift:93-154: the patch embedding's two temporal slices are summed in float32 then
    rounded to fp16; matrices fp16, biases / norms / positions float32; every slot the engine and
    the synthetic images use, with their sizes."""
    from instantcua_amd import convert, synth
    from instantcua_amd.modelfile import TensorID
    rng = np.random.default_rng(3)
    sizes = _hf_vision_sizes()
    special = {k: rng.standard_normal(sizes[k]).astype(np.float32) for k in (
        "model.visual.patch_embed.proj.weight", "model.visual.blocks.3.attn.qkv.weight",
        "model.visual.merger.norm.weight", "model.visual.deepstack_merger_list.2.norm.bias")}
    read = set()

    class FakeST:
        entries = sizes

        def floats(self, name):
            read.add(name)
            return None, special.get(name, np.zeros(sizes[name], np.float32))

    out = convert.vision_tensors(FakeST())
    assert read == set(sizes)
    specs = {tid: (dt, shape) for tid, dt, shape in synth.vision_tensor_specs()}
    assert set(out) == set(specs)
    for tid, (dt, shape) in specs.items():
        assert out[tid].dtype == dt and out[tid].size == int(np.prod(shape)), tid
    pw = special["model.visual.patch_embed.proj.weight"].reshape(1024, 3, 2, 256)
    folded = (pw[:, :, 0] + pw[:, :, 1]).astype(np.float16).reshape(-1)
    assert np.array_equal(out[TensorID.vit_patch_w].view(np.uint16), folded.view(np.uint16))
    q = special["model.visual.blocks.3.attn.qkv.weight"]
    assert np.array_equal(out[TensorID.vit_layer(3, TensorID.v_qkv_w)].view(np.uint16), q.astype(np.float16).view(np.uint16))
    assert np.array_equal(out[TensorID.merger(3, TensorID.m_norm_w)], special["model.visual.merger.norm.weight"])
    assert np.array_equal(out[TensorID.merger(2, TensorID.m_norm_b)],
                          special["model.visual.deepstack_merger_list.2.norm.bias"])
