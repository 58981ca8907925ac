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
