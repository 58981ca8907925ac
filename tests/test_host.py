"""CPU tests of the host side: the .icua format, the synthetic generator, the golden fixtures,
and the C ABI library (load, exported symbols, error paths that need no GPU)."""
import ctypes as C
import hashlib
import os
import re

import numpy as np
import pytest

from instantcua_amd import engine as eng
from instantcua_amd import modelfile as mf
from instantcua_amd import synth
from instantcua_amd.modelfile import Dims, TensorID, WeightFormat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def test_tensor_ids_match_reference_layout():
    # ModelFile.swift:62-111: 3 global vision + 24 x 12 ViT + 4 x 6 merger, then the LLM.
    assert TensorID.merger_base == 291
    assert TensorID.llm_base == 315
    assert (TensorID.embed, TensorID.embed_sb, TensorID.final_norm) == (315, 316, 317)
    assert TensorID.llm_layer_base == 318
    assert TensorID.count == 710
    assert TensorID.llm_layer(27, TensorID.wd_sb) == 318 + 27 * 14 + 11


def test_icua_roundtrip(tmp_path):
    p = str(tmp_path / "m.icua")
    blobs = {TensorID.embed: np.arange(1000, dtype=np.uint8), TensorID.final_norm: np.ones(7, np.float32),
             5: b"abc"}
    n = mf.write_icua(p, WeightFormat.Q8, blobs)
    assert n % mf.PAGE_SIZE == 0 and os.path.getsize(p) == n
    m = mf.ModelFile.open(p)
    assert m.fmt == WeightFormat.Q8
    for tid in blobs:
        assert m.offset(tid) % 256 == 0 and m.offset(tid) >= mf.HEADER_SIZE
    assert np.array_equal(m.array(TensorID.embed, np.uint8), blobs[TensorID.embed])
    assert np.array_equal(m.array(TensorID.final_norm, np.float32), blobs[TensorID.final_norm])
    assert bytes(m.array(5, np.uint8)) == b"abc"
    assert m.size(6) == 0 and m.num_layers() == 0
    m.close()


def test_icua_rejects_bad_files(tmp_path):
    p = str(tmp_path / "bad.icua")
    with open(p, "wb") as f:
        f.write(b"\0" * mf.HEADER_SIZE)
    with pytest.raises(ValueError, match="not an instantcua model"):
        mf.ModelFile.open(p)
    with open(p, "wb") as f:
        f.write(b"\0" * 100)
    with pytest.raises(ValueError, match="bad size"):
        mf.ModelFile.open(p)


def test_synthetic_image_layout_and_determinism():
    a = synth.build_model_image(WeightFormat.Q4, n_layers=1, tag="det")
    b = synth.build_model_image(WeightFormat.Q4, n_layers=1, tag="det")
    assert np.array_equal(a, b)
    tab = a[16:16 + TensorID.count * 16].view("<u8").reshape(-1, 2)
    L = lambda k: TensorID.llm_layer(0, k)
    assert tab[L(TensorID.wqkv), 1] == Dims.qkv_rows * Dims.hidden // 2
    assert tab[L(TensorID.wgu_sb), 1] == Dims.gu_rows * (Dims.hidden // 64) * 4
    assert tab[TensorID.llm_layer(1, TensorID.wqkv), 1] == 0
    # q4 bias = fp16(-scale * zero-point) with zero-points in 0..15: -b/s is (nearly) an integer
    off, n = tab[L(TensorID.wo_sb)]
    sb = a[off:off + n].view(np.float16).reshape(-1, 2).astype(np.float64)
    z = -sb[:, 1] / np.where(sb[:, 0] == 0, 1, sb[:, 0])
    ok = sb[:, 0] > 1e-3
    assert np.all(np.abs(z[ok] - np.round(z[ok])) < 0.02) and z[ok].min() > -0.5 and z[ok].max() < 15.5


def test_golden_codec_vectors_against_oracle(oracle_mod):
    g = np.load(os.path.join(GOLDEN, "codec_kat.npz"))
    w4 = oracle_mod.dequant(WeightFormat.Q4, g["q4_packed"].reshape(-1), g["q4_sb"], 4, 128)
    assert np.array_equal(w4.view(np.uint32), g["q4_w"].view(np.uint32))
    w8 = oracle_mod.dequant(WeightFormat.Q8, g["q8_codes"].reshape(-1), g["q8_scales"], 3, 64)
    assert np.array_equal(w8.view(np.uint32), g["q8_w"].view(np.uint32))


def test_golden_oracle_fingerprint(oracle_mod):
    g = np.load(os.path.join(GOLDEN, "oracle_1layer.npz"))
    img = synth.build_model_image(WeightFormat.Q4, n_layers=1, tag="golden-1layer")
    assert hashlib.sha256(img.tobytes()).digest() == g["image_sha256"].tobytes()
    om = oracle_mod.OracleModel(img, 64)
    out, margins, first = om.generate(g["tokens"], 8)
    assert np.array_equal(first[g["top_ids"]], g["top_logits"])
    assert np.array_equal(out, g["greedy"])
    assert np.array_equal(margins, g["margins"])


def test_bench_byte_model_matches_survey_figures():
    import bench

    # SURVEY/BASELINE: q4 g64 decode weights 968,249,344 B/token; KV 114,688 B per context slot
    assert bench.weight_bytes_per_token() == 968_249_344
    assert bench.kv_bytes_per_token(1) == 114_688
    assert bench.weight_bytes_per_token() + bench.kv_bytes_per_token(4096) == 1_438_011_392


# ------------------------------------------------------------------------------------------
# C ABI library (no GPU needed)

def _header_functions():
    names = set()
    for h in ("icua.h", "icua_tok.h"):
        with open(os.path.join(ROOT, "include", h)) as f:
            names |= set(re.findall(r"\b(icua_[a-z0-9_]+)\s*\(", f.read()))
    return sorted(names)


@pytest.fixture(scope="module")
def libicua():
    if not os.path.exists(eng.LIB_PATH):
        from instantcua_amd import build
        build.build()
    return eng.lib()


def test_library_exports_every_header_symbol(libicua):
    names = _header_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(libicua, n)]
    assert not missing, missing
    assert set(names) <= set(eng.EXPORTS)


def test_create_errors_without_gpu_work(libicua, tmp_path):
    h = C.c_void_p()
    rc = libicua.icua_engine_create(b"/nonexistent/model.icua", 2048, 512, 256, 0, C.byref(h))
    assert rc != 0 and b"cannot open" in libicua.icua_last_error()
    bad = tmp_path / "bad.icua"
    bad.write_bytes(b"\0" * mf.HEADER_SIZE)
    rc = libicua.icua_engine_create(str(bad).encode(), 2048, 512, 256, 0, C.byref(h))
    assert rc != 0 and b"not an instantcua model" in libicua.icua_last_error()
    with pytest.raises(eng.EngineError, match="tensor table mismatch|not an instantcua"):
        img = np.zeros(mf.HEADER_SIZE, np.uint8)
        img[:16] = np.array([mf.MAGIC, 1, 2, 5], dtype="<u4").view(np.uint8)
        eng.Engine(flags=0, image=img)


def test_noalloc_quantize_rejects_matrices_beyond_its_scratch(libicua):
    """The size check runs before any device work: 8,388,608 q4 groups is the static limit."""
    fake = C.c_void_p(256)  # never dereferenced: the call fails on the size first
    rc = libicua.icua_quantize_noalloc(2, fake, 262145, 2048, fake, fake)
    assert rc != 0 and b"exceed the static scratch of 8388608 groups" in libicua.icua_last_error()
