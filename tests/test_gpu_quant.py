"""GPU parity of the converter's quantisers and of the whole converter (Convert.swift:83-320):
bit-exact codes and scales against the oracle's restatement, through the C ABI."""
import os

import numpy as np
import pytest

from conftest import compare_greedy
from instantcua_amd import convert
from instantcua_amd.engine import Engine
from instantcua_amd.modelfile import Dims, ModelFile, TensorID, WeightFormat

pytestmark = pytest.mark.gpu


def edge_matrix(rows=96, cols=512, seed=7):
    """Rows of 64-groups that exercise every branch: constant, all-zero, tiny-range (no
    accepted candidate, carrying codes), exactly representable, one outlier, wide dynamic
    ranges up to fp16 overflow of the scale, fp16-subnormal scales."""
    rng = np.random.default_rng(seed)
    m = np.empty((rows, cols), np.float32)
    for r in range(rows):
        for g in range(cols // 64):
            kind = (r * 7 + g) % 10
            if kind == 0:
                w = np.full(64, rng.choice([0.0, 0.375, -3.0]))
            elif kind == 1:
                w = 1.0 + np.arange(64) * 1e-9 * rng.uniform(0.5, 2.0)
            elif kind == 2:
                q = rng.integers(0, 16, 64)
                w = q * 2.0 ** -6 - 0.25
            elif kind == 3:
                w = rng.uniform(-1, 1, 64)
                w[rng.integers(0, 64)] = rng.choice([-40.0, 40.0])
            elif kind == 4:
                w = rng.standard_normal(64) * 10.0 ** rng.uniform(-6, 4)
            elif kind == 5:
                w = rng.standard_normal(64) * 2e5
            elif kind == 6:
                w = rng.standard_normal(64) * 1e-7
            else:
                w = rng.standard_normal(64) * 0.02
            m[r, 64 * g:64 * g + 64] = w
    return m


@pytest.mark.parametrize("shape", [(96, 512), (130, 2048)])
def test_quantisers_match_the_oracle_on_edge_groups(oracle_mod, shape):
    m = edge_matrix(*shape)
    c8, s8 = convert.quantize_q8(m)
    r8, rs8 = oracle_mod.quant_q8(m)
    assert np.array_equal(c8, r8) and np.array_equal(s8, rs8)
    c4, s4 = convert.quantize_q4_raw(m)
    r4, rs4 = oracle_mod.quant_q4(m)
    assert np.array_equal(s4, rs4), f"{(s4 != rs4).sum()} (scale, bias) words differ"
    assert np.array_equal(c4, r4), f"{(c4 != r4).sum()} code bytes differ"


@pytest.mark.parametrize("rows,cols", [(Dims.hidden, Dims.ff), (Dims.qkv_rows, Dims.hidden)])
def test_quantisers_match_the_oracle_on_projection_shapes(oracle_mod, rows, cols):
    """Down [2048 x 6144] and QKV [4096 x 2048] matrices of N(0, 0.02) weights."""
    m = (np.random.default_rng(rows + cols).standard_normal((rows, cols)) * 0.02).astype(np.float32)
    for fmt, ours, ref in ((WeightFormat.Q8, convert.quantize_q8, oracle_mod.quant_q8),
                           (WeightFormat.Q4, convert.quantize_q4_raw, oracle_mod.quant_q4)):
        c, s = ours(m)
        rc, rsb = ref(m)
        assert np.array_equal(c, rc) and np.array_equal(s, rsb), WeightFormat.NAMES[fmt]


def _hf_model(path, rng):
    """A 1-layer Qwen3-VL-shaped language model in bf16 (HF tensor names of Convert.swift:172-199)."""
    H, F, V, HD = Dims.hidden, Dims.ff, Dims.vocab, Dims.head_dim
    t = {"model.language_model.embed_tokens.weight": rng.standard_normal((V, H), dtype=np.float32) * 0.05,
         "model.language_model.norm.weight": 1.0 + 0.1 * rng.standard_normal(H, dtype=np.float32)}
    p = "model.language_model.layers.0."
    for name, shape, sd in (("self_attn.q_proj.weight", (H, H), 0.02), ("self_attn.k_proj.weight", (1024, H), 0.02),
                            ("self_attn.v_proj.weight", (1024, H), 0.02), ("self_attn.o_proj.weight", (H, H), 0.02),
                            ("mlp.gate_proj.weight", (F, H), 0.02), ("mlp.up_proj.weight", (F, H), 0.02),
                            ("mlp.down_proj.weight", (H, F), 0.015)):
        t[p + name] = rng.standard_normal(shape, dtype=np.float32) * sd
    for name, n in (("input_layernorm.weight", H), ("post_attention_layernorm.weight", H),
                    ("self_attn.q_norm.weight", HD), ("self_attn.k_norm.weight", HD)):
        t[p + name] = 1.0 + 0.1 * rng.standard_normal(n, dtype=np.float32)
    convert.write_safetensors(os.path.join(path, "model.safetensors"), t, "BF16")


@pytest.fixture(scope="module")
def hf_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("hf")
    _hf_model(str(d), np.random.default_rng(11))
    return d


@pytest.mark.parametrize("fmt", [WeightFormat.Q4, WeightFormat.Q8])
def test_converted_model_matches_oracle(oracle_mod, hf_dir, fmt):
    """Converts a bf16 model, checks each matrix's bytes against the oracle's quantisation of
    the same bf16 weights (the embedding on three 64-row chunks), then decodes the converted
    file on the GPU and with the oracle."""
    d = hf_dir
    out = str(d / f"model_{WeightFormat.NAMES[fmt]}.icua")
    convert.convert(str(d), out, fmt, layers=1, log=lambda s: None)
    st = convert.SafeTensors(str(d / "model.safetensors"))
    mf = ModelFile.open(out)
    quant = oracle_mod.quant_q4 if fmt == WeightFormat.Q4 else oracle_mod.quant_q8
    try:
        assert mf.num_layers() == 1
        p = "model.language_model.layers.0."
        mats = {
            TensorID.llm_layer(0, TensorID.wqkv): np.concatenate(
                [st.floats(p + f"self_attn.{x}_proj.weight")[1] for x in "qkv"]).reshape(Dims.qkv_rows, -1),
            TensorID.llm_layer(0, TensorID.wo): st.floats(p + "self_attn.o_proj.weight")[1].reshape(Dims.hidden, -1),
            TensorID.llm_layer(0, TensorID.wgu): np.concatenate(
                [st.floats(p + f"mlp.{x}_proj.weight")[1] for x in ("gate", "up")]).reshape(Dims.gu_rows, -1),
            TensorID.llm_layer(0, TensorID.wd): st.floats(p + "mlp.down_proj.weight")[1].reshape(Dims.hidden, -1),
        }
        for tid, m in mats.items():
            rc, rs = quant(m)
            assert np.array_equal(mf.array(tid, np.uint8), rc.view(np.uint8).reshape(-1)), tid
            assert np.array_equal(mf.array(tid + 1, np.uint8), rs.view(np.uint8).reshape(-1)), tid + 1
        E = st.floats("model.language_model.embed_tokens.weight")[1].reshape(Dims.vocab, Dims.hidden)
        codes = np.array(mf.array(TensorID.embed, np.uint8))  # copies: the file's map is closed below
        sb = np.array(mf.array(TensorID.embed_sb, np.uint8))
        cpr = codes.size // Dims.vocab
        spr = sb.size // Dims.vocab
        for r0 in (0, 64 * 1111, Dims.vocab - 64):
            rc, rs = quant(E[r0:r0 + 64])
            assert np.array_equal(codes[r0 * cpr:(r0 + 64) * cpr], rc.view(np.uint8).reshape(-1)), r0
            assert np.array_equal(sb[r0 * spr:(r0 + 64) * spr], rs.view(np.uint8).reshape(-1)), r0
        norm = st.floats(p + "self_attn.k_norm.weight")[1]
        assert np.array_equal(mf.array(TensorID.llm_layer(0, TensorID.k_norm), np.float32), norm)
    finally:
        mf.close()

    img = np.fromfile(out, dtype=np.uint8)
    toks = np.random.default_rng(12).integers(0, Dims.vocab, 9).astype(np.int32)
    steps = 12
    om = oracle_mod.OracleModel(img, 64)
    ref, margins, first = om.generate(toks, steps)
    with Engine(flags=0, image=img, max_context=64, max_steps=steps) as e:
        e.eos = (-1, -1)
        e.prefill(toks, max_new=steps)
        e.decode_steps(steps - 1)
        got = e.tokens(e.state()["step"])
    n, note = compare_greedy(got, ref, margins, first.max() * np.ones(steps))
    print(f"{WeightFormat.NAMES[fmt]} converted model: {n}/{steps} greedy tokens identical ({note})")
