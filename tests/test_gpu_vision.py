"""GPU parity of the vision tower and its mergers (Engine.swift:317-473; Shaders.swift:59-454) and
of generateVision (Engine.swift:696-827) through the C ABI, against the oracle.

Tolerance: the tower's outputs (pooler and the three DeepStack sets, float32) within 1e-2 of the
oracle's largest magnitude, the bar stated for logits.  Both sides round to fp16 at the
reference engine's points; they differ in float32 accumulation order only."""
import numpy as np
import pytest

from conftest import compare_greedy
from instantcua_amd import synth
from instantcua_amd.engine import Engine, EngineError
from instantcua_amd.modelfile import WeightFormat

pytestmark = pytest.mark.gpu

TOL = 1e-2
PAD = synth.IMAGE_PAD_ID


@pytest.fixture(scope="module")
def vimg():
    return synth.build_model_image(WeightFormat.Q4, n_layers=1, tag="q4-vision", vision=True)


def rel(got, ref):
    return float(np.abs(got - ref).max() / np.abs(ref).max())


# 8 x 8: one 64-patch tile; 12 x 20: 240 patches, a partial last tile of queries and keys;
# 16 x 16: 256 patches, four whole tiles.
@pytest.mark.parametrize("gh,gw", [(8, 8), (12, 20), (16, 16)])
def test_tower_matches_oracle(oracle_mod, vimg, gh, gw):
    rgb = synth.random_rgb(gh, gw, "tower", 100 * gh + gw)
    ref_p, ref_ds = oracle_mod.vision(vimg, rgb)
    with Engine(flags=0, image=vimg, max_context=64, max_steps=4) as e:
        assert e.has_vision
        e.vision(rgb)
        assert e.last_timing["vision_ms"] > 0
        p, ds = e.visual_rows()
    errs = [rel(p, ref_p)] + [rel(d, r) for d, r in zip(ds, ref_ds)]
    print(f"grid {gh}x{gw}: pooler / deepstack max rel err {['%.2e' % x for x in errs]}")
    assert max(errs) < TOL, errs


def _prompt(nvis, tag):
    vis_offset = 5
    toks = synth.random_tokens(vis_offset + nvis + 6, tag)
    toks = np.where(toks == PAD, 0, toks).astype(np.int32)
    toks[vis_offset:vis_offset + nvis] = PAD
    return toks, vis_offset


def test_generate_vision_matches_oracle(oracle_mod, vimg):
    gh, gw = 8, 12
    rgb = synth.random_rgb(gh, gw, "genvis")
    toks, vis_offset = _prompt(gh * gw // 4, "genvis")
    steps = 10
    ref_p, ref_ds = oracle_mod.vision(vimg, rgb)
    om = oracle_mod.OracleModel(vimg, 128)
    om.prepare_mrope(vis_offset, gh // 2, gw // 2)
    ref, margins, first = om.generate(toks, steps, pooler=ref_p, vis_offset=vis_offset, deepstack=ref_ds)
    with Engine(flags=0, image=vimg, max_context=128, max_steps=steps) as e:
        e.eos = (-1, -1)
        got = e.generate_vision(rgb, toks, max_new_tokens=steps, write_first_logits=True)
        t = e.last_timing
        lg = e.logits(1)[0]  # writeFirstLogits (Engine.swift:697): the golden command's first logits
        p, ds = e.visual_rows()  # poolerBuf / deepstackBufs after the call
    err = float(np.abs(lg - first).max() / np.abs(first).max())
    assert err < 1e-2, err
    assert rel(p, ref_p) < TOL and max(rel(d, r) for d, r in zip(ds, ref_ds)) < TOL
    assert t["vision_ms"] > 0 and t["prefill_tokens"] == toks.size and t["generated_tokens"] == steps
    assert t["total_ms"] >= t["vision_ms"] + t["decode_ms"]
    n, note = compare_greedy(got, ref, margins, first.max() * np.ones(steps))
    print(f"generate_vision: {n}/{steps} greedy tokens identical ({note})")


def test_vision_delta_cache(vimg):
    gh, gw = 4, 6
    rgb = synth.random_rgb(gh, gw, "delta")
    toks, _ = _prompt(gh * gw // 4, "delta")
    with Engine(flags=0, image=vimg, max_context=64, max_steps=4) as e:
        e.eos = (-1, -1)
        e.use_vision_delta_cache = True
        a = e.generate_vision(rgb, toks, 4)
        assert e.last_timing["vision_ms"] > 0
        b = e.generate_vision(rgb, toks, 4)
        assert e.last_timing["vision_ms"] == 0 and a == b  # identical frame: encoder skipped
        rgb2 = rgb.copy()
        rgb2[-1, -1, 2] ^= 1  # last byte of the frame
        e.generate_vision(rgb2, toks, 4)
        assert e.last_timing["vision_ms"] > 0
        e.use_vision_delta_cache = False
        e.generate_vision(rgb2, toks, 4)
        assert e.last_timing["vision_ms"] > 0


def test_vision_errors(vimg):
    with Engine(flags=0, image=vimg, max_context=64, max_steps=4) as e:
        with pytest.raises(EngineError, match="multiples of 32"):
            e.vision(np.zeros((48, 64, 3), np.uint8))
        with pytest.raises(EngineError, match="1024 patches"):
            e.vision(np.zeros((32 * 17, 32 * 16, 3), np.uint8))
    img = synth.build_model_image(WeightFormat.Q4, n_layers=1, tag="q4-novision")
    with Engine(flags=0, image=img, max_context=64, max_steps=4) as e:
        assert not e.has_vision
        with pytest.raises(EngineError, match="no vision tower"):
            e.vision(np.zeros((64, 64, 3), np.uint8))


def test_text_generate_after_generate_vision(oracle_mod, vimg):
    """A text prompt after generate_vision on the same engine decodes with 1-D positions."""
    gh, gw = 4, 8
    rgb = synth.random_rgb(gh, gw, "vis-then-text")
    toks, _ = _prompt(gh * gw // 4, "vis-then-text")
    text = synth.random_tokens(20, "vis-then-text2")
    steps = 6
    om = oracle_mod.OracleModel(vimg, 64)
    ref, margins, first = om.generate(text, steps)
    with Engine(flags=0, image=vimg, max_context=64, max_steps=steps) as e:
        e.eos = (-1, -1)
        e.generate_vision(rgb, toks, max_new_tokens=steps)
        got = e.generate(text, max_new_tokens=steps)
    compare_greedy(got, ref, margins, first.max() * np.ones(steps))


def test_tower_matches_oracle_at_the_default_frame(vimg):
    """The reference's default 640 x 384 frame (24 x 40 patches: 960 patches in 15 whole 64-patch
    tiles, 240 visual rows) against tests/golden/oracle_vision_24x40.npz (make_golden_vision.py):
    every 15th row of the pooler and of each DeepStack set within TOL of the set's largest
    magnitude, and for every row the sum within 1e-3 of sqrt(2048 x sum of squares) and the sum
    of squares within 1e-2 relative."""
    import hashlib
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oracle_vision_24x40.npz")
    with np.load(path, allow_pickle=False) as z:
        fx = {k: z[k] for k in z.files}
    gh, gw = (int(v) for v in fx["grid"])
    assert hashlib.sha256(vimg.tobytes()).digest() == fx["image_sha256"].tobytes()
    rgb = synth.random_rgb(gh, gw, "tower-24x40")
    assert hashlib.sha256(np.ascontiguousarray(rgb).tobytes()).digest() == fx["rgb_sha256"].tobytes()
    with Engine(flags=0, image=vimg, max_context=64, max_steps=4) as e:
        e.vision(rgb)
        p, ds = e.visual_rows()
    sets = np.stack([p] + list(ds)).astype(np.float32)
    assert sets.shape == (4, gh * gw // 4, 2048)
    for i, name in enumerate(["pooler", "deepstack 0", "deepstack 1", "deepstack 2"]):
        got = sets[i][fx["rows"]]
        ref = fx["row_values"][i].astype(np.float32)
        err = float(np.abs(got - ref).max() / fx["max_abs"][i])
        s_err = float((np.abs(sets[i].sum(axis=1, dtype=np.float64) - fx["row_sum"][i])
                       / np.sqrt(2048.0 * fx["row_sumsq"][i])).max())
        q_err = float((np.abs((sets[i].astype(np.float64) ** 2).sum(axis=1) - fx["row_sumsq"][i])
                       / fx["row_sumsq"][i]).max())
        print(f"24x40 {name}: sampled rows {err:.2e}, row sums {s_err:.2e}, row sums of squares {q_err:.2e}")
        assert err < TOL and s_err < 1e-3 and q_err < 1e-2, (name, err, s_err, q_err)
