"""Full-size parity of the north-star workloads on the 28-layer q4 group-64 decoder of the decode
benchmark, against oracle fixtures committed under tests/golden/ (tests/golden/make_golden_28.py
wrote them; the oracle needs minutes of CPU time at these sizes):

* text context: a 1024-token prefill (one matrix-core chunk) and 255 decode steps through the
  persistent kernel, 256 greedy tokens in all;
* vision-shaped context: a 4096-token prefill (16 text tokens, a 32 x 32 grid of visual rows with
  3D M-RoPE and DeepStack after layers 0-2, 3056 text tokens) and 127 persistent decode steps.

Checked: the model image is the fixture's (sha256); first-token logits within 1e-4 (max |d| /
max |ref|, fp32 logits; the north-star tolerance is 1e-2, the kernels meet 4.5e-5 and 9.2e-6);
every one of the greedy tokens compared with the oracle's: a divergence is allowed only at an
oracle near-tie (margin below 1e-3 of that step's top-1 logit), after which the decode continues
teacher-forced from the oracle's token so the remaining steps are compared too; K/V cache rows
of layers 0 and 27 at prompt and decode slots within a bound scaled by the row (differences of
fp32 accumulation order carried through 28 layers and rounded to fp16).

Also here: one 4096-row matrix-core prefill chunk of a 2-layer model against the oracle run live."""
import hashlib
import os

import numpy as np
import pytest

from conftest import compare_greedy, compare_greedy_forced, rel_err
from instantcua_amd import synth
from instantcua_amd.engine import Engine
from instantcua_amd.modelfile import Dims, WeightFormat

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LAYERS = Dims.layers


def _fixture(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def model28():
    img = synth.build_model_image(WeightFormat.Q4, n_layers=LAYERS, tag="bench-q4")
    return img, hashlib.sha256(img.tobytes()).digest()


def _kv_bound_ok(got, ref, rel=2e-3):
    """|got - ref| <= rel * (the row's largest |ref|) + one fp16 ulp of ref, elementwise."""
    g = got.astype(np.float32)
    r = ref.astype(np.float32)
    d = np.abs(g - r)
    lim = rel * np.abs(r).max(axis=-1, keepdims=True) + np.spacing(np.abs(r).astype(np.float16)).astype(np.float32)
    return float((d / np.abs(r).max(axis=-1, keepdims=True)).max()), bool((d <= lim).all())


def _check(e, fx, steps, label):
    # The engine runs with grammar pairs on (the reference's setting).  The oracle's sequence
    # holds no token that fires a rule (")" = 8, 11, a first-step action), so it is also the
    # sequence under the rules.
    g = fx["greedy"]
    assert e.grammar_pairs and not ((g == 8) | (g == 11)).any()
    assert int(g[0]) not in (3678, 7241, 12476, 10855, 11862, 1339, 1472, 24769)
    lg = e.logits(1)[0]
    e.decode_steps(steps - 1)
    st = e.state()
    err = rel_err(lg, fx["first_logits"])
    assert st["step"] == steps and st["done"] == 1, st
    ties = compare_greedy_forced(e, fx["prompt"].size, g, fx["margins"], fx["top1"], steps)
    note = f"{label}: first-token logits rel err {err:.3g}; {steps}/{steps} greedy steps compared, " \
           f"oracle near-ties (teacher-forced past them) at steps {ties}"
    print(note)
    assert err < 1e-4, note
    # Decode step i writes the K/V row of token i - 1 at slot prompt + i - 1; after a near-tie the
    # decode was repeated from the oracle's token, so every row holds the oracle's sequence.
    slots = fx["kv_slots"]
    for i, l in enumerate(fx["kv_layers"]):
        for kind in (0, 1):
            got_rows = np.stack([e.read_kv(int(l), kind, int(s), 1)[:, 0] for s in slots], axis=1)
            ref_rows = fx["kv"][i, kind][:, :slots.size].view(np.float16)
            worst, ok = _kv_bound_ok(got_rows, ref_rows)
            print(f"{label}: layer {l} {'KV'[kind]} rows at slots {list(slots)}: max |d| / row max {worst:.3g}")
            assert ok, (int(l), kind, worst)


def test_text_context_1024_prefill_256_greedy(model28):
    img, sha = model28
    fx = _fixture("oracle_c3_28layer.npz")
    assert sha == fx["image_sha256"].tobytes(), "the synthetic model differs from the fixture's"
    toks = synth.random_tokens(1024, "c3-prompt")
    assert np.array_equal(toks, fx["prompt"])
    steps = fx["greedy"].size
    with Engine(image=img, max_context=toks.size + steps + 8, max_steps=steps) as e:
        e.eos = (-1, -1)
        assert e.persistent_decode
        e.prefill(toks, max_new=steps, write_logits=True)
        _check(e, fx, steps, "config 3")
        assert e.last_decode_persistent


def test_vision_context_4096_prefill_128_greedy(model28):
    img, sha = model28
    fx = _fixture("oracle_c4_28layer.npz")
    assert sha == fx["image_sha256"].tobytes(), "the synthetic model differs from the fixture's"
    vp = synth.visual_prompt(4096, 16, 32, 32, tag="bench-vis")
    assert np.array_equal(vp.tokens, fx["prompt"]) and int(fx["vis_offset"]) == vp.vis_offset
    steps = fx["greedy"].size
    with Engine(image=img, max_context=vp.tokens.size + steps + 8, max_steps=steps) as e:
        e.eos = (-1, -1)
        assert e.persistent_decode
        e.prepare_mrope(vp.vis_offset, vp.llm_h, vp.llm_w)
        e.set_visual(vp.pooler.astype(np.float32), [d.astype(np.float32) for d in vp.deepstack])
        e.prefill(vp.tokens, vis_offset=vp.vis_offset, max_new=steps, write_logits=True)
        _check(e, fx, steps, "config 4")
        assert e.last_decode_persistent


def test_prefill_chunk_of_4096_rows_matches_the_oracle(oracle_mod):
    """One full 4096-row matrix-core chunk (2 layers) against the oracle: first logits, K/V rows of
    the last layer at spread slots, and the first greedy tokens."""
    img = synth.build_model_image(WeightFormat.Q4, n_layers=2, tag="q4-small")
    toks = synth.random_tokens(4096, "chunk4096")
    steps = 4
    om = oracle_mod.OracleModel(img, 4096 + steps + 8)
    ref, margins, first = om.generate(toks, steps)
    slots = [0, 1, 63, 64, 2047, 4000, 4095]
    with Engine(flags=0, image=img, max_context=4096 + steps + 8, max_steps=steps) as e:
        e.eos = (-1, -1)
        e.prefill(toks, max_new=steps, write_logits=True)
        lg = e.logits(1)[0]
        assert e.last_timing["prefill_tokens"] == 4096
        kv = [np.stack([e.read_kv(1, kind, s, 1)[:, 0] for s in slots], axis=1) for kind in (0, 1)]
        e.decode_steps(steps - 1)
        got = e.tokens(steps)
    err = rel_err(lg, first)
    print(f"4096-row chunk: first-token logits rel err {err:.3g}")
    assert err < 1e-4, err
    for kind in (0, 1):
        ref_rows = om.kv(1, kind)[:, slots]
        worst, ok = _kv_bound_ok(kv[kind], ref_rows, rel=1e-4)
        print(f"4096-row chunk: layer 1 {'KV'[kind]} max |d| / row max {worst:.3g}")
        assert ok, worst
    compare_greedy(got, ref, margins, first.max() * np.ones(steps))


@pytest.mark.parametrize("n", [9, 600])
def test_grammar_pairs_28_layers_match_the_oracle_fixture(model28, n):
    """The reference's product setting on the 28-layer benchmark decoder: grammar pairs on, with
    the embedding rows of tokens 11 and 3678 scaled so that forced pairs fire (5 pairs in 24
    tokens).  Each pair runs as one two-row pass of the persistent kernel (pair_passes counts
    them); the tokens equal the oracle's token loop (tests/golden/make_golden_pairs.py).  With a
    9-token prompt the pair's two rows fall in different attention splits; with 600 one split
    holds both rows and ~18 cached rows."""
    img, sha = model28
    fx = _fixture("oracle_pairs_28layer.npz")
    assert sha == fx["image_sha256"].tobytes(), "the synthetic model differs from the fixture's"
    im = synth.scale_embedding_rows(img, {int(t): float(c) for t, c in fx["scales"]})
    toks, ref = fx[f"prompt_{n}"], [int(t) for t in fx[f"tokens_{n}"]]
    steps = len(ref)
    # Pairs whose pass runs: (11, 220) anywhere, or a step-1 action followed by 7, with the
    # forced token before the last step (a pair forced into the last step ends the loop).
    actions = (3678, 7241, 12476, 10855, 11862, 1339, 1472, 24769)
    pairs = sum(1 for i in range(steps - 2) if (ref[i], ref[i + 1]) == (11, 220) or
                (i == 0 and ref[0] in actions and ref[1] == 7))
    assert pairs >= 2, ref
    with Engine(image=im, max_context=n + steps + 8, max_steps=steps) as e:
        e.eos = (-1, -1)
        assert e.grammar_pairs and e.persistent_decode
        p0 = e.pair_passes
        got = e.generate(toks, max_new_tokens=steps)
        assert e.last_decode_persistent
        ran = e.pair_passes - p0
    print(f"grammar pairs, prompt {n}: {len(got)} tokens, {ran} two-row passes; identical: {got == ref}")
    assert got == ref, (got, ref)
    assert ran == pairs, (ran, pairs)
