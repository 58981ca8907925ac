"""GPU parity of the generate API's host semantics (Engine.swift:696-827): the commit rules with
grammar pairs and the ")" stop (Shaders.swift:1531-1561), the system-prompt KV prefix cache
(Engine.swift:719-735) and the timing record, through the C ABI."""
import numpy as np
import pytest

from conftest import compare_greedy
from instantcua_amd import synth
from instantcua_amd.synth import scale_embedding_rows
from instantcua_amd.engine import Engine
from instantcua_amd.modelfile import Dims, WeightFormat

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def grammar_base():
    return synth.build_model_image(WeightFormat.Q4, n_layers=2, tag="q4-grammar")


# (row scales, prompt seed, the rule the sequence must show)
GRAMMAR_CASES = [
    ({11: 8, 3678: 16, 8: 3}, 5, "step-1 action then 11"),
    ({11: 10, 3678: 10, 8: 4}, 2, "stop on )"),
    ({11: 8, 3678: 8, 8: 3}, 3, "11 pairs"),
]


@pytest.mark.parametrize("scales,seed,rule", GRAMMAR_CASES)
def test_grammar_pairs_match_the_oracle(oracle_mod, grammar_base, scales, seed, rule):
    img = scale_embedding_rows(grammar_base, scales)
    toks = synth.random_tokens(9, "gram", seed)
    steps = 20
    om = oracle_mod.OracleModel(img, 128)
    ref = [int(t) for t in om.generate_commit(toks, steps, grammar=True)]
    # The case exercises its rule.
    if rule == "step-1 action then 11":
        assert ref[:2] == [3678, 7] and any(a == 11 and b == 220 for a, b in zip(ref, ref[1:])), ref
    elif rule == "stop on )":
        assert ref[-1] == 8 and len(ref) < steps, ref
    else:
        assert sum(a == 11 and b == 220 for a, b in zip(ref, ref[1:])) >= 3, ref
    with Engine(flags=0, image=img, max_context=128, max_steps=steps) as e:
        e.eos = (-1, -1)
        e.grammar_pairs = True
        got = e.generate(toks, max_new_tokens=steps)
        st = e.state()
        assert e.last_decode_persistent  # the reference's normal setting stays on the fast path
        e.graph_decode = True
        got_graph = e.generate(toks, max_new_tokens=steps)
        assert not e.last_decode_persistent
    assert got == ref, (got, ref)
    assert got_graph == ref, (got_graph, ref)
    assert st["done"] == 1 and st["step"] == len(ref)


@pytest.mark.parametrize("scales,seed", [({11: 8, 3678: 8, 8: 3}, 2), ({11: 4, 3678: 8}, 4)])
def test_grammar_pairs_f16_match_the_oracle(oracle_mod, scales, seed):
    """f16 weights: single-row passes on the persistent kernel, each forced pair's two-row pass on
    the per-stage graph (the kernel has no two-row f16 form); both sequences force two pairs."""
    img = scale_embedding_rows(synth.build_model_image(WeightFormat.F16, n_layers=2, tag="f16-grammar"), scales)
    toks = synth.random_tokens(9, "gram", seed)
    steps = 20
    om = oracle_mod.OracleModel(img, 128)
    ref = [int(t) for t in om.generate_commit(toks, steps, grammar=True)]
    assert sum(a == 11 and b == 220 for a, b in zip(ref, ref[1:])) == 2, ref
    with Engine(flags=0, image=img, max_context=128, max_steps=steps) as e:
        e.eos = (-1, -1)
        e.grammar_pairs = True
        got = e.generate(toks, max_new_tokens=steps)
        assert e.last_decode_persistent
        assert e.pair_passes == 0  # the pairs ran on the graph
        e.prefill(toks, max_new=steps)
        for _ in range(steps):  # one pass per call: pairs pending between calls
            e.decode_steps(1)
        got_split = e.tokens(e.state()["step"])
    assert got == ref, (got, ref)
    assert list(got_split) == ref, (list(got_split), ref)


@pytest.mark.parametrize("scales,seed,n_pairs", [({11: 16, 3678: 16, 8: 4}, 4, 2), ({11: 24, 3678: 24, 8: 6}, 4, 1)])
def test_grammar_pairs_q8_match_the_oracle(oracle_mod, scales, seed, n_pairs):
    """q8 weights: single-row passes on the persistent kernel's slice-streaming form, each forced
    pair as a two-row pass of its register-tile form (the state handed between the two forms by
    the control block and the residual rows); the first sequence forces the step-1 action pair
    and an 11 pair, the second the action pair and then stops on ")"."""
    img = scale_embedding_rows(synth.build_model_image(WeightFormat.Q8, n_layers=2, tag="q8-grammar"), scales)
    toks = synth.random_tokens(9, "gram", seed)
    steps = 20
    om = oracle_mod.OracleModel(img, 128)
    ref = [int(t) for t in om.generate_commit(toks, steps, grammar=True)]
    assert ref[:2] == [3678, 7] and ref.count(220) + 1 == n_pairs, ref
    with Engine(flags=0, image=img, max_context=128, max_steps=steps) as e:
        e.eos = (-1, -1)
        e.grammar_pairs = True
        p0 = e.pair_passes
        got = e.generate(toks, max_new_tokens=steps)
        assert e.last_decode_persistent
        assert e.pair_passes - p0 == n_pairs  # each pair as one two-row persistent pass
        e.prefill(toks, max_new=steps)
        for _ in range(steps):  # one pass per call: pairs pending between calls
            if e.state()["done"]:
                break
            e.decode_steps(1)
        got_split = e.tokens(e.state()["step"])
    assert got == ref, (got, ref)
    assert list(got_split) == ref, (list(got_split), ref)


@pytest.mark.parametrize("split", [1, 2, 3])
def test_grammar_pairs_across_decode_calls(oracle_mod, grammar_base, split):
    """A forced pair left pending at the end of a decode call (state n = 2) continues in the next
    call: decode in calls of `split` steps and compare with the oracle's loop."""
    img = scale_embedding_rows(grammar_base, {11: 8, 3678: 8, 8: 3})
    toks = synth.random_tokens(9, "gram", 3)
    steps = 16
    om = oracle_mod.OracleModel(img, 128)
    ref = [int(t) for t in om.generate_commit(toks, steps, grammar=True)]
    assert any(a == 11 and b == 220 for a, b in zip(ref, ref[1:])), ref
    with Engine(flags=0, image=img, max_context=128, max_steps=steps) as e:
        e.eos = (-1, -1)
        e.grammar_pairs = True
        e.prefill(toks, max_new=steps)
        for _ in range(4 * steps):
            st = e.state()
            if st["done"]:
                break
            e.decode_steps(split)
            assert e.last_decode_persistent
        st = e.state()
        got = [int(t) for t in e.tokens(st["step"])]
    assert got == ref, (got, ref)


def test_without_grammar_pairs_no_token_is_forced(oracle_mod, grammar_base):
    """The same model without the flag: plain greedy, ")" does not stop, nothing is forced."""
    img = scale_embedding_rows(grammar_base, {11: 8, 3678: 16, 8: 3})
    toks = synth.random_tokens(9, "gram", 5)
    steps = 12
    om = oracle_mod.OracleModel(img, 128)
    ref = [int(t) for t in om.generate_commit(toks, steps, grammar=False)]
    assert ref[0] == 3678 and ref[1] != 7
    with Engine(flags=0, image=img, max_context=128, max_steps=steps) as e:
        e.eos = (-1, -1)
        got = e.generate(toks, max_new_tokens=steps)
    assert got == ref


@pytest.fixture(scope="module")
def q4_small():
    return synth.build_model_image(WeightFormat.Q4, n_layers=2, tag="q4-small")


def test_prefix_cache_reuses_the_system_prompt(oracle_mod, q4_small):
    """Two prompts with the same text prefix before the image: the second prefills only from the
    first image row, and decodes the tokens of a fresh engine and of the oracle."""
    vp1 = synth.visual_prompt(40, vis_offset=6, llm_h=4, llm_w=4, tag="pfx1")
    vp2 = synth.visual_prompt(44, vis_offset=6, llm_h=4, llm_w=4, tag="pfx2")
    vp2.tokens[:6] = vp1.tokens[:6]
    steps = 10
    ds2 = [d.astype(np.float32) for d in vp2.deepstack]
    with Engine(flags=0, image=q4_small, max_context=128, max_steps=steps) as e:
        e.eos = (-1, -1)
        e.use_prefix_cache = True
        e.prepare_mrope(vp1.vis_offset, vp1.llm_h, vp1.llm_w)
        e.set_visual(vp1.pooler.astype(np.float32), [d.astype(np.float32) for d in vp1.deepstack])
        first = e.generate(vp1.tokens, vis_offset=vp1.vis_offset, max_new_tokens=steps)
        t1 = e.last_timing
        e.prepare_mrope(vp2.vis_offset, vp2.llm_h, vp2.llm_w)
        e.set_visual(vp2.pooler.astype(np.float32), ds2)
        cached = e.generate(vp2.tokens, vis_offset=vp2.vis_offset, max_new_tokens=steps)
        t2 = e.last_timing
    assert len(first) == steps and t1["prefill_tokens"] == 40
    assert t2["prefill_tokens"] == 44 - 6, t2
    with Engine(flags=0, image=q4_small, max_context=128, max_steps=steps) as e:
        e.eos = (-1, -1)
        e.prepare_mrope(vp2.vis_offset, vp2.llm_h, vp2.llm_w)
        e.set_visual(vp2.pooler.astype(np.float32), ds2)
        fresh = e.generate(vp2.tokens, vis_offset=vp2.vis_offset, max_new_tokens=steps)
        assert e.last_timing["prefill_tokens"] == 44
    assert cached == fresh
    om = oracle_mod.OracleModel(q4_small, 128)
    om.prepare_mrope(vp2.vis_offset, vp2.llm_h, vp2.llm_w)
    ref, margins, lg = om.generate(vp2.tokens, steps, pooler=vp2.pooler.astype(np.float32),
                                   vis_offset=vp2.vis_offset, deepstack=ds2)
    compare_greedy(np.array(cached), ref, margins, lg.max() * np.ones(steps))


def test_prefix_cache_misses_on_a_new_prefix(q4_small):
    vp1 = synth.visual_prompt(30, vis_offset=4, llm_h=2, llm_w=4, tag="pfx3")
    vp2 = synth.visual_prompt(30, vis_offset=4, llm_h=2, llm_w=4, tag="pfx4")
    with Engine(flags=0, image=q4_small, max_context=64, max_steps=4) as e:
        e.eos = (-1, -1)
        e.use_prefix_cache = True
        for vp, want in ((vp1, 30), (vp2, 30), (vp2, 26)):
            e.prepare_mrope(vp.vis_offset, vp.llm_h, vp.llm_w)
            e.set_visual(vp.pooler.astype(np.float32), None)
            e.generate(vp.tokens, vis_offset=vp.vis_offset, max_new_tokens=4)
            assert e.last_timing["prefill_tokens"] == want


def test_generate_timing_record(q4_small):
    toks = synth.random_tokens(12, "timing")
    with Engine(flags=0, image=q4_small, max_context=64, max_steps=16) as e:
        e.eos = (-1, -1)
        out = e.generate(toks, max_new_tokens=16)
        t = e.last_timing
    assert len(out) == 16 and t["generated_tokens"] == 16 and t["prefill_tokens"] == 12
    assert t["prefill_ms"] > 0 and t["decode_ms"] > 0 and t["vision_ms"] == 0
    assert t["total_ms"] >= t["decode_ms"]


def test_prefix_cache_survives_failed_calls_and_text_prompts(oracle_mod, q4_small):
    """The prefix key names only K/V rows the cache holds: a call that fails validation leaves it
    alone, a text prompt (which rewrites slots 0..) clears it, and every output still equals the
    oracle's."""
    from instantcua_amd.engine import EngineError

    vp1 = synth.visual_prompt(30, vis_offset=5, llm_h=2, llm_w=4, tag="pfx5")
    vp2 = synth.visual_prompt(30, vis_offset=5, llm_h=2, llm_w=4, tag="pfx6")
    text = synth.random_tokens(20, "pfx-text")
    steps = 6
    pool1 = vp1.pooler.astype(np.float32)
    om = oracle_mod.OracleModel(q4_small, 64)
    om.prepare_mrope(vp1.vis_offset, vp1.llm_h, vp1.llm_w)
    ref_vis, m_vis, lg_vis = om.generate(vp1.tokens, steps, pooler=pool1, vis_offset=vp1.vis_offset)
    om.prepare_mrope(-1, 1, 1)
    ref_txt, m_txt, lg_txt = om.generate(text, steps)
    with Engine(flags=0, image=q4_small, max_context=64, max_steps=steps) as e:
        e.eos = (-1, -1)
        e.use_prefix_cache = True
        e.prepare_mrope(vp1.vis_offset, vp1.llm_h, vp1.llm_w)
        e.set_visual(pool1, None)
        a = e.generate(vp1.tokens, vis_offset=vp1.vis_offset, max_new_tokens=steps)
        assert e.last_timing["prefill_tokens"] == 30
        bad = vp2.tokens.copy()
        bad[-1] = Dims.vocab  # out of range: rejected before any K/V row is written
        with pytest.raises(EngineError, match="out of range"):
            e.generate(bad, vis_offset=vp2.vis_offset, max_new_tokens=steps)
        with pytest.raises(EngineError, match="vis_offset"):
            e.generate(vp1.tokens[:4], vis_offset=vp1.vis_offset, max_new_tokens=steps)
        b = e.generate(vp1.tokens, vis_offset=vp1.vis_offset, max_new_tokens=steps)
        assert e.last_timing["prefill_tokens"] == 30 - 5  # hit: the failed calls kept the key
        t = e.generate(text, max_new_tokens=steps)  # text-only: rewrites slots 0..19
        e.prepare_mrope(vp1.vis_offset, vp1.llm_h, vp1.llm_w)
        c = e.generate(vp1.tokens, vis_offset=vp1.vis_offset, max_new_tokens=steps)
        assert e.last_timing["prefill_tokens"] == 30  # miss: the text prompt cleared the key
    for got in (a, b, c):
        compare_greedy(np.array(got), ref_vis, m_vis, lg_vis.max() * np.ones(steps))
    compare_greedy(np.array(t), ref_txt, m_txt, lg_txt.max() * np.ones(steps))


def test_text_generate_after_a_visual_table(oracle_mod, q4_small):
    """generate() on a text prompt builds the 1-D table itself, whatever grid an earlier call
    prepared; a visual prompt without a table for its offset is refused."""
    from instantcua_amd.engine import EngineError

    vp = synth.visual_prompt(30, vis_offset=5, llm_h=2, llm_w=4, tag="pfx7")
    text = synth.random_tokens(24, "pfx-text2")
    steps = 6
    om = oracle_mod.OracleModel(q4_small, 64)
    ref, margins, lg = om.generate(text, steps)
    with Engine(flags=0, image=q4_small, max_context=64, max_steps=steps) as e:
        e.eos = (-1, -1)
        e.prepare_mrope(vp.vis_offset, vp.llm_h, vp.llm_w)
        e.set_visual(vp.pooler.astype(np.float32), None)
        e.generate(vp.tokens, vis_offset=vp.vis_offset, max_new_tokens=steps)
        got = e.generate(text, max_new_tokens=steps)
        with pytest.raises(EngineError, match="M-RoPE table"):
            e.generate(vp.tokens, vis_offset=vp.vis_offset + 1, max_new_tokens=steps)
    compare_greedy(np.array(got), ref, margins, lg.max() * np.ones(steps))
