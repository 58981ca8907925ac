"""GPU parity of the matrix-core prefill (fp16 hi/lo GEMMs over q4 / q8 / f16 weights, flash
attention, chunking) against the oracle and against the 8-row pass path, through the C ABI."""
import numpy as np
import pytest

from conftest import compare_greedy, fp16_close, rel_err
from instantcua_amd import synth
from instantcua_amd.engine import Engine
from instantcua_amd.modelfile import Dims, WeightFormat

pytestmark = pytest.mark.gpu

LAYERS = 2


@pytest.fixture(scope="module")
def q4_small():
    return synth.build_model_image(WeightFormat.Q4, n_layers=LAYERS, tag="q4-small")


_IMAGES = {}


def small_image(fmt):
    """The 2-layer model of each weight format (q4 group 64, q8 group 32, f16)."""
    if fmt not in _IMAGES:
        _IMAGES[fmt] = synth.build_model_image(fmt, n_layers=LAYERS, tag=f"fmt{fmt}-small")
    return _IMAGES[fmt]


def _kv_close(got_rows, ref_rows, layer):
    # Layer 0's K/V come from one projection of the embedding: fp32-level differences only
    # flip fp16 rounding boundaries, or move a value near zero (RoPE cancellation) by a few of
    # its own ulps but less than 1e-6 of its row.  Layer 1 inherits layer 0's fp16-cache reads
    # and summation order, so small values of a row can be several of their own ulps off
    # (bounded against the row scale, as in the decode-path tests).
    if layer == 0:
        fp16_close(got_rows, ref_rows, max_ulp=1, row_tol=1e-6, frac_over_1ulp=1e-3)
    else:
        fp16_close(got_rows, ref_rows, max_ulp=2, row_tol=2e-3, frac_over_1ulp=5e-2)


@pytest.mark.parametrize("fmt", [WeightFormat.Q4, WeightFormat.Q8, WeightFormat.F16], ids=["q4", "q8", "f16"])
@pytest.mark.parametrize("n", [9, 130, 400])
def test_prefill_matches_oracle(oracle_mod, q4_small, n, fmt):
    """Prompts of one partial 16-row block up to several 128-row tiles, for each weight format:
    first logits, every prompt K/V row of both layers and the greedy continuation."""
    img = q4_small if fmt == WeightFormat.Q4 else small_image(fmt)
    toks = synth.random_tokens(n, f"pf-oracle-{n}")
    steps = 6
    om = oracle_mod.OracleModel(img, n + 16)
    ref, margins, first = om.generate(toks, steps)
    with Engine(flags=0, image=img, max_context=n + 16, max_steps=steps) as e:
        e.eos = (-1, -1)
        assert not e.pass_prefill
        tok0 = e.prefill(toks, max_new=steps, write_logits=True)
        lg = e.logits(1)[0]
        kv = {(l, k): e.read_kv(l, k, 0, n) for l in range(LAYERS) for k in range(2)}
        e.decode_steps(steps - 1)
        got = e.tokens(steps)
        t = e.last_timing
    assert rel_err(lg, first) < 1e-2  # the stated logits tolerance
    assert rel_err(lg, first) < 1e-4, f"first-logit rel err {rel_err(lg, first):.3g}"
    assert tok0 == ref[0]
    for (l, k), rows in kv.items():
        _kv_close(rows, om.kv(l, k)[:, :n], l)
    cnt, note = compare_greedy(got, ref, margins, first.max() * np.ones(steps))
    print(f"fmt {fmt} n {n}: logits rel err {rel_err(lg, first):.3g}; {cnt}/{steps} identical ({note}); "
          f"prefill {t['prefill_ms']:.2f} ms")


@pytest.mark.parametrize("fmt", [WeightFormat.Q4, WeightFormat.Q8, WeightFormat.F16], ids=["q4", "q8", "f16"])
def test_prefill_fp16_operands_match_oracle(oracle_mod, q4_small, fmt):
    """ICUA_FLAG_PREFILL_FP16: the GEMMs and the attention on fp16 operands alone (the reference
    engine's precision) instead of fp16 hi + lo.  The error is then that of fp16 activations
    (~2^-12 per operand): first logits within the stated 1e-2 (measured 1-3e-3), K/V rows within
    1e-2 of their row, and the greedy tokens of the oracle (a divergence only at a near-tie)."""
    n = 400
    img = q4_small if fmt == WeightFormat.Q4 else small_image(fmt)
    toks = synth.random_tokens(n, f"pf-oracle-{n}")
    steps = 6
    om = oracle_mod.OracleModel(img, n + 16)
    ref, margins, first = om.generate(toks, steps)
    with Engine(flags=0, image=img, max_context=n + 16, max_steps=steps) as e:
        e.eos = (-1, -1)
        e.prefill_fp16 = True
        e.prefill(toks, max_new=steps, write_logits=True)
        lg = e.logits(1)[0]
        kv = {(l, k): e.read_kv(l, k, 0, n) for l in range(LAYERS) for k in range(2)}
        e.decode_steps(steps - 1)
        got = e.tokens(steps)
    err = rel_err(lg, first)
    print(f"fmt {fmt}: fp16-operand prefill, first-logit rel err {err:.3g}")
    assert err < 1e-2
    for (l, k), rows in kv.items():
        g = rows.astype(np.float32)
        r = om.kv(l, k)[:, :n].astype(np.float32)
        assert np.all(np.abs(g - r) <= 1e-2 * np.abs(r).max(axis=-1, keepdims=True)), (l, k)
    compare_greedy(got, ref, margins, first.max() * np.ones(steps))


@pytest.mark.parametrize("fp16", [False, True], ids=["hi-lo", "fp16-operands"])
def test_prefill_continuation_at_offset(oracle_mod, q4_small, fp16):
    """A second prefill call at start_pos 200 (not a multiple of the attention's 64-slot halves or
    32-query tiles) attends over the cache rows of the first, in both operand modes (fp16 operands
    alone: first logits within 1e-2, K/V rows within 1e-2 of their row, as in the test above)."""
    toks = synth.random_tokens(500, "pf-offset")
    om = oracle_mod.OracleModel(q4_small, 512)
    ref_lg = om.run_pass(toks, 0, logits_rows=1)[0]
    with Engine(flags=0, image=q4_small, max_context=512, max_steps=8) as e:
        e.eos = (-1, -1)
        e.prefill_fp16 = fp16
        e.prefill(toks[:200], max_new=2)
        e.prefill(toks[200:], start_pos=200, max_new=2, write_logits=True)
        lg = e.logits(1)[0]
        st = e.state()
        kv = {(l, k): e.read_kv(l, k, 0, 500) for l in range(LAYERS) for k in range(2)}
    assert st["pos"] == 500 and st["step"] == 1
    err = rel_err(lg, ref_lg)
    assert err < (1e-2 if fp16 else 1e-4), err
    for (l, k), rows in kv.items():
        if fp16:
            g, r = rows.astype(np.float32), om.kv(l, k)[:, :500].astype(np.float32)
            assert np.all(np.abs(g - r) <= 1e-2 * np.abs(r).max(axis=-1, keepdims=True)), (l, k)
        else:
            _kv_close(rows, om.kv(l, k)[:, :500], l)


@pytest.mark.parametrize("fp16", [False, True], ids=["hi-lo", "fp16-operands"])
def test_visual_prefill_matches_oracle(oracle_mod, q4_small, fp16):
    """Image-pad rows over several 16-row blocks: visual embeddings, 3D M-RoPE, DeepStack; with
    fp16 operands alone at that mode's bounds (first logits 1e-2, K/V within 1e-2 of their row)."""
    vp = synth.visual_prompt(300, vis_offset=16, llm_h=8, llm_w=16, tag="pf-vis")
    pooler = vp.pooler.astype(np.float32)
    ds = [d.astype(np.float32) for d in vp.deepstack]
    steps = 6
    om = oracle_mod.OracleModel(q4_small, 320)
    om.prepare_mrope(vp.vis_offset, vp.llm_h, vp.llm_w)
    ref, margins, first = om.generate(vp.tokens, steps, pooler=pooler, vis_offset=vp.vis_offset, deepstack=ds)
    with Engine(flags=0, image=q4_small, max_context=320, max_steps=steps) as e:
        e.eos = (-1, -1)
        e.prefill_fp16 = fp16
        e.prepare_mrope(vp.vis_offset, vp.llm_h, vp.llm_w)
        e.set_visual(pooler, ds)
        e.prefill(vp.tokens, vis_offset=vp.vis_offset, max_new=steps, write_logits=True)
        lg = e.logits(1)[0]
        kv1 = e.read_kv(1, 0, 0, 300)
        e.decode_steps(steps - 1)
        got = e.tokens(steps)
    err = rel_err(lg, first)
    assert err < (1e-2 if fp16 else 1e-4), err
    if fp16:
        g, r = kv1.astype(np.float32), om.kv(1, 0)[:, :300].astype(np.float32)
        assert np.all(np.abs(g - r) <= 1e-2 * np.abs(r).max(axis=-1, keepdims=True))
    else:
        _kv_close(kv1, om.kv(1, 0)[:, :300], 1)
    compare_greedy(got, ref, margins, first.max() * np.ones(steps))


def test_two_chunks_match_pass_path(q4_small):
    """4296 rows = a full 4096-row chunk + 200: the matrix-core path against the 8-row passes
    (the same oracle-checked decode kernels) on first logits and every cache row of layer 1."""
    n = 4096 + 200
    toks = synth.random_tokens(n, "pf-chunks")
    out = {}
    for passes in (False, True):
        with Engine(flags=0, image=q4_small, max_context=n + 8, max_steps=4) as e:
            e.eos = (-1, -1)
            e.pass_prefill = passes
            tok0 = e.prefill(toks, max_new=2, write_logits=True)
            out[passes] = (tok0, e.logits(1)[0], e.read_kv(1, 0, 0, n), e.read_kv(1, 1, 0, n),
                           e.last_timing["prefill_ms"])
    mm, ps = out[False], out[True]
    print(f"prefill {n} rows: matrix-core {mm[4]:.1f} ms, passes {ps[4]:.1f} ms")
    assert rel_err(mm[1], ps[1]) < 1e-4, rel_err(mm[1], ps[1])
    assert mm[0] == ps[0]
    for kind in (2, 3):
        fp16_close(mm[kind], ps[kind], max_ulp=2, row_tol=2e-3, frac_over_1ulp=5e-2)


@pytest.mark.parametrize("fmt", [WeightFormat.Q8, WeightFormat.F16], ids=["q8", "f16"])
@pytest.mark.parametrize("n", [1024, 4096])
def test_large_tile_prefill_matches_oracle(oracle_mod, n, fmt):
    """Prompts long enough for the larger GEMM tiles (prefill.hip pf_gemm_fmt picks the largest
    tile whose count fills the 256 CUs evenly), q8 and f16, against the oracle run live:

      n = 1024: q8 QKV and gate|up on 128 x 128 tiles (8 row-tiles x 32 / 96 column tiles), O and
                down on 64 x 128; f16 the same.
      n = 4096: q8 every GEMM on 128 x 256 tiles (32 x 16 / 8 / 48 / 8 tiles); f16 (never 256-row
                tiles) every GEMM on 128 x 128.

    Checked: first logits within 1e-4, K/V rows of the last layer at spread slots, first greedy
    tokens; then the same prompt with fp16 operands alone (ICUA_FLAG_PREFILL_FP16, whose q8 GEMMs
    keep 128-row tiles and take the dequantised weights as B operands) against the same oracle
    run: first logits within 1e-2, K/V rows within 1e-2 of their row, the first greedy token."""
    img = small_image(fmt)
    toks = synth.random_tokens(n, f"pf-large-{n}")
    steps = 3
    om = oracle_mod.OracleModel(img, n + 8)
    ref, margins, first = om.generate(toks, steps)
    slots = sorted({0, 1, 127, 128, n // 2, n - 129, n - 1})
    with Engine(flags=0, image=img, max_context=n + 8, max_steps=steps) as e:
        e.eos = (-1, -1)
        assert not e.pass_prefill
        e.prefill(toks, max_new=steps, write_logits=True)
        lg = e.logits(1)[0]
        assert e.last_timing["prefill_tokens"] == n
        kv = [np.stack([e.read_kv(LAYERS - 1, kind, s, 1)[:, 0] for s in slots], axis=1) for kind in (0, 1)]
        e.decode_steps(steps - 1)
        got = e.tokens(steps)
    err = rel_err(lg, first)
    print(f"fmt {fmt} n {n}: first-token logits rel err {err:.3g}")
    assert err < 1e-4, err
    for kind in (0, 1):
        fp16_close(kv[kind], om.kv(LAYERS - 1, kind)[:, slots], max_ulp=2, row_tol=2e-3, frac_over_1ulp=5e-2)
    compare_greedy(got, ref, margins, first.max() * np.ones(steps))

    with Engine(flags=0, image=img, max_context=n + 8, max_steps=steps) as e:
        e.eos = (-1, -1)
        e.prefill_fp16 = True
        tok0 = e.prefill(toks, max_new=steps, write_logits=True)
        lg = e.logits(1)[0]
        kv = [np.stack([e.read_kv(LAYERS - 1, kind, s, 1)[:, 0] for s in slots], axis=1) for kind in (0, 1)]
    err = rel_err(lg, first)
    print(f"fmt {fmt} n {n}: fp16-operand first-token logits rel err {err:.3g}")
    assert err < 1e-2, err
    for kind in (0, 1):
        g, r = kv[kind].astype(np.float32), om.kv(LAYERS - 1, kind)[:, slots].astype(np.float32)
        assert np.all(np.abs(g - r) <= 1e-2 * np.abs(r).max(axis=-1, keepdims=True)), kind
    compare_greedy(np.array([tok0]), ref[:1], margins[:1], first.max() * np.ones(1))
