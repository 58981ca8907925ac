"""Full-size parity runs: the q8 speculative verify (8 random drafts over 8192 fp16 N(0,1) cache
rows, 28 layers) and 256-step greedy decode through the persistent kernel, against the oracle."""
import numpy as np
import pytest

from conftest import compare_greedy, rel_err
from instantcua_amd import synth
from instantcua_amd.engine import Engine
from instantcua_amd.modelfile import Dims, WeightFormat

pytestmark = pytest.mark.gpu

NKV, HD = Dims.kv_heads, Dims.head_dim


def _accepted(draft, argmax):
    """Accepted prefix of a greedy verify: draft[i + 1] must equal the argmax after row i."""
    n = 0
    while n + 1 < len(draft) and int(argmax[n]) == int(draft[n + 1]):
        n += 1
    return n


def test_verify_q8_28_layers_8192_context(oracle_mod):
    ctx, m, layers = 8192, 8, Dims.layers
    img = synth.build_model_image(WeightFormat.Q8, n_layers=layers, tag="verify-q8")
    draft = synth.random_tokens(m, "verify-q8-draft")
    om = oracle_mod.OracleModel(img, ctx + m + 8)
    with Engine(flags=0, image=img, max_context=ctx + m + 8, max_steps=8) as e:
        for l in range(layers):
            for kind in (0, 1):
                rows = synth.fp16_normal((NKV, ctx, HD), f"verify-q8-kv{kind}", l)
                om.kv(l, kind)[:, :ctx] = rows
                e.write_kv(l, kind, 0, rows)
        e.set_position(ctx, int(draft[0]), 0, 4)
        am, lg = e.verify(draft, want_logits=True)
        st = e.state()
        new_k = e.read_kv(layers - 1, 0, ctx, m)
    ref_lg = om.run_pass(draft, ctx, logits_rows=m)
    assert st["pos"] == ctx  # verify leaves the position to the caller
    assert rel_err(lg, ref_lg) < 1e-2  # the stated logits tolerance
    assert rel_err(lg, ref_lg) < 1e-4, rel_err(lg, ref_lg)
    ref_am = ref_lg.argmax(axis=1)
    for i in range(m):
        if am[i] != ref_am[i]:
            srt = np.sort(ref_lg[i])
            assert srt[-1] - srt[-2] < 1e-3 * abs(srt[-1]), f"row {i}: {am[i]} vs {ref_am[i]}"
    assert _accepted(draft, am) == _accepted(draft, ref_am)
    # The drafts' K rows of the last layer: fp32-level differences accumulated over 28 layers,
    # bounded against the row scale.
    r = om.kv(layers - 1, 0)[:, ctx:ctx + m].astype(np.float32)
    d = np.abs(new_k.astype(np.float32) - r)
    assert (d <= 2e-3 * np.abs(r).max(axis=-1, keepdims=True) + np.spacing(np.abs(r).astype(np.float16))).all()


@pytest.mark.parametrize("fmt_name", ["q4", "q8"])
def test_greedy_256_steps(oracle_mod, fmt_name):
    """256 greedy steps after a 64-token prompt through the persistent kernel (2-layer models)."""
    fmt = WeightFormat.Q4 if fmt_name == "q4" else WeightFormat.Q8
    img = synth.build_model_image(fmt, n_layers=2, tag=f"{fmt_name}-small")
    toks = synth.random_tokens(64, f"g256-{fmt_name}")
    steps = 256
    om = oracle_mod.OracleModel(img, 64 + steps + 8)
    ref, margins, first = om.generate(toks, steps)
    with Engine(flags=0, image=img, max_context=64 + steps + 8, max_steps=steps) as e:
        e.eos = (-1, -1)
        assert e.persistent_decode
        e.prefill(toks, max_new=steps)
        e.decode_steps(steps - 1)
        st = e.state()
        got = e.tokens(st["step"])
    assert st["step"] == steps and st["done"] == 1
    n, note = compare_greedy(got, ref, margins, first.max() * np.ones(steps))
    print(f"{fmt_name}: {n}/{steps} identical ({note})")
