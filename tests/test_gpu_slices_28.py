"""Full-depth GPU parity of the persistent kernel's slice-streaming form (q8 and f16 weights: every
wave multiplies a K-slice of each stage's blocks): 28-layer synthetic decoders against the oracle
run live, from a short prompt and from a 4095-slot random cache (the decode benchmark's context,
with the uneven attention splits)."""
import numpy as np
import pytest

from conftest import compare_greedy, rel_err
from instantcua_amd import synth
from instantcua_amd.engine import Engine
from instantcua_amd.modelfile import Dims, WeightFormat

pytestmark = pytest.mark.gpu

NKV, HD = Dims.kv_heads, Dims.head_dim
LAYERS = 28
FORMATS = {"q8": WeightFormat.Q8, "f16": WeightFormat.F16}


@pytest.fixture(scope="module", params=list(FORMATS))
def model28(request):
    name = request.param
    return name, synth.build_model_image(FORMATS[name], n_layers=LAYERS, tag=f"{name}-28")


def _oracle_greedy(om, tok, pos, steps):
    """Greedy decode on the oracle from cache slot pos: tokens, top-2 margins, top logits."""
    toks, margins, tops = [], [], []
    for i in range(steps):
        lg = om.run_pass([tok], pos + i, logits_rows=1)[0]
        top2 = np.partition(lg, -2)[-2:]
        tok = int(np.argmax(lg))
        toks.append(tok)
        margins.append(float(top2[1] - top2[0]))
        tops.append(float(top2[1]))
    return toks, np.array(margins), np.array(tops)


def test_prompt_decode_28_layers(oracle_mod, model28):
    """A 16-token prompt, then 24 greedy steps on the persistent kernel in two calls: the tokens
    against the oracle's (a divergence must be an oracle near-tie), the prefill's logits within
    5e-4 of the oracle's (measured 1.2e-4 for q8 over 28 layers)."""
    name, img = model28
    toks = synth.random_tokens(16, f"slices28-{name}")
    steps = 24
    om = oracle_mod.OracleModel(img, 64)
    ref, margins, first = om.generate(toks, steps)
    with Engine(flags=0, image=img, max_context=64, max_steps=steps) as e:
        assert e.persistent_decode
        e.eos = (-1, -1)
        e.prefill(toks, max_new=steps, write_logits=True)
        first_gpu = e.logits(1)[0]
        e.decode_steps(9)
        e.decode_steps(steps - 10)
        assert e.last_decode_persistent
        st = e.state()
        got = e.tokens(st["step"])
    assert st["step"] == steps and st["done"] == 1, st
    assert rel_err(first_gpu, first) < 5e-4
    n, note = compare_greedy(got, ref, margins, first.max() * np.ones(steps))
    print(f"{name} 28 layers, prompt 16: {n}/{steps} identical ({note})")


def test_long_context_decode_28_layers(oracle_mod, model28):
    """Six greedy steps from slot 4095 of a random 28-layer cache: tokens against the oracle's."""
    name, img = model28
    pos, steps = 4095, 6
    maxctx = pos + 64
    tok0 = int(synth.random_tokens(1, f"slices28-long-{name}")[0])
    om = oracle_mod.OracleModel(img, maxctx)
    with Engine(flags=0, image=img, max_context=maxctx, max_steps=steps) as e:
        e.eos = (-1, -1)
        for l in range(LAYERS):
            for k in range(2):
                arr = synth.fp16_normal((NKV, pos, HD), f"slices28-{name}-{l}-{k}", pos)
                om.kv(l, k)[:, :pos] = arr
                e.write_kv(l, k, 0, arr)
        e.set_position(pos, tok0, 0, steps)
        e.decode_steps(steps)
        assert e.last_decode_persistent
        st = e.state()
        got = e.tokens(st["step"])
    ref, margins, tops = _oracle_greedy(om, tok0, pos, steps)
    assert st["step"] == steps and st["pos"] == pos + steps and st["done"] == 1
    n, note = compare_greedy(got, ref, margins, tops)
    print(f"{name} 28 layers, pos {pos}: {n}/{steps} identical ({note})")
