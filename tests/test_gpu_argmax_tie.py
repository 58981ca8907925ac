"""Exact greedy-argmax ties on the GPU: the lower token id wins an equal logit
(Shaders.swift:1514-1536, k_commit's `v == best && id < bi`).

The models are the oracle's tie models (test_oracle_pins.tie_models): a lower id u is given the
embedding row of the winner t of greedy step k, so the tied lm_head's logits of u and t are
bit-identical on every path.  Checked for k = 0 (the prefill's first token: the lm_head GEMV and
its argmax merge) and k = 3 (a decode step of the persistent kernel, and of the per-stage graph
path), each against the oracle on the same image."""
import numpy as np
import pytest

from conftest import compare_greedy
from instantcua_amd.engine import FLAG_GRAPH_DECODE, Engine
from test_oracle_pins import tie_models

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("graph", [False, True], ids=["persistent", "graph"])
def test_gpu_argmax_tie_takes_the_lower_id(oracle_mod, graph):
    _, toks, ref, cases = tie_models(oracle_mod)
    steps = len(ref)
    for k, t, u, img_k in cases:
        om = oracle_mod.OracleModel(img_k, 64)
        want, margins, first = om.generate(toks, steps)
        om.close()
        assert int(want[k]) == u
        with Engine(flags=FLAG_GRAPH_DECODE if graph else 0, image=img_k, max_context=64, max_steps=steps) as e:
            e.eos = (-1, -1)
            e.prefill(toks, max_new=steps, write_logits=True)
            lg = e.logits(1)[0]
            e.decode_steps(steps - 1)
            got = e.tokens(steps)
            assert e.last_decode_persistent == (not graph)
        print(f"tie at step {k}: t={t} u={u} gpu {got.tolist()} oracle {want.tolist()}")
        if k == 0:
            assert lg[u] == lg[t] and lg[u] == lg.max()
        assert np.array_equal(got[:k + 1], want[:k + 1]), (k, got, want)
        assert int(got[k]) == u
        compare_greedy(got[k + 1:], want[k + 1:], margins[k + 1:], first.max() * np.ones(steps - k - 1))
