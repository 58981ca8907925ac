"""The fp32 CPU port (oracle/port32.c), timed as the benchmark's CPU baseline, against the
oracle (CPU only).

The port is not the checker: it is the reference decoder math in fp32 arithmetic, written for
speed on the host.  These tests show that what the benchmark times computes the same decoder:
logits within fp32 rounding of the oracle's, the same greedy tokens, and the same fp16 K/V rows
to about an fp16 ulp of their largest value, for every weight format and for one-token (fused dequantise-and-dot) and
many-token (dequantised-row) GEMVs.
"""
import numpy as np
import pytest

from instantcua_amd import synth
from instantcua_amd.modelfile import WeightFormat


@pytest.mark.parametrize("fmt", [WeightFormat.Q4, WeightFormat.Q8, WeightFormat.F16])
def test_port32_matches_the_oracle(oracle_mod, fmt):
    img = synth.build_model_image(fmt, n_layers=2, tag="port32")
    a = oracle_mod.OracleModel(img, 48)
    b = oracle_mod.OracleModel(img, 48)
    try:
        toks = synth.random_tokens(21, "port32", 1)  # a partial 8-token block in the GEMMs
        la = a.run_pass(toks, 0).reshape(-1)
        lb = b.port32_pass(toks, 0)
        assert np.abs(la - lb).max() <= 2e-4 * np.abs(la).max()
        assert int(np.argmax(la)) == int(np.argmax(lb))
        for layer in range(2):
            for kind in range(2):
                ka = a.kv(layer, kind)[:, :21].view(np.float16).astype(np.float32)
                kb = b.kv(layer, kind)[:, :21].view(np.float16).astype(np.float32)
                assert np.abs(ka - kb).max() <= 1e-3 * np.abs(ka).max()  # fp16 ulp is 2^-11 relative
        tok = int(np.argmax(la))
        for s in range(4):  # one-token passes: the fused GEMV
            la = a.run_pass([tok], 21 + s).reshape(-1)
            lb = b.port32_pass([tok], 21 + s)
            assert np.abs(la - lb).max() <= 2e-4 * np.abs(la).max()
            assert int(np.argmax(la)) == int(np.argmax(lb))
            tok = int(np.argmax(la))
    finally:
        a.close()
        b.close()


def test_port32_rejects_a_pass_past_the_context(oracle_mod):
    img = synth.build_model_image(WeightFormat.Q4, n_layers=1, tag="port32")
    m = oracle_mod.OracleModel(img, 8)
    try:
        with pytest.raises(RuntimeError):
            m.port32_pass(np.arange(4, dtype=np.int32), 6)
    finally:
        m.close()
