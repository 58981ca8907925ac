"""GPU parity of the standalone kernels against the oracle: bit-exact dequantisation and the
dequant-GEMV at the decoder's shapes (all through the C ABI)."""
import numpy as np
import pytest

from conftest import rel_err
from instantcua_amd import engine as eng
from instantcua_amd import synth
from instantcua_amd.modelfile import WeightFormat

pytestmark = pytest.mark.gpu

FMTS = [WeightFormat.Q4, WeightFormat.Q8, WeightFormat.F16]


@pytest.mark.parametrize("fmt", FMTS)
def test_dequant_bit_exact(oracle_mod, fmt):
    K, N = 2048, 96
    m = synth.make_matrix(fmt, N, K, tag="dq", index=fmt)
    ref = oracle_mod.dequant(fmt, m.codes, m.sb, N, K)
    c = eng.DeviceBuffer.from_array(m.codes)
    s = eng.DeviceBuffer.from_array(m.sb)
    out = eng.DeviceBuffer(N * K * 4)
    eng.dequant(fmt, c, s, K, 0, N, out)
    got = out.to_array(np.float32, (N, K))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # a sub-range of rows
    out2 = eng.DeviceBuffer(7 * K * 4)
    eng.dequant(fmt, c, s, K, 40, 7, out2)
    assert np.array_equal(out2.to_array(np.float32, (7, K)).view(np.uint32), ref[40:47].view(np.uint32))


# The isolated GEMV shapes (K x N): fused QKV, O, gate+up, down, lm_head.
SHAPES = [(2048, 4096), (2048, 2048), (2048, 12288), (6144, 2048), (2048, 151936)]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("K,N", SHAPES)
@pytest.mark.parametrize("m", [1, 3, 8])
def test_gemv_parity(oracle_mod, fmt, K, N, m):
    if N == 151936 and m != 1:
        pytest.skip("lm_head-sized multi-row case covered by the decoder tests")
    mat = synth.make_matrix(fmt, N, K, tag="gemv", index=fmt)
    x = synth.fp16_normal((m, K), "gemvx", m)
    ref = oracle_mod.gemv(fmt, mat.codes, mat.sb, N, K, x)
    c = eng.DeviceBuffer.from_array(mat.codes)
    s = eng.DeviceBuffer.from_array(mat.sb)
    xb = eng.DeviceBuffer.from_array(x)
    y = eng.DeviceBuffer(m * N * 4)
    eng.gemv(fmt, c, s, N, K, xb, m, y)
    got = y.to_array(np.float32, (m, N))
    err = rel_err(got, ref)
    # fp32 accumulation against the double-accumulated oracle
    assert err < 2e-5, f"rel err {err:.3g}"
