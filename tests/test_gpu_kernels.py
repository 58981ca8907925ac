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
    """Dequantised weights equal fl32(s*q + b) (q4), s*q (q8), half (f16) bit for bit, from the
    .icua layout and from the repacked device layout."""
    K, N = 2048, 96
    m = synth.make_matrix(fmt, N, K, tag="dq", index=fmt)
    ref = oracle_mod.dequant(fmt, m.codes, m.sb, N, K)
    c = eng.DeviceBuffer.from_array(m.codes)
    s = eng.DeviceBuffer.from_array(m.sb)
    out = eng.DeviceBuffer(N * K * 4)
    eng.dequant(fmt, c, s, K, 0, N, out)
    got = out.to_array(np.float32, (N, K))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    out2 = eng.DeviceBuffer(7 * K * 4)
    eng.dequant(fmt, c, s, K, 40, 7, out2)
    assert np.array_equal(out2.to_array(np.float32, (7, K)).view(np.uint32), ref[40:47].view(np.uint32))
    tc, ts = eng.repack(fmt, c, s, N, K)
    eng.dequant(fmt, tc, ts, K, 0, N, out, tiled=True)
    assert np.array_equal(out.to_array(np.float32, (N, K)).view(np.uint32), ref.view(np.uint32))


# The isolated GEMV shapes (K x N): fused QKV, O, gate+up, down, lm_head, at 1, 3 and 8 rows;
# the lm_head shape at one row only (its multi-row passes run in the decoder and verify tests).
SHAPES = [(2048, 4096), (2048, 2048), (2048, 12288), (6144, 2048), (2048, 151936)]
GEMV_CASES = [(K, N, m) for K, N in SHAPES for m in (1, 3, 8) if N != 151936 or m == 1]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("K,N,m", GEMV_CASES)
def test_gemv_parity(oracle_mod, fmt, K, N, m):
    mat = synth.make_matrix(fmt, N, K, tag="gemv", index=fmt)
    x = synth.fp16_normal((m, K), "gemvx", m).astype(np.float32)  # fp16 N(0,1) activations
    ref = oracle_mod.gemv(fmt, mat.codes, mat.sb, N, K, x)
    c = eng.DeviceBuffer.from_array(mat.codes)
    s = eng.DeviceBuffer.from_array(mat.sb)
    tc, ts = eng.repack(fmt, c, s, N, K)
    xb = eng.DeviceBuffer.from_array(x)
    y = eng.DeviceBuffer(m * N * 4)
    eng.gemv(fmt, tc, ts, N, K, xb, m, y)
    got = y.to_array(np.float32, (m, N))
    err = rel_err(got, ref)
    # exact integer code x activation sums, fp32 group scaling, 22-bit activation slices
    assert err < 2e-6, f"rel err {err:.3g}"


def test_gemv_fp32_activations(oracle_mod):
    """Activations that are not fp16 values (wide dynamic range, zeros, a zero group) keep
    fp32-level accuracy: there is no fp16 rounding of the GEMV input."""
    K, N = 6144, 2048
    mat = synth.make_matrix(WeightFormat.Q4, N, K, tag="gemv32")
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((2, K)) * np.exp(rng.uniform(-6, 6, (2, K)))).astype(np.float32)
    x[0, :64] = 0.0          # an all-zero group
    x[1, 100:300] = 0.0
    ref = oracle_mod.gemv(WeightFormat.Q4, mat.codes, mat.sb, N, K, x)
    c = eng.DeviceBuffer.from_array(mat.codes)
    s = eng.DeviceBuffer.from_array(mat.sb)
    tc, ts = eng.repack(WeightFormat.Q4, c, s, N, K)
    y = eng.DeviceBuffer(2 * N * 4)
    eng.gemv(WeightFormat.Q4, tc, ts, N, K, eng.DeviceBuffer.from_array(x), 2, y)
    err = rel_err(y.to_array(np.float32, (2, N)), ref)
    assert err < 2e-6, f"rel err {err:.3g}"
