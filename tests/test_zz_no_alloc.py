"""GPU check of the allocation-free quantiser entry point, icua_quantize_noalloc, against
icua_quantize (its allocating counterpart) through the C ABI: bit-identical codes and scales on
two calls in a row, the second on a smaller matrix, so the static scratch keeps the first call's
contents when the second one starts."""
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from test_gpu_quant import edge_matrix  # noqa: E402
from instantcua_amd import engine as eng  # noqa: E402
from instantcua_amd.modelfile import WeightFormat, matrix_bytes  # noqa: E402

pytestmark = pytest.mark.gpu


def _run(entry: str, fmt: int, m: np.ndarray):
    rows, cols = m.shape
    cb, sbb = matrix_bytes(fmt, rows, cols)
    dm = eng.DeviceBuffer.from_array(np.ascontiguousarray(m, dtype=np.float32))
    dc, ds = eng.DeviceBuffer(cb), eng.DeviceBuffer(sbb)
    try:
        eng._check(getattr(eng.lib(), entry)(fmt, dm.ptr, rows, cols, dc.ptr, ds.ptr))
        return dc.to_array(np.uint8, (cb,)), ds.to_array(np.uint8, (sbb,))
    finally:
        for b in (dm, dc, ds):
            b.free()


@pytest.mark.parametrize("fmt", [WeightFormat.Q4, WeightFormat.Q8])
def test_noalloc_quantize_matches_the_allocating_entry_point(fmt):
    # Edge groups include tiny-range ones that accept no clip candidate and take carried codes,
    # which is what the scratch records.  The second matrix is smaller than the first.
    for shape, seed in (((130, 2048), 7), ((96, 512), 8)):
        m = edge_matrix(*shape, seed=seed)
        want_c, want_s = _run("icua_quantize", fmt, m)
        got_c, got_s = _run("icua_quantize_noalloc", fmt, m)
        assert np.array_equal(got_s, want_s), f"{shape}: {(got_s != want_s).sum()} scale bytes differ"
        assert np.array_equal(got_c, want_c), f"{shape}: {(got_c != want_c).sum()} code bytes differ"
