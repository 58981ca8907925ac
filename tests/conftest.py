import ctypes
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def _keep_freed_memory() -> None:
    """The tests build many synthetic model images of 100-300 MB.  Serving large allocations
    from the heap and never trimming it lets each image reuse the pages of the previous one
    instead of mapping and first-touching fresh ones, which on some hosts costs more than the
    test's own work (mallopt M_MMAP_THRESHOLD = 1 GiB, M_TRIM_THRESHOLD = 2 GiB - 1)."""
    try:
        libc = ctypes.CDLL("libc.so.6")
        libc.mallopt(-3, 1 << 30)
        libc.mallopt(-1, 2**31 - 1)
    except OSError:
        pass


_keep_freed_memory()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running full-size check")


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle

    oracle.build()
    return oracle


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / max |ref| (the logits tolerance metric)."""
    ref = np.asarray(ref, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def near_tie(logits_margin: float, top1: float) -> bool:
    """A greedy divergence is a reported near-tie when the oracle's top-1/top-2 margin is
    below 1e-3 of the top logit."""
    return logits_margin < 1e-3 * max(abs(top1), 1.0)


def compare_greedy(gpu_tokens, ref_tokens, ref_margins, ref_top=None):
    """Returns (n_identical_prefix, note).  Raises AssertionError on a divergence that is not a
    near-tie of the oracle."""
    gpu_tokens = list(gpu_tokens)
    ref_tokens = list(ref_tokens)
    n = min(len(gpu_tokens), len(ref_tokens))
    for i in range(n):
        if gpu_tokens[i] != ref_tokens[i]:
            top = 10.0 if ref_top is None else ref_top[i]
            if near_tie(float(ref_margins[i]), top):
                return i, f"near-tie at step {i}: oracle margin {ref_margins[i]:.3g}"
            raise AssertionError(
                f"greedy divergence at step {i}: gpu {gpu_tokens[i]} oracle {ref_tokens[i]} "
                f"(oracle top-2 margin {ref_margins[i]:.4g})")
    return n, "identical"


def fp16_close(got, ref, max_ulp=1, row_tol=1e-6, frac_over_1ulp=0.0):
    """fp16 cache rows [..., HD]: every value within max_ulp fp16 ulps of itself or row_tol of its
    row's largest magnitude, and at most frac_over_1ulp of the values more than one ulp away."""
    g = np.asarray(got).astype(np.float32)
    r = np.asarray(ref).astype(np.float32)
    ulp = np.spacing(np.abs(r).astype(np.float16)).astype(np.float32)
    rowmax = np.abs(r).max(axis=-1, keepdims=True)
    d = np.abs(g - r)
    bad = d > np.maximum(max_ulp * ulp, row_tol * rowmax)
    assert not bad.any(), f"{bad.sum()} cache values beyond {max_ulp} ulp / {row_tol:g} of the row"
    over = (d > ulp).mean()
    assert over <= frac_over_1ulp, f"{over:.3g} of the cache values beyond one ulp"


def compare_greedy_forced(e, n_prompt, ref, margins, top1, steps):
    """Compares all `steps` greedy tokens of a decode (token 0 from the prefill, the rest from
    e.decode_steps) with the oracle's, step by step.  A divergence must be a near-tie of the
    oracle at that step (its margin below 1e-3 of that step's top-1 logit); the decode then
    continues teacher-forced: icua_set_position feeds the oracle's token at its slot and the later
    steps are decoded again, so every step after a near-tie is compared as well
    (qwen3vl_ref.py:294-336 is the loop being followed).  Returns the near-tie steps."""
    got = e.tokens(steps)
    ties = []
    i = 0
    while True:
        diff = np.nonzero(got[i:] != ref[i:steps])[0]
        if diff.size == 0:
            return ties
        j = i + int(diff[0])
        if not near_tie(float(margins[j]), float(top1[j])):
            raise AssertionError(
                f"greedy divergence at step {j}: gpu {got[j]} oracle {ref[j]} "
                f"(oracle top-2 margin {margins[j]:.4g}, top-1 {top1[j]:.4g}; earlier near-ties {ties})")
        ties.append(j)
        if j == steps - 1:
            return ties
        e.set_position(n_prompt + j, int(ref[j]), j + 1, steps)
        e.decode_steps(steps - 1 - j)
        got = e.tokens(steps)
        i = j + 1
