"""Pins of the oracle's quantisers (Convert.swift:214-320) -- CPU only.

Known-answer groups fix the codes, the (scale, bias) words and the packing; invariants fix the
code assignment and the q8 scale; an independent float64 evaluation of all 25 clip candidates
fixes the q4 candidate choice.
"""
import numpy as np
import pytest

orc = None


@pytest.fixture(autouse=True)
def _oracle(oracle_mod):
    global orc
    orc = oracle_mod

CLIPS = (0.0, 0.03, 0.06, 0.1, 0.15)


def h2f(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def f16(x):
    return np.float16(x).view(np.uint16)


def unpack_q4(packed):
    lo = packed & 0x0F
    hi = packed >> 4
    return np.stack([lo, hi], axis=-1).reshape(packed.shape[0], -1)


# ---------------------------------------------------------------------------------------- q8

def test_q8_known_answer_multiples_of_the_scale():
    """w = k * s0 with k = -127..127 (127 present): scale s0, codes k."""
    s0 = np.float32(2.0 ** -7)
    k = np.concatenate([[127, -127], np.arange(-15, 15)]).astype(np.int32)
    m = (k.astype(np.float32) * s0).reshape(1, 32)
    codes, scales = orc.quant_q8(m)
    assert scales[0, 0] == f16(s0)
    assert np.array_equal(codes[0].astype(np.int32), k)


def test_q8_rounds_half_away_from_zero():
    """Scale 2^-7 (max 127 * 2^-7); w / s = +-2.5, +-0.5, 126.5 -> 3, -3, 1, -1, 127."""
    s0 = 2.0 ** -7
    vals = [127.0, 2.5, -2.5, 0.5, -0.5, 126.5, 1.5, -1.5] + [0.0] * 24
    m = (np.array(vals, dtype=np.float32) * np.float32(s0)).reshape(1, 32)
    codes, scales = orc.quant_q8(m)
    assert scales[0, 0] == f16(s0)
    assert list(codes[0, :8]) == [127, 3, -3, 1, -1, 127, 2, -2]


def test_q8_zero_group():
    codes, scales = orc.quant_q8(np.zeros((2, 64), np.float32))
    assert not codes.any() and not scales.any()


def test_q8_scale_is_the_smallest_sufficient_half():
    """s * 127 >= amax, and the next smaller fp16 would not reach amax; |s*q - w| <= s/2."""
    rng = np.random.default_rng(1)
    m = (rng.standard_normal((70, 256)) * rng.uniform(1e-4, 3, (70, 1))).astype(np.float32)
    codes, scales = orc.quant_q8(m)
    g = m.reshape(70, 8, 32)
    amax = np.abs(g).max(axis=2)
    s = h2f(scales)
    prev = h2f(scales - 1)
    assert np.all(s * np.float32(127) >= amax)
    assert np.all(prev * np.float32(127) < amax)
    rec = codes.reshape(70, 8, 32).astype(np.float64) * s[..., None]
    assert np.all(np.abs(rec - g) <= s[..., None].astype(np.float64) * (0.5 + 1e-6))


# ---------------------------------------------------------------------------------------- q4

def representable_group(s0, b0, rng):
    q = rng.integers(0, 16, 64)
    q[3], q[40] = 0, 15  # the group spans the full code range
    w = (q.astype(np.float32) * np.float32(s0) + np.float32(b0)).astype(np.float32)
    return q, w


def test_q4_known_answer_exact_group():
    """w = s0 * q + b0 exactly (s0 = 2^-6, b0 = -0.25): the first candidate fits with zero error,
    so (s, b) = (s0, b0) and the codes are q, packed low nibble first."""
    rng = np.random.default_rng(2)
    q, w = representable_group(2.0 ** -6, -0.25, rng)
    q2, w2 = representable_group(2.0 ** -3, 1.5, rng)
    m = np.concatenate([w, w2]).reshape(1, 128)
    packed, sb = orc.quant_q4(m)
    assert sb[0, 0, 0] == f16(2.0 ** -6) and sb[0, 0, 1] == f16(-0.25)
    assert sb[0, 1, 0] == f16(2.0 ** -3) and sb[0, 1, 1] == f16(1.5)
    assert np.array_equal(unpack_q4(packed)[0], np.concatenate([q, q2]))
    assert packed[0, 0] == (q[0] | (q[1] << 4))


def test_q4_constant_group():
    m = np.full((1, 64), 0.375, np.float32)
    packed, sb = orc.quant_q4(m)
    assert not packed.any()
    assert sb[0, 0, 0] == 0 and sb[0, 0, 1] == f16(0.375)


def test_q4_no_accepted_candidate_keeps_the_previous_codes():
    """A range above 1e-12 whose every candidate scale rounds to fp16 zero accepts no candidate:
    (s, b) = (0, 0) and the group keeps the chunk's previous codes (zeros at a chunk start)."""
    rng = np.random.default_rng(3)
    q, w = representable_group(2.0 ** -6, -0.25, rng)
    tiny = (np.float32(1.0) + np.arange(64, dtype=np.float32) * np.float32(1e-9)).astype(np.float32)
    assert tiny.max() - tiny.min() >= np.float32(1e-12)
    m = np.concatenate([w, tiny, tiny, w]).reshape(2, 128)
    packed, sb = orc.quant_q4(m)
    codes = unpack_q4(packed)
    assert sb[0, 1, 0] == 0 and sb[0, 1, 1] == 0
    assert np.array_equal(codes[0, 64:], q)          # carried from group 0 of row 0
    assert np.array_equal(codes[1, :64], q)          # carried across the row end, same chunk
    # Alone (first group of its chunk) the tiny group keeps the chunk's initial zeros.
    p1, sb1 = orc.quant_q4(tiny.reshape(1, 64))
    assert not p1.any() and sb1[0, 0, 0] == 0 and sb1[0, 0, 1] == 0


def candidate_errors(w):
    """Independent float64 evaluation of the 25 clip candidates (Convert.swift:284-317):
    returns [(err, s16, b16)] in search order, None for a skipped candidate."""
    w = w.astype(np.float64)
    mn, mx = w.min(), w.max()
    rng_ = mx - mn
    out = []
    for a in CLIPS:
        for c in CLIPS:
            lo, hi = mn + a * rng_, mx - c * rng_
            s, b = (hi - lo) / 15, lo
            v = np.clip(np.floor((w - b) / s + 0.5), 0, 15)
            den = 64 * (v * v).sum() - v.sum() ** 2
            if den > 0:
                s2 = (64 * (v * w).sum() - v.sum() * w.sum()) / den
                if s2 > 0:
                    s, b = s2, (w.sum() - s2 * v.sum()) / 64
            s16, b16 = float(np.float16(s)), float(np.float16(b))
            if s16 <= 0:
                out.append(None)
                continue
            v = np.clip(np.floor((w - b16) / s16 + 0.5), 0, 15)
            out.append((float(((s16 * v + b16 - w) ** 2).sum()), s16, b16))
    return out


def test_q4_choice_is_the_least_squares_candidate():
    rng = np.random.default_rng(4)
    rows = []
    for k in range(48):
        kind = k % 3
        if kind == 0:
            w = rng.standard_normal(64) * 0.02
        elif kind == 1:  # one outlier: clipping pays
            w = rng.uniform(-1, 1, 64)
            w[rng.integers(0, 64)] = 25.0
        else:
            w = rng.uniform(0.5, 0.7, 64) ** 3
        rows.append(w.astype(np.float32))
    m = np.stack(rows).reshape(48, 64)
    packed, sb = orc.quant_q4(m)
    codes = unpack_q4(packed)
    s, b = h2f(sb[:, 0, 0]), h2f(sb[:, 0, 1])
    for r in range(48):
        cands = [c for c in candidate_errors(m[r]) if c is not None]
        best = min(e for e, _, _ in cands)
        w = m[r].astype(np.float64)
        err = ((s[r] * codes[r] + b[r] - w) ** 2).sum()
        assert err <= best * (1 + 1e-5) + 1e-12, (r, err, best)
        assert any(abs(cs - s[r]) == 0 and abs(cb - b[r]) == 0 for _, cs, cb in cands), r
        # Every code is the nearest level of (s, b) (up to a rounding tie).
        lvl = s[r] * np.arange(16, dtype=np.float64) + b[r]
        d = np.abs(w[:, None] - lvl[None, :])
        assert np.all(d[np.arange(64), codes[r]] <= d.min(axis=1) + 1e-6 * s[r])
        if r % 3 == 1:  # the outlier group chooses a clipped range over plain min / max
            naive_s, naive_b = float(np.float16((w.max() - w.min()) / 15)), float(np.float16(w.min()))
            vn = np.clip(np.floor((w - naive_b) / naive_s + 0.5), 0, 15)
            assert err < ((naive_s * vn + naive_b - w) ** 2).sum()


def test_q4_chunks_are_independent():
    """Rows of one 64-row chunk quantise the same inside a larger matrix and alone."""
    rng = np.random.default_rng(5)
    m = (rng.standard_normal((192, 128)) * 0.05).astype(np.float32)
    p_all, sb_all = orc.quant_q4(m)
    p_mid, sb_mid = orc.quant_q4(m[64:128])
    assert np.array_equal(p_all[64:128], p_mid) and np.array_equal(sb_all[64:128], sb_mid)
    c_all, s_all = orc.quant_q8(m)
    c_mid, s_mid = orc.quant_q8(m[64:128])
    assert np.array_equal(c_all[64:128], c_mid) and np.array_equal(s_all[64:128], s_mid)


@pytest.mark.parametrize("threads", [1, 4])
def test_quantisers_do_not_depend_on_threads(threads):
    rng = np.random.default_rng(6)
    m = (rng.standard_normal((256, 192)) * 0.03).astype(np.float32)
    old = orc.get_threads()
    orc.set_threads(threads)
    try:
        a = orc.quant_q4(m), orc.quant_q8(m)
    finally:
        orc.set_threads(old)
    b = orc.quant_q4(m), orc.quant_q8(m)
    for x, y in zip(a, b):
        assert np.array_equal(x[0], y[0]) and np.array_equal(x[1], y[1])
