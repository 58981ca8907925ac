"""Pins of the oracle's vision-tower restatement (oracle/vision.c) against independent
formulations: einops patch layout, closed forms of the bilinear table and RoPE angles, float64
numpy LayerNorm / products / attention, math.erf and math.tanh GELU, and a whole-tower special
case (zero blocks: every block is the identity) evaluated in float64 numpy from the image's own
tensors.  References: Sources/Engine/Engine.swift:189-246, 317-473; Shaders.swift:59-454;
tools/reference/qwen3vl_ref.py:25-85, 142-216."""
import math

import numpy as np
import pytest
from einops import rearrange

from instantcua_amd import synth
from instantcua_amd.modelfile import Dims, TensorID, WeightFormat


@pytest.fixture(autouse=True)
def _o(oracle_mod):
    global o
    o = oracle_mod


def test_patchify_is_the_merge_block_layout():
    """Patch p = ((block row, block col), (in-row, in-col)), element (channel, dy, dx)."""
    gh, gw = 4, 6
    rgb = np.random.default_rng(1).integers(0, 256, (16 * gh, 16 * gw, 3)).astype(np.uint8)
    got = o.vit_patchify(rgb)
    val = (rgb.astype(np.float32) * np.float32(2.0 / 255.0) - np.float32(1.0)).astype(np.float16)
    want = rearrange(val, "(bh ir py) (bw ic px) c -> (bh bw ir ic) (c py px)", ir=2, ic=2, py=16, px=16)
    assert np.array_equal(got.view(np.uint16), np.ascontiguousarray(want).view(np.uint16))
    # The normalisation maps 0 and 255 to -1 and 1 exactly.
    edge = np.zeros((32, 32, 3), np.uint8)
    edge[0, 0, 0] = 255
    p = o.vit_patchify(edge)
    assert p[0, 0] == 1.0 and p[0, 1] == -1.0


def _grid_rc(gh, gw):
    """(row, col) of each patch in merge-block order, from the patch layout itself: an image
    whose red channel is the patch row and green channel the patch column."""
    img = np.zeros((16 * gh, 16 * gw, 3), np.uint8)
    img[..., 0] = (np.arange(16 * gh) // 16)[:, None]
    img[..., 1] = (np.arange(16 * gw) // 16)[None, :]
    p = o.vit_patchify(img).astype(np.float32)
    to_u8 = lambda v: np.rint((v + 1.0) * 255.0 / 2.0).astype(int)
    return to_u8(p[:, 0]), to_u8(p[:, 256])


def test_pos_interp_hits_the_table_on_a_48_grid_and_is_exact_on_linear_tables():
    table = np.random.default_rng(2).standard_normal((48 * 48, 1024)).astype(np.float32)
    r, c = _grid_rc(48, 48)
    got = o.vit_pos_interp(table, 48, 48)
    assert np.array_equal(got, table[r * 48 + c])
    # A table affine in (row, col) interpolates to the affine function (align_corners=True).
    a, b, k = (np.random.default_rng(3).uniform(-1, 1, (3, 1024))).astype(np.float32)
    yy, xx = np.mgrid[0:48, 0:48]
    lin = (yy.reshape(-1, 1) * a + xx.reshape(-1, 1) * b + k).astype(np.float32)
    for gh, gw in ((6, 10), (24, 40), (2, 2)):
        r, c = _grid_rc(gh, gw)
        y = r * 47.0 / max(gh - 1, 1)
        x = c * 47.0 / max(gw - 1, 1)
        want = y[:, None] * a + x[:, None] * b + k
        got = o.vit_pos_interp(lin, gh, gw)
        assert np.abs(got - want).max() < 1e-4 * np.abs(want).max(), (gh, gw)


def test_rope_table_angles_follow_patch_rows_and_columns():
    gh, gw = 6, 8
    t = o.vit_rope_table(gh, gw).astype(np.float64)
    assert np.allclose(t[..., 0] ** 2 + t[..., 1] ** 2, 1.0, atol=1e-6)
    r, c = _grid_rc(gh, gw)
    ang = np.arctan2(t[..., 1], t[..., 0])
    # Frequency 0 is 1: the angle is the row (j = 0) or column (j = 16) index itself, mod 2 pi.
    wrap = lambda v: (v + np.pi) % (2 * np.pi) - np.pi
    assert np.allclose(ang[:, 0], wrap(r), atol=1e-6) and np.allclose(ang[:, 16], wrap(c), atol=1e-6)
    # Frequency i is 10000^(-i / 16); small angles are unwrapped.
    f = 10000.0 ** (-np.arange(16) / 16.0)
    assert np.allclose(ang[:, 15], r * f[15], atol=1e-6) and np.allclose(ang[:, 31], c * f[15], atol=1e-6)
    # The origin patch is unrotated.
    assert np.array_equal(t[0, :, 0], np.ones(32)) and np.array_equal(t[0, :, 1], np.zeros(32))


def test_layernorm_against_float64():
    rng = np.random.default_rng(4)
    for n in (1024, 4096):
        x = (rng.standard_normal((5, n)) * 3 + 1).astype(np.float32)
        w = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        got = o.layernorm_f16(x, w, b).astype(np.float64)
        xd = x.astype(np.float64)
        want = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-6) * w + b
        assert np.all(np.abs(got - want) <= 2 ** -10 * np.abs(want) + 1e-7), n
        # A constant row normalises to the bias exactly.
        c = o.layernorm_f16(np.full((1, n), 2.5, np.float32), w, b)
        assert np.array_equal(c[0], b.astype(np.float16))


def test_linear_against_float64():
    rng = np.random.default_rng(5)
    X = rng.standard_normal((7, 192)).astype(np.float16)
    W = rng.standard_normal((40, 192)).astype(np.float16)
    bias = rng.standard_normal(40).astype(np.float32)
    got = o.linear_f16(X, W, bias)
    want = X.astype(np.float64) @ W.astype(np.float64).T + bias
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()
    # Row / column roles: X row 3 against W row 5 only.
    e = np.zeros_like(W)
    e[5] = W[5]
    assert np.count_nonzero(o.linear_f16(X, e, np.zeros(40, np.float32))[:, [i for i in range(40) if i != 5]]) == 0


def test_gelu_against_math():
    for x in (-6.0, -1.5, -0.3, 0.0, 0.2, 1.0, 3.7, 9.0):
        xf = float(np.float32(x))
        assert o.gelu_erf(x) == pytest.approx(0.5 * xf * (1 + math.erf(xf / math.sqrt(2))), rel=1e-6, abs=1e-7)
        assert o.gelu_tanh(x) == pytest.approx(
            0.5 * xf * (1 + math.tanh(math.sqrt(2 / math.pi) * (xf + 0.044715 * xf ** 3))), rel=1e-6, abs=1e-7)
    # The two forms differ (tanh is an approximation of erf).
    assert abs(o.gelu_erf(1.0) - o.gelu_tanh(1.0)) > 1e-5


def test_attention_against_float64():
    rng = np.random.default_rng(6)
    n = 40
    q, k, v = (rng.standard_normal((3, 16, n, 64)) * 1.5).astype(np.float16)
    got = o.vit_attention(q, k, v).astype(np.float64).reshape(n, 16, 64)
    s = np.einsum("hqd,hkd->hqk", q.astype(np.float64), k.astype(np.float64)) / 8.0
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    want = np.einsum("hqk,hkd->qhd", p, v.astype(np.float64))
    # fp16 probabilities and output: a few fp16 ulps of the largest values.
    assert np.abs(got - want).max() < 4e-3 * np.abs(want).max()
    # Attention is bidirectional: the first query attends to the last key.
    v2 = v.copy()
    v2[:, -1] += np.float16(4.0)
    assert not np.array_equal(o.vit_attention(q, k, v2)[0], o.vit_attention(q, k, v)[0])


def _ln64(x, w, b):
    x = x.astype(np.float64)
    return ((x - x.mean(-1, keepdims=True)) / np.sqrt(x.var(-1, keepdims=True) + 1e-6) * w + b).astype(np.float16)


def test_whole_tower_with_identity_blocks():
    """Zero block tensors make every block the identity: the tower reduces to patch embedding +
    interpolated positions, then the mergers, which float64 numpy evaluates from the image."""
    img = synth.build_model_image(WeightFormat.Q4, n_layers=0, tag="vis-zero", vision=True, zero_vision_blocks=True)
    gh, gw = 4, 6
    rgb = synth.random_rgb(gh, gw, "vis-zero")
    pooler, ds = o.vision(img, rgb)

    table = np.frombuffer(img[16:16 + 16 * TensorID.count].tobytes(), dtype="<u8").reshape(-1, 2)

    def T(tid, dt, shape):
        off, n = int(table[tid, 0]), int(table[tid, 1])
        return img[off:off + n].view(dt).reshape(shape)

    # Patches and positions from the layout rule restated with einops and a numpy bilinear form.
    val = (rgb.astype(np.float32) * np.float32(2.0 / 255.0) - np.float32(1.0)).astype(np.float16)
    patches = rearrange(val, "(bh ir py) (bw ic px) c -> (bh bw ir ic) (c py px)", ir=2, ic=2, py=16, px=16)
    pos = T(TensorID.vit_pos_emb, np.float32, (48, 48, 1024)).astype(np.float64)
    r, c = _grid_rc(gh, gw)
    y, x = r * 47.0 / (gh - 1), c * 47.0 / (gw - 1)
    y0, x0 = np.floor(y).astype(int), np.floor(x).astype(int)
    y1, x1 = np.minimum(y0 + 1, 47), np.minimum(x0 + 1, 47)
    dy, dx = (y - y0)[:, None], (x - x0)[:, None]
    pe = (1 - dy) * ((1 - dx) * pos[y0, x0] + dx * pos[y0, x1]) + dy * ((1 - dx) * pos[y1, x0] + dx * pos[y1, x1])
    X = patches.astype(np.float64) @ T(TensorID.vit_patch_w, np.float16, (1024, 768)).astype(np.float64).T \
        + T(TensorID.vit_patch_b, np.float32, (1024,)) + pe
    nvis = gh * gw // 4
    gelu = np.vectorize(lambda v: 0.5 * v * (1 + math.erf(v / math.sqrt(2))))

    def merger(i, xn):
        M = lambda k, dt, shape: T(TensorID.merger(i, k), dt, shape).astype(np.float64)
        h = xn.astype(np.float64) @ M(TensorID.m_fc1_w, np.float16, (4096, 4096)).T + M(TensorID.m_fc1_b, np.float32, (4096,))
        h = gelu(h).astype(np.float16).astype(np.float64)
        return h @ M(TensorID.m_fc2_w, np.float16, (2048, 4096)).T + M(TensorID.m_fc2_b, np.float32, (2048,))

    for i in range(3):
        xn = _ln64(X.reshape(nvis, 4096), T(TensorID.merger(i, 0), np.float32, (4096,)),
                   T(TensorID.merger(i, 1), np.float32, (4096,)))
        want = merger(i, xn)
        assert np.abs(ds[i] - want).max() < 1e-2 * np.abs(want).max(), i
    xn = _ln64(X, T(TensorID.merger(3, 0), np.float32, (1024,)), T(TensorID.merger(3, 1), np.float32, (1024,)))
    want = merger(3, xn.reshape(nvis, 4096))
    err = np.abs(pooler - want).max() / np.abs(want).max()
    assert err < 1e-2, err
    # Identity blocks leave the three DeepStack inputs equal, so the three mergers see one x.
    assert not np.array_equal(ds[0], ds[1])  # different merger weights, same input


def test_vision_rejects_bad_grids():
    img = np.zeros(16384, np.uint8)
    with pytest.raises(RuntimeError):
        o.vision(img, np.zeros((48, 64, 3), np.uint8))  # 3 x 4 grid: odd side


def _tensor_view(img, tid, dt, shape):
    table = np.frombuffer(img[16:16 + 16 * TensorID.count].tobytes(), dtype="<u8").reshape(-1, 2)
    off, n = int(table[tid, 0]), int(table[tid, 1])
    return img[off:off + n].view(dt).reshape(shape)


def test_one_block_against_float64():
    """A block with random weights on random residual rows, against the reference's block math
    (qwen3vl_ref.py:178-197: qkv reshaped [np][3][16][64], q * cos + rotate_half(q) * sin with the
    angles of the row / column halves repeated, softmax over all patches, GELU-tanh MLP) in
    float64, with the engine's fp16 rounding of the LayerNorm outputs."""
    img = synth.build_model_image(WeightFormat.Q4, n_layers=0, tag="vis-blk", vision=True, zero_vision_blocks=True)
    l, gh, gw = 7, 4, 6
    rng = np.random.default_rng(8)
    V = lambda k, dt, shape: _tensor_view(img, TensorID.vit_layer(l, k), dt, shape)
    shapes = {TensorID.v_norm1_w: (1024,), TensorID.v_norm1_b: (1024,), TensorID.v_qkv_w: (3072, 1024),
              TensorID.v_qkv_b: (3072,), TensorID.v_proj_w: (1024, 1024), TensorID.v_proj_b: (1024,),
              TensorID.v_norm2_w: (1024,), TensorID.v_norm2_b: (1024,), TensorID.v_fc1_w: (4096, 1024),
              TensorID.v_fc1_b: (4096,), TensorID.v_fc2_w: (1024, 4096), TensorID.v_fc2_b: (1024,)}
    for k, shape in shapes.items():
        dt = np.float16 if len(shape) == 2 else np.float32
        sd = {TensorID.v_qkv_w: 0.06, TensorID.v_proj_w: 0.05, TensorID.v_fc1_w: 0.04, TensorID.v_fc2_w: 0.03}.get(k, 0.1)
        base = 1.0 if k in (TensorID.v_norm1_w, TensorID.v_norm2_w) else 0.0
        V(k, dt, shape)[:] = (base + sd * rng.standard_normal(shape)).astype(dt)
    np_ = gh * gw
    x = rng.standard_normal((np_, 1024)).astype(np.float32)
    got = o.vit_block(img, l, x, gh, gw)

    W = {k: V(k, np.float16 if len(s) == 2 else np.float32, s).astype(np.float64) for k, s in shapes.items()}
    r, c = _grid_rc(gh, gw)
    inv = 1.0 / 10000.0 ** (np.arange(0, 32, 2) / 32.0)
    fhw = np.concatenate([r[:, None] * inv, c[:, None] * inv], axis=1)
    ang = np.concatenate([fhw, fhw], axis=1)[:, None, :]  # [np][1][64]
    cos, sin = np.cos(ang), np.sin(ang)
    rot = lambda t: np.concatenate([-t[..., 32:], t[..., :32]], axis=-1)
    h = _ln64(x, W[TensorID.v_norm1_w], W[TensorID.v_norm1_b]).astype(np.float64)
    qkv = (h @ W[TensorID.v_qkv_w].T + W[TensorID.v_qkv_b]).reshape(np_, 3, 16, 64)
    q = qkv[:, 0] * cos + rot(qkv[:, 0]) * sin
    k = qkv[:, 1] * cos + rot(qkv[:, 1]) * sin
    v = qkv[:, 2]
    s = np.einsum("qhd,khd->hqk", q, k) / 8.0
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    a = np.einsum("hqk,khd->qhd", p, v).reshape(np_, 1024)
    x1 = x + a @ W[TensorID.v_proj_w].T + W[TensorID.v_proj_b]
    h2 = _ln64(x1, W[TensorID.v_norm2_w], W[TensorID.v_norm2_b]).astype(np.float64)
    f = h2 @ W[TensorID.v_fc1_w].T + W[TensorID.v_fc1_b]
    f = 0.5 * f * (1 + np.tanh(math.sqrt(2 / math.pi) * (f + 0.044715 * f ** 3)))
    want = x1 + f @ W[TensorID.v_fc2_w].T + W[TensorID.v_fc2_b]
    d_got, d_want = got - x, want - x
    err = np.abs(d_got - d_want).max() / np.abs(d_want).max()
    assert err < 1e-2, err
    # The attention branch alone is resolved too (it is not hidden by the MLP).
    a_part = a @ W[TensorID.v_proj_w].T
    assert np.abs(a_part).max() > 20 * err * np.abs(d_want).max()
