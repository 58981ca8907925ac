"""Pins the CPU oracle against what the mathematics fixes (CPU only).

The reference ships no golden vectors for this path, so each oracle function is checked
against closed forms, invariants, hand-computed known answers and an independent numpy
restatement written from tools/reference/qwen3vl_ref.py's formulation (vectorised matmuls,
rotate_half, repeat-GQA, additive causal mask, softmax), chosen so that a plausible mistake
(dropped term, wrong sign or index, transposed operand, wrong nibble order) fails one of them.
"""
import numpy as np
import pytest

from instantcua_amd import synth
from instantcua_amd.modelfile import Dims, TensorID, WeightFormat, matrix_bytes

H, FF, NH, NKV, HD = Dims.hidden, Dims.ff, Dims.heads, Dims.kv_heads, Dims.head_dim


# ------------------------------------------------------------------------------------------
# fp16 conversions

def test_fp16_roundtrip_matches_ieee(oracle_mod):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(2000).astype(np.float32) * np.float32(10) ** rng.integers(-8, 5, 2000),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e-8, 5.96e-8, 2.98e-8, 6.1e-5, -6.1e-5, np.inf, -np.inf],
                 dtype=np.float32),
    ])
    for v in vals:
        want = np.float32(v).astype(np.float16).view(np.uint16)
        assert oracle_mod.f2h(float(v)) == int(want), v
    for h in list(range(0, 0x7C00, 97)) + [0x0001, 0x03FF, 0x0400, 0x7BFF, 0x8001, 0xFBFF]:
        want = np.uint16(h).view(np.float16).astype(np.float32)
        assert oracle_mod.h2f(h) == float(want)


# ------------------------------------------------------------------------------------------
# Codecs: hand-computed known answers (Convert.swift:215-262; Shaders.swift:464-476)

def test_q4_known_answer(oracle_mod):
    # one row, K = 64: codes q_k = k % 16 packed low nibble first; s = 0.5, b = -1.25
    q = np.arange(64) % 16
    packed = (q[0::2] | (q[1::2] << 4)).astype(np.uint8)
    sb = np.array([0.5, -1.25], dtype=np.float16).view(np.uint8)
    w = oracle_mod.dequant(WeightFormat.Q4, packed, sb, 1, 64)[0]
    assert np.array_equal(w, 0.5 * q - 1.25)
    # nibble order: swapping nibbles must change the result
    swapped = ((packed >> 4) | (packed << 4)).astype(np.uint8)
    assert not np.array_equal(oracle_mod.dequant(WeightFormat.Q4, swapped, sb, 1, 64)[0], w)


def test_q4_dequant_is_fl32_of_s_q_plus_b(oracle_mod):
    m = synth.make_matrix(WeightFormat.Q4, 32, 2048, tag="kat")
    w = oracle_mod.dequant(WeightFormat.Q4, m.codes, m.sb, 32, 2048)
    codes = np.stack([m.codes & 15, m.codes >> 4], axis=-1).reshape(32, 2048).astype(np.float32)
    sb = m.sb.view(np.float16).reshape(32, 32, 2).astype(np.float32)
    s = np.repeat(sb[:, :, 0], 64, axis=1)
    b = np.repeat(sb[:, :, 1], 64, axis=1)
    want = (s * codes + b).astype(np.float32)  # numpy float32: round(s*q) exact, then + b rounded once
    assert np.array_equal(w.view(np.uint32), want.view(np.uint32))


def test_q8_known_answer(oracle_mod):
    codes = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    scale = np.array([0.125], dtype=np.float16).view(np.uint8)
    w = oracle_mod.dequant(WeightFormat.Q8, codes, scale, 1, 32)[0]
    assert np.array_equal(w, 0.125 * np.arange(-16, 16))


# ------------------------------------------------------------------------------------------
# GEMV against an independent numpy dequantisation

def _np_dequant(fmt, m):
    if fmt == WeightFormat.Q4:
        c = np.stack([m.codes & 15, m.codes >> 4], axis=-1).reshape(m.rows, m.cols).astype(np.float64)
        sb = m.sb.view(np.float16).reshape(m.rows, m.cols // 64, 2).astype(np.float64)
        return c * np.repeat(sb[:, :, 0], 64, 1) + np.repeat(sb[:, :, 1], 64, 1)
    if fmt == WeightFormat.Q8:
        c = m.codes.view(np.int8).reshape(m.rows, m.cols).astype(np.float64)
        return c * np.repeat(m.sb.view(np.float16).reshape(m.rows, -1).astype(np.float64), 32, 1)
    return m.codes.view(np.float16).reshape(m.rows, m.cols).astype(np.float64)


@pytest.mark.parametrize("fmt", [WeightFormat.Q4, WeightFormat.Q8, WeightFormat.F16])
def test_gemv_matches_numpy(oracle_mod, fmt):
    N, K = 64, 2048
    m = synth.make_matrix(fmt, N, K, tag="np-gemv", index=fmt)
    x = np.random.default_rng(1).standard_normal((3, K)).astype(np.float32)
    y = oracle_mod.gemv(fmt, m.codes, m.sb, N, K, x)
    want = x.astype(np.float64) @ _np_dequant(fmt, m).T
    assert np.max(np.abs(y - want)) <= 1e-6 * np.max(np.abs(want))


# ------------------------------------------------------------------------------------------
# M-RoPE table (Engine.swift:121-125, 254-298; qwen3vl_ref.py:87-118)

def _np_mrope(maxctx, vis_offset, llm_h, llm_w):
    invf = 1.0 / (5e6 ** (np.arange(64) * 2 / 128.0))
    n_vis = llm_h * llm_w
    delta = max(llm_h, llm_w) - n_vis
    out = np.empty((maxctx, 64, 2), np.float32)
    for slot in range(maxctx):
        if vis_offset < 0 or slot < vis_offset:
            t = h = w = slot
        elif slot < vis_offset + n_vis:
            v = slot - vis_offset
            t, h, w = vis_offset, vis_offset + v // llm_w, vis_offset + v % llm_w
        else:
            t = h = w = slot + delta
        for i in range(64):
            p = h if (i < 60 and i % 3 == 1) else w if (i < 60 and i % 3 == 2) else t
            ang = float(np.float32(p) * np.float32(invf[i]))
            out[slot, i] = (np.float32(np.cos(ang)), np.float32(np.sin(ang)))
    return out


def test_mrope_text_only_is_1d_rope(oracle_mod):
    tab = oracle_mod.mrope_table(300, -1, 1, 1)
    assert np.array_equal(tab, _np_mrope(300, -1, 1, 1))
    # 1-D RoPE closed form (float64 reference, fp32 rounding of the angle allowed)
    invf = 1.0 / (5e6 ** (np.arange(64) * 2 / 128.0))
    p = np.arange(300)[:, None] * invf[None, :]
    assert np.max(np.abs(tab[:, :, 0] - np.cos(p))) < 1e-4
    assert np.max(np.abs(tab[:, :, 1] - np.sin(p))) < 1e-4


def test_mrope_vision_grid_sections(oracle_mod):
    vo, lh, lw = 7, 3, 5
    tab = oracle_mod.mrope_table(64, vo, lh, lw)
    assert np.array_equal(tab, _np_mrope(64, vo, lh, lw))
    # the visual slot of grid cell (r, c) uses T = vo, H = vo + r, W = vo + c on the interleave
    invf = 1.0 / (5e6 ** (np.arange(64) * 2 / 128.0))
    r, c = 2, 3
    slot = vo + r * lw + c
    for i in range(64):
        p = vo + r if (i < 60 and i % 3 == 1) else vo + c if (i < 60 and i % 3 == 2) else vo
        assert abs(tab[slot, i, 0] - np.cos(np.float32(p) * np.float32(invf[i]))) < 1e-6
    # text after the image continues at slot + max(h, w) - n_vis (rope_delta)
    after = vo + lh * lw
    want_p = after + 2 + max(lh, lw) - lh * lw
    assert abs(tab[after + 2, 0, 0] - np.cos(float(np.float32(want_p)))) < 1e-6


def test_mrope_matches_reference_float32_formulation(oracle_mod):
    """qwen3vl_ref.compute_mrope_cos_sin evaluates in float32 numpy; the engine table uses a
    double inv-freq and double cos.  They agree to fp32 precision."""
    vo, lh, lw, L = 4, 4, 6, 48
    n_vis = lh * lw
    pos = np.zeros((3, L), np.float32)
    pos[:, :vo] = np.arange(vo)
    for rr in range(lh):
        for cc in range(lw):
            pos[:, vo + rr * lw + cc] = (vo, vo + rr, vo + cc)
    after = vo + max(lh, lw)
    for i in range(vo + n_vis, L):
        pos[:, i] = after + (i - (vo + n_vis))
    inv = 1.0 / (5e6 ** (np.arange(0, 128, 2, dtype=np.float32) / 128))
    ft, fh, fw = (pos[j, :, None] * inv[None, :] for j in range(3))
    f = ft.copy()
    f[:, 1:60:3] = fh[:, 1:60:3]
    f[:, 2:60:3] = fw[:, 2:60:3]
    tab = oracle_mod.mrope_table(L, vo, lh, lw)
    assert np.max(np.abs(tab[:, :, 0] - np.cos(f))) < 2e-5
    assert np.max(np.abs(tab[:, :, 1] - np.sin(f))) < 2e-5


# ------------------------------------------------------------------------------------------
# One decoder layer against an independent numpy restatement of qwen3vl_ref.py:247-277


def _np_rmsnorm(x, w, eps=np.float64(np.float32(1e-6))):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def _np_rotate_half(x):
    d = x.shape[-1] // 2
    return np.concatenate([-x[..., d:], x[..., :d]], axis=-1)


class _NpLayer:
    def __init__(self, img, fmt, l):
        self.fmt = fmt
        tab = img[16:16 + TensorID.count * 16].view("<u8").reshape(-1, 2)

        def arr(tid, dtype):
            off, n = int(tab[tid, 0]), int(tab[tid, 1])
            return img[off:off + n].view(dtype)

        L = lambda k: TensorID.llm_layer(l, k)

        def mat(wid, sid, rows, cols):
            c = arr(L(wid), np.uint8)
            s = arr(L(sid), np.uint8)
            return _np_dequant(fmt, synth.QMatrix(fmt, rows, cols, c, s))

        self.attn_norm = arr(L(TensorID.attn_norm), np.float32).astype(np.float64)
        self.q_norm = arr(L(TensorID.q_norm), np.float32).astype(np.float64)
        self.k_norm = arr(L(TensorID.k_norm), np.float32).astype(np.float64)
        self.mlp_norm = arr(L(TensorID.mlp_norm), np.float32).astype(np.float64)
        qkv = mat(TensorID.wqkv, TensorID.wqkv_sb, Dims.qkv_rows, H)
        self.wq, self.wk, self.wv = qkv[:H], qkv[H:H + NKV * HD], qkv[H + NKV * HD:]
        self.wo = mat(TensorID.wo, TensorID.wo_sb, H, H)
        gu = mat(TensorID.wgu, TensorID.wgu_sb, Dims.gu_rows, H)
        self.wg, self.wu = gu[:FF], gu[FF:]
        self.wd = mat(TensorID.wd, TensorID.wd_sb, H, FF)

    def forward(self, x, k_prior, v_prior, cos, sin):
        """x [n, H]; k/v_prior [NKV, pos, HD] (float); cos/sin [n, 128] for the new rows."""
        n = x.shape[0]
        pos = k_prior.shape[1]
        h = _np_rmsnorm(x, self.attn_norm)
        q = (h @ self.wq.T).reshape(n, NH, HD)
        k = (h @ self.wk.T).reshape(n, NKV, HD)
        v = (h @ self.wv.T).reshape(n, NKV, HD)
        q = _np_rmsnorm(q, self.q_norm)
        k = _np_rmsnorm(k, self.k_norm)
        q = q * cos[:, None, :] + _np_rotate_half(q) * sin[:, None, :]
        k = k * cos[:, None, :] + _np_rotate_half(k) * sin[:, None, :]
        k16 = k.astype(np.float32).astype(np.float16).astype(np.float64)  # fp16 cache
        v16 = v.astype(np.float32).astype(np.float16).astype(np.float64)
        K = np.concatenate([k_prior, np.transpose(k16, (1, 0, 2))], axis=1)  # [NKV, L, HD]
        V = np.concatenate([v_prior, np.transpose(v16, (1, 0, 2))], axis=1)
        Kr = np.repeat(K, 2, axis=0)  # GQA 16:8
        Vr = np.repeat(V, 2, axis=0)
        qt = np.transpose(q, (1, 0, 2))  # [NH, n, HD]
        scores = qt @ np.transpose(Kr, (0, 2, 1)) * (128.0 ** -0.5)
        Ltot = pos + n
        mask = np.triu(np.full((n, Ltot), -1e9), k=pos + 1)
        scores = scores + mask
        scores = scores - scores.max(-1, keepdims=True)
        p = np.exp(scores)
        p /= p.sum(-1, keepdims=True)
        att = np.transpose(p @ Vr, (1, 0, 2)).reshape(n, H)
        x = x + att @ self.wo.T
        h2 = _np_rmsnorm(x, self.mlp_norm)
        g = h2 @ self.wg.T
        u = h2 @ self.wu.T
        act = g / (1.0 + np.exp(-g)) * u
        return x + act @ self.wd.T, att


@pytest.mark.parametrize("fmt", [WeightFormat.Q4, WeightFormat.Q8])
def test_layer_matches_numpy_reference(oracle_mod, fmt):
    img = synth.build_model_image(fmt, n_layers=1, tag=f"pin{fmt}")
    pos, n = 11, 3
    kc = synth.fp16_normal((NKV, pos, HD), "pin-k")
    vc = synth.fp16_normal((NKV, pos, HD), "pin-v")
    x = synth.fp16_normal((n, H), "pin-x").astype(np.float32)
    om = oracle_mod.OracleModel(img, 64)
    om.kv(0, 0)[:, :pos] = kc
    om.kv(0, 1)[:, :pos] = vc
    got, _, got_att, _ = om.layer_taps(0, x, pos)
    tab = oracle_mod.mrope_table(64, -1, 1, 1)
    cos = np.concatenate([tab[pos:pos + n, :, 0]] * 2, axis=1).astype(np.float64)
    sin = np.concatenate([tab[pos:pos + n, :, 1]] * 2, axis=1).astype(np.float64)
    want, want_att = _NpLayer(img, fmt, 0).forward(x.astype(np.float64), kc.astype(np.float64),
                                                   vc.astype(np.float64), cos, sin)
    assert np.max(np.abs(got_att - want_att)) <= 1e-5 * np.max(np.abs(want_att))
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
    # the new K rows are the fp16 rounding of the rotated, normalised k
    assert np.array_equal(om.kv(0, 0)[:, :pos].view(np.uint16), kc.view(np.uint16))


def test_single_slot_attention_returns_v(oracle_mod):
    """With one cache slot softmax is 1: each head's output is its KV group's (fp16) v row,
    which pins the head -> group mapping h // 2."""
    img = synth.build_model_image(WeightFormat.Q4, n_layers=1, tag="pin1")
    om = oracle_mod.OracleModel(img, 8)
    x = synth.fp16_normal((1, H), "pin1-x").astype(np.float32)
    _, qkv, att, _ = om.layer_taps(0, x, 0)
    v = qkv[0, H + NKV * HD:].reshape(NKV, HD).astype(np.float16).astype(np.float32)
    for h in range(NH):
        assert np.array_equal(att[0, h * HD:(h + 1) * HD], v[h // 2])
    assert np.array_equal(om.kv(0, 1)[:, 0].astype(np.float32), v)


def test_lm_head_scale_invariance(oracle_mod):
    """RMSNorm makes the logits invariant to scaling the residual (up to eps)."""
    img = synth.build_model_image(WeightFormat.Q4, n_layers=1, tag="pin2")
    om = oracle_mod.OracleModel(img, 8)
    x = synth.fp16_normal((H,), "pin2-x").astype(np.float32)
    a = om.lm_head(x)
    b = om.lm_head(np.float32(8.0) * x)
    assert np.max(np.abs(a - b)) <= 1e-6 * np.max(np.abs(a))
    assert om.lm_head(-x).argmax() != a.argmax() or np.allclose(a, 0)


def test_deepstack_and_visual_rows(oracle_mod):
    """Visual rows take the pooler embeddings; DeepStack adds after layers 0-2 only at them."""
    img = synth.build_model_image(WeightFormat.Q4, n_layers=1, tag="pin3")
    vp = synth.visual_prompt(12, vis_offset=3, llm_h=2, llm_w=2, tag="pin3")
    pool = vp.pooler.astype(np.float32)
    ds = [d.astype(np.float32) for d in vp.deepstack]
    om = oracle_mod.OracleModel(img, 32)
    om.prepare_mrope(3, 2, 2)
    base = om.run_pass(vp.tokens, 0, pooler=pool, vis_offset=3, logits_rows=12)
    om2 = oracle_mod.OracleModel(img, 32)
    om2.prepare_mrope(3, 2, 2)
    with_ds = om2.run_pass(vp.tokens, 0, pooler=pool, vis_offset=3, deepstack=ds, logits_rows=12)
    changed = np.abs(with_ds - base).max(axis=1) > 0
    # one layer: DeepStack touches only the visual rows (their own logits), text rows unchanged
    assert changed[3:7].all() and not changed[:3].any() and not changed[7:].any()
    # the pooler rows replace the token embedding of image-pad rows
    om3 = oracle_mod.OracleModel(img, 32)
    om3.prepare_mrope(3, 2, 2)
    pool2 = pool.copy()
    pool2[1] += 1.0
    other = om3.run_pass(vp.tokens, 0, pooler=pool2, vis_offset=3, logits_rows=12)
    diff = np.abs(other - base).max(axis=1) > 0
    assert not diff[:4].any() and diff[4:].all()  # row 4 and everything after attends to it


def test_greedy_decode_is_consistent_with_passes(oracle_mod):
    """or_generate equals explicit prefill + single-token passes (token feedback, positions)."""
    img = synth.build_model_image(WeightFormat.Q4, n_layers=1, tag="pin4")
    toks = synth.random_tokens(6, "pin4")
    om = oracle_mod.OracleModel(img, 32)
    out, margins, first, top1 = om.generate(toks, 4, with_top1=True)
    om2 = oracle_mod.OracleModel(img, 32)
    lg = om2.run_pass(toks, 0)[0]
    assert np.array_equal(lg, first) and lg.argmax() == out[0] and top1[0] == lg.max()
    seq = [int(out[0])]
    for s in range(1, 4):
        lg = om2.run_pass(np.array([seq[-1]], np.int32), len(toks) + s - 1)[0]
        seq.append(int(lg.argmax()))
        srt = np.sort(lg)
        assert abs((srt[-1] - srt[-2]) - margins[s]) < 1e-6
        assert top1[s] == srt[-1]
    assert seq == list(out)


def _scaled_embedding(img, scales):
    from instantcua_amd.modelfile import TensorID as T
    img = img.copy()
    table = np.frombuffer(img[16:16 + 16 * T.count].tobytes(), dtype="<u8").reshape(-1, 2)
    off = int(table[T.embed_sb, 0])
    sb = img[off:off + Dims.vocab * (Dims.hidden // 64) * 4].view(np.float16).reshape(Dims.vocab, -1, 2)
    for tok, c in scales.items():
        sb[tok] = (sb[tok].astype(np.float32) * c).astype(np.float16)
    return img


def test_commit_loop_without_grammar_is_plain_greedy(oracle_mod):
    img = synth.build_model_image(WeightFormat.Q4, n_layers=1, tag="pin5")
    toks = synth.random_tokens(6, "pin5")
    a = oracle_mod.OracleModel(img, 32).generate_commit(toks, 5)
    b, _, _ = oracle_mod.OracleModel(img, 32).generate(toks, 5)
    assert np.array_equal(a, b)
    # EOS ends the loop with the EOS token as its last entry.
    c = oracle_mod.OracleModel(img, 32).generate_commit(toks, 5, eos=(int(b[2]), -1))
    assert list(c) == list(b[:3])


def test_commit_loop_grammar_pairs_replay_as_explicit_passes(oracle_mod):
    """With grammar pairs the loop equals explicit passes: a forced token follows 11 (220) or a
    step-1 action token (7), the next pass carries both tokens at consecutive slots and commits
    its last row's argmax; ")" (8) ends the loop."""
    img = _scaled_embedding(synth.build_model_image(WeightFormat.Q4, n_layers=1, tag="pin6"),
                            {11: 8, 3678: 16, 8: 3})
    actions = {3678, 7241, 12476, 10855, 11862, 1339, 1472, 24769}
    fired = set()
    for seed in range(6):
        toks = synth.random_tokens(7, "pin6", seed)
        out = [int(t) for t in oracle_mod.OracleModel(img, 64).generate_commit(toks, 14, grammar=True)]
        om = oracle_mod.OracleModel(img, 64)
        pos, step, seq = 0, 0, []
        pass_toks = np.asarray(toks, np.int32)
        while step < 14:
            tok = int(om.run_pass(pass_toks, pos)[0].argmax())
            pos += pass_toks.size
            seq.append(tok)
            step += 1
            if tok == 8 or step >= 14:
                break
            if (step == 1 and tok in actions) or tok == 11:
                forced = 220 if tok == 11 else 7
                seq.append(forced)
                step += 1
                pass_toks = np.array([tok, forced], np.int32)
            else:
                pass_toks = np.array([tok], np.int32)
        assert out == seq, (seed, out, seq)
        assert 8 not in out[:-1]
        fired |= {"pair 11" for a, b in zip(out, out[1:]) if (a, b) == (11, 220)}
        fired |= {"stop )"} if out[-1] == 8 else set()
        fired |= {"action"} if out[:2] == [3678, 7] else set()
    assert fired >= {"pair 11", "stop )"}, fired  # the scaled rows make the rules fire


# ------------------------------------------------------------------------------------------
# Greedy argmax ties (Shaders.swift:1514-1536: the lower token id wins an equal logit)

def tie_models(oracle_mod, steps=6):
    """A 2-layer q4 model, its greedy run, and for tie steps k = 0 and k = 3 a copy of the image
    in which a lower id u takes the embedding row of the step's winner t (so logit u == logit t
    at every step): (image, prompt, plain greedy, [(k, t, u, image_k)])."""
    img = synth.build_model_image(WeightFormat.Q4, n_layers=2, tag="argmax-tie")
    toks = synth.random_tokens(16, "argmax-tie-prompt")
    om = oracle_mod.OracleModel(img, 64)
    ref, _, _ = om.generate(toks, steps)
    om.close()
    cases = []
    for k in (0, 3):
        t = int(ref[k])
        assert t not in ref[:k].tolist(), "pick a step whose winner is new (no earlier tie)"
        used = set(toks.tolist()) | set(ref[:k + 1].tolist())
        u = next(i for i in range(t - 1, -1, -1) if i not in used)
        img_k = img.copy()
        synth.copy_embedding_row(img_k, t, u)
        cases.append((k, t, u, img_k))
    return img, toks, ref, cases


def test_argmax_tie_takes_the_lower_id(oracle_mod):
    _, toks, ref, cases = tie_models(oracle_mod)
    for k, t, u, img_k in cases:
        om = oracle_mod.OracleModel(img_k, 64)
        got, _, first = om.generate(toks, len(ref))
        om.close()
        if k == 0:
            assert first[u] == first[t] and first[u] == first.max()
        assert np.array_equal(got[:k], ref[:k]), (k, got, ref)
        assert int(got[k]) == u, (k, t, u, got)
