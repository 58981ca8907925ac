"""ctypes bindings of the CPU oracle (oracle/liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests, the smoke check and the CPU-baseline leg of the benchmark import this
module; the product package never does.  The arithmetic contract is in oracle.h.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

H, FF, NH, NKV, HD, QKV, GU, VOCAB = 2048, 6144, 16, 8, 128, 4096, 12288, 151936

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def build(force: bool = False) -> str:
    """Compile liboracle.so with the Makefile next to this file."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "all", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.or_h2f.argtypes = [C.c_uint16]
        L.or_h2f.restype = C.c_float
        L.or_f2h.argtypes = [C.c_float]
        L.or_f2h.restype = C.c_uint16
        L.or_dequant.argtypes = [C.c_int, _u8p, C.c_void_p, C.c_int, C.c_int, _f32p]
        L.or_gemv.argtypes = [C.c_int, _u8p, C.c_void_p, C.c_int, C.c_int, _f32p, C.c_int, _f32p]
        L.or_mrope_table.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, _f32p]
        L.or_model_new.argtypes = [C.c_void_p, C.c_size_t, C.c_int]
        L.or_model_new.restype = C.c_void_p
        L.or_model_free.argtypes = [C.c_void_p]
        L.or_model_layers.argtypes = [C.c_void_p]
        L.or_model_format.argtypes = [C.c_void_p]
        L.or_last_error.restype = C.c_char_p
        L.or_prepare_mrope.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int]
        L.or_kv.argtypes = [C.c_void_p, C.c_int, C.c_int]
        L.or_kv.restype = C.POINTER(C.c_uint16)
        L.or_layer.argtypes = [C.c_void_p, C.c_int, _f32p, C.c_int, C.c_int]
        L.or_debug_taps.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
        L.or_embed.argtypes = [C.c_void_p, C.c_int, _f32p]
        L.or_lm_head.argtypes = [C.c_void_p, _f32p, _f32p]
        L.or_pass.argtypes = [C.c_void_p, _i32p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                              C.c_int, C.c_void_p]
        L.or_argmax.argtypes = [_f32p, C.c_int]
        L.or_generate.argtypes = [C.c_void_p, _i32p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int,
                                  _i32p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.or_generate_commit.argtypes = [C.c_void_p, _i32p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                         C.c_int, C.c_int, C.c_int, C.c_int, _i32p]
        L.or_quant_q8.argtypes = [_f32p, C.c_int, C.c_int, C.c_void_p, _u16p]
        L.or_quant_q4.argtypes = [_f32p, C.c_int, C.c_int, _u8p, _u16p]
        L.or_vit_patchify.argtypes = [_u8p, C.c_int, C.c_int, _u16p]
        L.or_vit_pos_interp.argtypes = [_f32p, C.c_int, C.c_int, _f32p]
        L.or_vit_rope_table.argtypes = [C.c_int, C.c_int, _f32p]
        L.or_layernorm_f16.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, _u16p]
        L.or_linear_f16.argtypes = [_u16p, _u16p, _f32p, C.c_int, C.c_int, C.c_int, _f32p]
        L.or_gelu_tanh.argtypes = [C.c_float]
        L.or_gelu_tanh.restype = C.c_float
        L.or_gelu_erf.argtypes = [C.c_float]
        L.or_gelu_erf.restype = C.c_float
        L.or_vit_attention.argtypes = [_u16p, _u16p, _u16p, C.c_int, _u16p]
        L.or_vision.argtypes = [C.c_void_p, C.c_size_t, _u8p, C.c_int, C.c_int, _f32p, C.c_void_p]
        L.or_vision_error.restype = C.c_char_p
        L.or_vit_block.argtypes = [C.c_void_p, C.c_size_t, C.c_int, _f32p, C.c_int, C.c_int]
        L.or_set_threads.argtypes = [C.c_int]
        L.or_get_threads.restype = C.c_int
        L.p32_pass.argtypes = [C.c_void_p, _i32p, C.c_int, C.c_int, _f32p]
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def set_threads(n: int) -> None:
    lib().or_set_threads(n)


def get_threads() -> int:
    return lib().or_get_threads()


def h2f(h: int) -> float:
    return lib().or_h2f(h)


def f2h(f: float) -> int:
    return lib().or_f2h(f)


def dequant(fmt: int, codes: np.ndarray, sb: np.ndarray, rows: int, K: int) -> np.ndarray:
    out = np.empty((rows, K), dtype=np.float32)
    sb = np.ascontiguousarray(sb, dtype=np.uint8)
    lib().or_dequant(fmt, np.ascontiguousarray(codes, dtype=np.uint8), _ptr(sb), rows, K, out)
    return out


def gemv(fmt: int, codes: np.ndarray, sb: np.ndarray, N: int, K: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    n = x.shape[0]
    y = np.empty((n, N), dtype=np.float32)
    sb = np.ascontiguousarray(sb, dtype=np.uint8)
    lib().or_gemv(fmt, np.ascontiguousarray(codes, dtype=np.uint8), _ptr(sb), N, K, x, n, y)
    return y


def quant_q8(m: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """quantizeQ8 (Convert.swift:215-241): int8 codes [rows][cols], fp16 bits [rows][cols/32]."""
    m = np.ascontiguousarray(m, dtype=np.float32)
    rows, cols = m.shape
    codes = np.empty((rows, cols), dtype=np.int8)
    scales = np.empty((rows, cols // 32), dtype=np.uint16)
    lib().or_quant_q8(m, rows, cols, _ptr(codes), scales)
    return codes, scales


def quant_q4(m: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """quantizeQ4Raw (Convert.swift:243-320): packed codes [rows][cols/2], (scale, bias) fp16
    bits [rows][cols/64][2]."""
    m = np.ascontiguousarray(m, dtype=np.float32)
    rows, cols = m.shape
    packed = np.empty((rows, cols // 2), dtype=np.uint8)
    sb = np.empty((rows, cols // 64, 2), dtype=np.uint16)
    lib().or_quant_q4(m, rows, cols, packed, sb)
    return packed, sb


def mrope_table(maxctx: int, vis_offset: int, llm_h: int, llm_w: int) -> np.ndarray:
    out = np.empty((maxctx, 64, 2), dtype=np.float32)
    lib().or_mrope_table(maxctx, vis_offset, llm_h, llm_w, out)
    return out


class OracleModel:
    """The whole-decoder oracle over an in-memory ``.icua`` image."""

    def __init__(self, image: np.ndarray, maxctx: int):
        self.image = np.ascontiguousarray(image, dtype=np.uint8)
        self.maxctx = maxctx
        h = lib().or_model_new(_ptr(self.image), self.image.nbytes, maxctx)
        if not h:
            raise RuntimeError("oracle: " + lib().or_last_error().decode())
        self.h = h
        self.layers = lib().or_model_layers(h)
        self.fmt = lib().or_model_format(h)

    def close(self):
        if self.h:
            lib().or_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def prepare_mrope(self, vis_offset: int, llm_h: int, llm_w: int) -> None:
        lib().or_prepare_mrope(self.h, vis_offset, llm_h, llm_w)

    def kv(self, layer: int, kind: int) -> np.ndarray:
        """Writable view of the fp16 cache of one layer: [NKV][maxctx][HD] (kind 0 K, 1 V)."""
        p = lib().or_kv(self.h, layer, kind)
        arr = np.ctypeslib.as_array(p, shape=(NKV * self.maxctx * HD,))
        return arr.view(np.float16).reshape(NKV, self.maxctx, HD)

    def layer(self, l: int, x: np.ndarray, pos: int) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, H).copy()
        lib().or_layer(self.h, l, x, x.shape[0], pos)
        return x

    def layer_taps(self, l: int, x: np.ndarray, pos: int):
        """or_layer with the intermediate taps: (x_out, qkv_raw, attn_out, act)."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, H).copy()
        n = x.shape[0]
        qkv = np.empty((n, QKV), np.float32)
        att = np.empty((n, H), np.float32)
        act = np.empty((n, FF), np.float32)
        lib().or_debug_taps(qkv.ctypes.data, att.ctypes.data, act.ctypes.data)
        try:
            lib().or_layer(self.h, l, x, n, pos)
        finally:
            lib().or_debug_taps(None, None, None)
        return x, qkv, att, act

    def embed(self, tok: int) -> np.ndarray:
        x = np.empty(H, dtype=np.float32)
        lib().or_embed(self.h, tok, x)
        return x

    def lm_head(self, x: np.ndarray) -> np.ndarray:
        out = np.empty(VOCAB, dtype=np.float32)
        lib().or_lm_head(self.h, np.ascontiguousarray(x, dtype=np.float32), out)
        return out

    def port32_pass(self, toks, pos: int) -> np.ndarray:
        """The fp32 CPU port (port32.c, the benchmark's CPU baseline, not the checker): a pass of
        text tokens at slots pos.., writing their K/V into this model's cache; the last row's
        logits."""
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        out = np.empty(VOCAB, dtype=np.float32)
        if lib().p32_pass(self.h, toks, toks.size, pos, out) != 0:
            raise RuntimeError("port32 pass exceeds the context")
        return out

    @staticmethod
    def _visual(pooler, deepstack):
        pool = None if pooler is None else np.ascontiguousarray(pooler, dtype=np.float32)
        ds_keep = None
        ds_ptr = None
        if deepstack is not None:
            ds_keep = [np.ascontiguousarray(d, dtype=np.float32) for d in deepstack]
            arr = (C.c_void_p * 3)(*[d.ctypes.data for d in ds_keep])
            ds_ptr = C.cast(arr, C.c_void_p)
            ds_keep.append(arr)
        return pool, ds_keep, ds_ptr

    def run_pass(self, toks, pos: int, pooler=None, vis_offset: int = -1, deepstack=None,
                 logits_rows: int = 1) -> np.ndarray:
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        n = toks.size
        pool, keep, ds_ptr = self._visual(pooler, deepstack)
        n_vis = 0 if pool is None else pool.shape[0]
        out = np.empty((max(logits_rows, 1), VOCAB), dtype=np.float32)
        rc = lib().or_pass(self.h, toks, n, pos, _ptr(pool), vis_offset, n_vis, ds_ptr, logits_rows,
                           _ptr(out) if logits_rows else None)
        if rc:
            raise RuntimeError("oracle: " + lib().or_last_error().decode())
        return out[:logits_rows]

    def generate_commit(self, toks, max_steps: int, eos=(-1, -1), grammar: bool = False, pooler=None,
                        vis_offset: int = -1, deepstack=None) -> np.ndarray:
        """The reference's token loop with its commit rules (or_generate_commit)."""
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        pool, keep, ds_ptr = self._visual(pooler, deepstack)
        n_vis = 0 if pool is None else pool.shape[0]
        out = np.zeros(max_steps, dtype=np.int32)
        n = lib().or_generate_commit(self.h, toks, toks.size, _ptr(pool), vis_offset, n_vis, ds_ptr, max_steps,
                                     int(eos[0]), int(eos[1]), int(grammar), out)
        if n < 0:
            raise RuntimeError("oracle: " + lib().or_last_error().decode())
        return out[:n]

    def generate(self, toks, steps: int, pooler=None, vis_offset: int = -1, deepstack=None, with_top1=False):
        """Greedy tokens, top-2 margins and first logits (prefill at slot 0, no EOS stop); with
        `with_top1`, also each step's top-1 logit."""
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        pool, keep, ds_ptr = self._visual(pooler, deepstack)
        n_vis = 0 if pool is None else pool.shape[0]
        out = np.empty(steps, dtype=np.int32)
        margins = np.empty(steps, dtype=np.float32)
        top1 = np.empty(steps, dtype=np.float32)
        first = np.empty(VOCAB, dtype=np.float32)
        rc = lib().or_generate(self.h, toks, toks.size, _ptr(pool), vis_offset, n_vis, ds_ptr, steps, out,
                               _ptr(margins), _ptr(top1), _ptr(first))
        if rc:
            raise RuntimeError("oracle: " + lib().or_last_error().decode())
        return (out, margins, first, top1) if with_top1 else (out, margins, first)


# ---------------------------------------------------------------------------------------------
# Vision encoder (oracle/vision.c).  fp16 arrays travel as uint16 bit patterns.

VH, VPATCH, VNH, VHD = 1024, 768, 16, 64


def _u16(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint16) if a.dtype == np.float16 else np.ascontiguousarray(a, dtype=np.uint16)


def vit_patchify(rgb: np.ndarray) -> np.ndarray:
    """RGB8 [16 gh][16 gw][3] -> fp16 patches [gh * gw][768] in 2 x 2 merge-block order."""
    rgb = np.ascontiguousarray(rgb, dtype=np.uint8)
    gh, gw = rgb.shape[0] // 16, rgb.shape[1] // 16
    out = np.empty((gh * gw, VPATCH), dtype=np.uint16)
    lib().or_vit_patchify(rgb.reshape(-1), gh, gw, out)
    return out.view(np.float16)


def vit_pos_interp(table: np.ndarray, gh: int, gw: int) -> np.ndarray:
    out = np.empty((gh * gw, VH), dtype=np.float32)
    lib().or_vit_pos_interp(np.ascontiguousarray(table, dtype=np.float32), gh, gw, out)
    return out


def vit_rope_table(gh: int, gw: int) -> np.ndarray:
    out = np.empty((gh * gw, 32, 2), dtype=np.float32)
    lib().or_vit_rope_table(gh, gw, out)
    return out


def layernorm_f16(x: np.ndarray, w: np.ndarray, b: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, n = x.shape
    out = np.empty((rows, n), dtype=np.uint16)
    lib().or_layernorm_f16(x, np.ascontiguousarray(w, dtype=np.float32), np.ascontiguousarray(b, dtype=np.float32),
                           rows, n, out)
    return out.view(np.float16)


def linear_f16(x: np.ndarray, w: np.ndarray, bias: np.ndarray) -> np.ndarray:
    x, w = _u16(x), _u16(w)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), dtype=np.float32)
    lib().or_linear_f16(x, w, np.ascontiguousarray(bias, dtype=np.float32), M, N, K, y)
    return y


def gelu_tanh(x: float) -> float:
    return lib().or_gelu_tanh(x)


def gelu_erf(x: float) -> float:
    return lib().or_gelu_erf(x)


def vit_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
    """q, k, v fp16 [16][np][64] -> fp16 [np][1024]."""
    np_ = q.shape[1]
    out = np.empty((np_, VH), dtype=np.uint16)
    lib().or_vit_attention(_u16(q).reshape(-1), _u16(k).reshape(-1), _u16(v).reshape(-1), np_, out)
    return out.view(np.float16)


def vision(image: np.ndarray, rgb: np.ndarray):
    """The encoder over an .icua image's vision tensors: (pooler, [deepstack x 3]) float32
    [np / 4][2048] each."""
    rgb = np.ascontiguousarray(rgb, dtype=np.uint8)
    gh, gw = rgb.shape[0] // 16, rgb.shape[1] // 16
    nvis = gh * gw // 4
    pooler = np.empty((nvis, H), dtype=np.float32)
    ds = [np.empty((nvis, H), dtype=np.float32) for _ in range(3)]
    arr = (C.c_void_p * 3)(*[d.ctypes.data for d in ds])
    img = np.ascontiguousarray(image, dtype=np.uint8)
    if lib().or_vision(img.ctypes.data_as(C.c_void_p), img.size, rgb.reshape(-1), gh, gw, pooler, arr) != 0:
        raise RuntimeError(lib().or_vision_error().decode())
    return pooler, ds


def vit_block(image: np.ndarray, l: int, x: np.ndarray, gh: int, gw: int) -> np.ndarray:
    """Block l of the tower on residual rows x [gh * gw][1024] (returns the updated rows)."""
    out = np.array(x, dtype=np.float32, order="C")
    img = np.ascontiguousarray(image, dtype=np.uint8)
    if lib().or_vit_block(img.ctypes.data_as(C.c_void_p), img.size, l, out, gh, gw) != 0:
        raise RuntimeError(lib().or_vision_error().decode())
    return out
