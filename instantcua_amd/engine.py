"""Python mirror of instantcua's ``Engine`` over the C ABI of ``include/icua.h``.

The method names and argument meanings follow the Swift class
(Sources/Engine/Engine.swift:5-827): ``prepare_mrope`` = ``prepareMRoPE`` (254-298),
``prefill`` = ``encodePrefill`` run to completion (658-673), ``decode_steps`` = k x
``encodeDecodeStep`` (675-681), ``generate`` = ``generateVision`` minus the vision encoder
(696-827), ``last_timing`` = ``lastTiming`` (44-52), ``layer_step`` = ``encodeLLMLayer``
(476-629).  Errors raise ``EngineError`` (ModelFile.swift:158-161).

There is no CPU fallback: the HIP library must be built (``instantcua_amd.build``) and a GPU
must be present, otherwise construction fails.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libicua.so")

H, FF, NH, NKV, HD, VOCAB = 2048, 6144, 16, 8, 128, 151936
MAXM = 8

FLAG_GRAMMAR_PAIRS = 1
FLAG_PREFIX_CACHE = 2
FLAG_GRAPH_DECODE = 4
FLAG_PASS_PREFILL = 8
FLAG_VISION_DELTA_CACHE = 16
FLAG_FIRST_LOGITS = 32
FLAG_PREFILL_FP16 = 64

EXPORTS = [
    "icua_last_error", "icua_engine_create", "icua_engine_create_from_memory", "icua_engine_destroy",
    "icua_engine_info", "icua_set_eos", "icua_set_flags", "icua_prepare_mrope", "icua_set_visual",
    "icua_prefill", "icua_decode_steps", "icua_generate", "icua_verify", "icua_set_position",
    "icua_read_state", "icua_read_tokens", "icua_logits", "icua_timing", "icua_layer_step",
    "icua_read_kv", "icua_write_kv", "icua_read_buffer", "icua_dev_alloc", "icua_dev_free", "icua_memcpy_h2d",
    "icua_memcpy_d2h", "icua_device_sync", "icua_repack", "icua_gemv", "icua_gemv_bench", "icua_dequant",
    "icua_quantize", "icua_quantize_noalloc", "icua_quantize_bench", "icua_vision", "icua_generate_vision",
    # include/icua_tok.h
    "icua_tok_last_error", "icua_tok_open", "icua_tok_close", "icua_tok_vocab_size", "icua_tok_special_id",
    "icua_tok_encode", "icua_tok_encode_chat", "icua_tok_encode_vision_chat", "icua_tok_token_bytes",
    "icua_tok_decode", "icua_tok_stream_new", "icua_tok_stream_free", "icua_tok_stream_push",
]


class EngineError(RuntimeError):
    pass


class _State(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "pos", "n", "step", "done", "maxctx", "maxsteps", "eos0", "eos1", "vis_offset", "n_vis",
        "rope_delta", "npatches", "flags", "logits_rows")]


class _Timing(C.Structure):
    _fields_ = [("vision_ms", C.c_double), ("prefill_ms", C.c_double), ("decode_ms", C.c_double),
                ("total_ms", C.c_double), ("prefill_tokens", C.c_int64), ("generated_tokens", C.c_int64)]


class _Info(C.Structure):
    _fields_ = [("format", C.c_int32), ("layers", C.c_int32), ("max_context", C.c_int32),
                ("max_pass", C.c_int32), ("max_steps", C.c_int32), ("weight_bytes", C.c_int64),
                ("kv_bytes", C.c_int64), ("persistent_decode", C.c_int32), ("vision", C.c_int32),
                ("last_decode_persistent", C.c_int32), ("visual_rows", C.c_int32), ("pair_passes", C.c_int32)]


_lib = None


def lib() -> C.CDLL:
    """Load libicua.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise EngineError(f"{LIB_PATH} is missing: run `python -m instantcua_amd.build` first")
        L = C.CDLL(LIB_PATH)
        vp, i32, sz = C.c_void_p, C.c_int, C.c_size_t
        L.icua_last_error.restype = C.c_char_p
        L.icua_engine_create.argtypes = [C.c_char_p, i32, i32, i32, C.c_uint32, C.POINTER(vp)]
        L.icua_engine_create_from_memory.argtypes = [vp, sz, i32, i32, i32, C.c_uint32, C.POINTER(vp)]
        L.icua_engine_destroy.argtypes = [vp]
        L.icua_engine_destroy.restype = None
        L.icua_engine_info.argtypes = [vp, C.POINTER(_Info)]
        L.icua_set_eos.argtypes = [vp, C.c_int32, C.c_int32]
        L.icua_set_flags.argtypes = [vp, C.c_uint32]
        L.icua_prepare_mrope.argtypes = [vp, i32, i32, i32]
        L.icua_set_visual.argtypes = [vp, vp, vp, i32]
        L.icua_prefill.argtypes = [vp, vp, i32, i32, i32, i32, i32]
        L.icua_decode_steps.argtypes = [vp, i32]
        L.icua_generate.argtypes = [vp, vp, i32, i32, i32, vp, C.POINTER(C.c_int)]
        L.icua_verify.argtypes = [vp, vp, i32, vp, vp]
        L.icua_vision.argtypes = [vp, vp, i32, i32]
        L.icua_generate_vision.argtypes = [vp, vp, i32, i32, vp, i32, i32, vp, C.POINTER(C.c_int)]
        L.icua_set_position.argtypes = [vp, i32, C.c_int32, i32, i32]
        L.icua_read_state.argtypes = [vp, C.POINTER(_State)]
        L.icua_read_tokens.argtypes = [vp, vp, i32]
        L.icua_logits.argtypes = [vp, vp, i32]
        L.icua_timing.argtypes = [vp, C.POINTER(_Timing)]
        L.icua_layer_step.argtypes = [vp, i32, vp, i32, i32, vp]
        L.icua_read_kv.argtypes = [vp, i32, i32, i32, i32, vp]
        L.icua_write_kv.argtypes = [vp, i32, i32, i32, i32, vp]
        L.icua_read_buffer.argtypes = [vp, i32, vp, sz]
        L.icua_dev_alloc.argtypes = [sz, C.POINTER(vp)]
        L.icua_dev_free.argtypes = [vp]
        L.icua_memcpy_h2d.argtypes = [vp, vp, sz]
        L.icua_memcpy_d2h.argtypes = [vp, vp, sz]
        L.icua_gemv.argtypes = [i32, vp, vp, i32, i32, vp, i32, vp]
        L.icua_gemv_bench.argtypes = [i32, vp, vp, i32, i32, i32, vp, vp, i32, C.POINTER(C.c_double)]
        L.icua_dequant.argtypes = [i32, vp, vp, i32, i32, i32, vp, i32]
        L.icua_repack.argtypes = [i32, vp, vp, i32, i32, vp, vp]
        L.icua_quantize.argtypes = [i32, vp, i32, i32, vp, vp]
        L.icua_quantize_noalloc.argtypes = [i32, vp, i32, i32, vp, vp]
        L.icua_quantize_bench.argtypes = [i32, vp, i32, i32, vp, vp, i32, C.POINTER(C.c_double)]
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        raise EngineError(lib().icua_last_error().decode())


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------------------------------------
# Device buffers for the standalone kernels

class DeviceBuffer:
    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        ptr = C.c_void_p()
        _check(lib().icua_dev_alloc(max(self.nbytes, 16), C.byref(ptr)))
        self.ptr = ptr.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            _check(lib().icua_memcpy_h2d(b.ptr, _p(a), a.nbytes))
        return b

    def to_array(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        _check(lib().icua_memcpy_d2h(_p(out), self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            _check(lib().icua_dev_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def gemv(fmt: int, codes: DeviceBuffer, sb: DeviceBuffer, N: int, K: int, x: DeviceBuffer, m: int,
         y: DeviceBuffer) -> None:
    _check(lib().icua_gemv(fmt, codes.ptr, sb.ptr, N, K, x.ptr, m, y.ptr))


def gemv_bench(fmt: int, codes: Sequence[DeviceBuffer], sbs: Sequence[DeviceBuffer], N: int, K: int,
               x: DeviceBuffer, y: DeviceBuffer, iters: int) -> float:
    n = len(codes)
    carr = (C.c_void_p * n)(*[c.ptr for c in codes])
    sarr = (C.c_void_p * n)(*[s.ptr for s in sbs])
    us = C.c_double()
    _check(lib().icua_gemv_bench(fmt, C.cast(carr, C.c_void_p), C.cast(sarr, C.c_void_p), n, N, K, x.ptr, y.ptr,
                                 iters, C.byref(us)))
    return us.value


def dequant(fmt: int, codes: DeviceBuffer, sb: DeviceBuffer, K: int, row0: int, rows: int,
            out: DeviceBuffer, tiled: bool = False) -> None:
    _check(lib().icua_dequant(fmt, codes.ptr, sb.ptr, K, row0, rows, out.ptr, int(tiled)))


def repack(fmt: int, codes: DeviceBuffer, sb: DeviceBuffer, N: int, K: int):
    """Row-major .icua matrix -> (tiled codes, scales) device buffers of the GEMV layout."""
    tc = DeviceBuffer(codes.nbytes)
    ts = DeviceBuffer(sb.nbytes)
    _check(lib().icua_repack(fmt, codes.ptr, sb.ptr, N, K, tc.ptr, ts.ptr))
    return tc, ts


# ---------------------------------------------------------------------------------------------

class Engine:
    """Drop-in mirror of ``Engine`` (Sources/Engine/Engine.swift:5)."""

    def __init__(self, model_path: Optional[str] = None, image: Optional[np.ndarray] = None,
                 max_context: int = 2048, max_pass: int = 512, max_steps: int = 256,
                 flags: int = FLAG_GRAMMAR_PAIRS):
        h = C.c_void_p()
        if model_path is not None:
            _check(lib().icua_engine_create(model_path.encode(), max_context, max_pass, max_steps, flags,
                                            C.byref(h)))
        elif image is not None:
            img = np.ascontiguousarray(image, dtype=np.uint8)
            _check(lib().icua_engine_create_from_memory(_p(img), img.nbytes, max_context, max_pass, max_steps,
                                                        flags, C.byref(h)))
        else:
            raise EngineError("model_path or image is required")
        self._h = h.value
        self._flags = flags
        self._eos = (151645, 151643)
        info = _Info()
        _check(lib().icua_engine_info(self._h, C.byref(info)))
        self.format = info.format
        self.layers = info.layers
        self.max_context = info.max_context
        self.max_pass = info.max_pass
        self.max_steps = info.max_steps
        self.has_vision = bool(info.vision)
        self._vis_rows = 0
        self.weight_bytes = info.weight_bytes
        self.kv_bytes = info.kv_bytes
        self.persistent_decode = bool(info.persistent_decode)

    @property
    def pair_passes(self) -> int:
        """Forced grammar pairs that ran as one two-row launch of the persistent kernel."""
        info = _Info()
        _check(lib().icua_engine_info(self._h, C.byref(info)))
        return int(info.pair_passes)

    @property
    def last_decode_persistent(self) -> bool:
        """Whether the last decode_steps call ran as the persistent kernel."""
        info = _Info()
        _check(lib().icua_engine_info(self._h, C.byref(info)))
        return bool(info.last_decode_persistent)

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().icua_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- properties of the Swift class -------------------------------------------------------
    @property
    def eos(self):
        return self._eos

    @eos.setter
    def eos(self, pair):
        _check(lib().icua_set_eos(self._h, int(pair[0]), int(pair[1])))
        self._eos = (int(pair[0]), int(pair[1]))

    @property
    def use_prefix_cache(self) -> bool:
        return bool(self._flags & FLAG_PREFIX_CACHE)

    @use_prefix_cache.setter
    def use_prefix_cache(self, v: bool):
        self.set_flags((self._flags | FLAG_PREFIX_CACHE) if v else (self._flags & ~FLAG_PREFIX_CACHE))

    @property
    def grammar_pairs(self) -> bool:
        return bool(self._flags & FLAG_GRAMMAR_PAIRS)

    @grammar_pairs.setter
    def grammar_pairs(self, v: bool):
        self.set_flags((self._flags | FLAG_GRAMMAR_PAIRS) if v else (self._flags & ~FLAG_GRAMMAR_PAIRS))

    @property
    def graph_decode(self) -> bool:
        """Decode through the per-kernel HIP graph instead of the persistent kernel."""
        return bool(self._flags & FLAG_GRAPH_DECODE)

    @graph_decode.setter
    def graph_decode(self, v: bool):
        self.set_flags((self._flags | FLAG_GRAPH_DECODE) if v else (self._flags & ~FLAG_GRAPH_DECODE))

    @property
    def use_vision_delta_cache(self) -> bool:
        """generate_vision skips the encoder on an identical consecutive frame."""
        return bool(self._flags & FLAG_VISION_DELTA_CACHE)

    @use_vision_delta_cache.setter
    def use_vision_delta_cache(self, v: bool):
        self.set_flags((self._flags | FLAG_VISION_DELTA_CACHE) if v else (self._flags & ~FLAG_VISION_DELTA_CACHE))

    @property
    def pass_prefill(self) -> bool:
        """Prefill q4 prompts in passes of 8 rows instead of the matrix-core GEMMs."""
        return bool(self._flags & FLAG_PASS_PREFILL)

    @pass_prefill.setter
    def pass_prefill(self, v: bool):
        self.set_flags((self._flags | FLAG_PASS_PREFILL) if v else (self._flags & ~FLAG_PASS_PREFILL))

    @property
    def prefill_fp16(self) -> bool:
        """Matrix-core prefill on fp16 operands alone (the reference engine's precision) instead
        of fp16 hi + lo parts."""
        return bool(self._flags & FLAG_PREFILL_FP16)

    @prefill_fp16.setter
    def prefill_fp16(self, v: bool):
        self.set_flags((self._flags | FLAG_PREFILL_FP16) if v else (self._flags & ~FLAG_PREFILL_FP16))

    def set_flags(self, flags: int) -> None:
        _check(lib().icua_set_flags(self._h, flags))
        self._flags = flags

    # -- decoder ------------------------------------------------------------------------------
    def prepare_mrope(self, vis_offset: int, llm_h: int, llm_w: int) -> None:
        _check(lib().icua_prepare_mrope(self._h, vis_offset, llm_h, llm_w))

    def set_visual(self, pooler: np.ndarray, deepstack: Optional[Sequence[np.ndarray]] = None) -> None:
        pool = np.ascontiguousarray(pooler, dtype=np.float32).reshape(-1, H)
        keep = [pool]
        ds_ptr = None
        if deepstack is not None:
            ds = [np.ascontiguousarray(d, dtype=np.float32).reshape(-1, H) for d in deepstack]
            keep += ds
            arr = (C.c_void_p * 3)(*[d.ctypes.data for d in ds])
            keep.append(arr)
            ds_ptr = C.cast(arr, C.c_void_p)
        _check(lib().icua_set_visual(self._h, _p(pool), ds_ptr, pool.shape[0]))
        self._vis_rows = pool.shape[0]

    # -- vision tower ------------------------------------------------------------------------
    @staticmethod
    def _rgb(rgb: np.ndarray) -> np.ndarray:
        img = np.ascontiguousarray(rgb, dtype=np.uint8)
        if img.ndim != 3 or img.shape[2] != 3:
            raise EngineError("rgb must be uint8 [height][width][3]")
        return img

    def vision(self, rgb: np.ndarray) -> None:
        """encodeVision (Engine.swift:317-473): the frame's pooler and DeepStack rows become the
        visual rows of the next prefill."""
        img = self._rgb(rgb)
        _check(lib().icua_vision(self._h, _p(img), img.shape[1], img.shape[0]))
        self._vis_rows = (img.shape[0] // 32) * (img.shape[1] // 32)

    def visual_rows(self):
        """(pooler, [deepstack x 3]) float32 [n_vis][2048] currently held by the engine."""
        info = _Info()
        _check(lib().icua_engine_info(self._h, C.byref(info)))
        n = info.visual_rows
        pool = np.empty((n, H), dtype=np.float32)
        _check(lib().icua_read_buffer(self._h, 4, _p(pool), pool.nbytes))
        ds = []
        for i in range(3):
            d = np.empty((n, H), dtype=np.float32)
            _check(lib().icua_read_buffer(self._h, 5 + i, _p(d), d.nbytes))
            ds.append(d)
        return pool, ds

    def _with_first_logits(self, on: bool, fn):
        """Runs fn with FLAG_FIRST_LOGITS set as `on` (writeFirstLogits), restoring the flags."""
        saved = self._flags
        self.set_flags((saved | FLAG_FIRST_LOGITS) if on else (saved & ~FLAG_FIRST_LOGITS))
        try:
            return fn()
        finally:
            self.set_flags(saved)

    def generate_vision(self, rgb: np.ndarray, tokens, max_new_tokens: int = 64,
                        write_first_logits: bool = False) -> list:
        """generateVision (Engine.swift:696-827) on an RGB8 frame [height][width][3];
        write_first_logits keeps the first token's logits for logits()."""
        img = self._rgb(rgb)
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(max(1, min(max_new_tokens, self.max_steps) + 1), dtype=np.int32)
        n = C.c_int(0)
        self._with_first_logits(write_first_logits, lambda: _check(lib().icua_generate_vision(
            self._h, _p(img), img.shape[1], img.shape[0], _p(toks), toks.size, max_new_tokens, _p(out), C.byref(n))))
        self._vis_rows = (img.shape[0] // 32) * (img.shape[1] // 32)
        return [int(t) for t in out[:n.value]]

    def prefill(self, tokens, start_pos: int = 0, vis_offset: int = -1, max_new: int = 1,
                write_logits: bool = False) -> int:
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        _check(lib().icua_prefill(self._h, _p(toks), toks.size, start_pos, vis_offset, max_new, int(write_logits)))
        return int(self.tokens(1)[0])

    def decode_steps(self, k: int) -> None:
        _check(lib().icua_decode_steps(self._h, k))

    def generate(self, tokens, vis_offset: int = -1, max_new_tokens: int = 64,
                 write_first_logits: bool = False) -> list:
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(max(max_new_tokens, 1) + 4, dtype=np.int32)
        n_out = C.c_int()
        self._with_first_logits(write_first_logits, lambda: _check(lib().icua_generate(
            self._h, _p(toks), toks.size, vis_offset, max_new_tokens, _p(out), C.byref(n_out))))
        return [int(t) for t in out[:n_out.value]]

    def verify(self, draft, want_logits: bool = False):
        d = np.ascontiguousarray(draft, dtype=np.int32)
        am = np.empty(d.size, dtype=np.int32)
        lg = np.empty((d.size, VOCAB), dtype=np.float32) if want_logits else None
        _check(lib().icua_verify(self._h, _p(d), d.size, _p(am), _p(lg) if lg is not None else None))
        return am, lg

    def set_position(self, pos: int, next_token: int, step: int = 0, max_steps: Optional[int] = None) -> None:
        _check(lib().icua_set_position(self._h, pos, next_token, step,
                                       self.max_steps if max_steps is None else max_steps))

    def state(self) -> dict:
        s = _State()
        _check(lib().icua_read_state(self._h, C.byref(s)))
        return {name: getattr(s, name) for name, _ in _State._fields_}

    def tokens(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.int32)
        _check(lib().icua_read_tokens(self._h, _p(out), n))
        return out

    def logits(self, rows: int = 1) -> np.ndarray:
        out = np.empty((rows, VOCAB), dtype=np.float32)
        _check(lib().icua_logits(self._h, _p(out), rows))
        return out

    @property
    def last_timing(self) -> dict:
        t = _Timing()
        _check(lib().icua_timing(self._h, C.byref(t)))
        return {name: getattr(t, name) for name, _ in _Timing._fields_}

    def layer_step(self, layer: int, x: np.ndarray, pos: int) -> np.ndarray:
        xi = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, H)
        xo = np.empty_like(xi)
        _check(lib().icua_layer_step(self._h, layer, _p(xi), xi.shape[0], pos, _p(xo)))
        return xo

    def read_buffer(self, which: str, rows: int = MAXM) -> np.ndarray:
        """Pass activations of the last layer run: 'x', 'qkv', 'attn' or 'mlp'."""
        spec = {"x": (0, np.float32, H), "qkv": (1, np.float32, 4096), "attn": (2, np.float32, H),
                "mlp": (3, np.float32, FF)}[which]
        out = np.empty((rows, spec[2]), dtype=spec[1])
        _check(lib().icua_read_buffer(self._h, spec[0], _p(out), out.nbytes))
        return out

    def read_kv(self, layer: int, kind: int, slot0: int, nslots: int) -> np.ndarray:
        out = np.empty((NKV, nslots, HD), dtype=np.float16)
        _check(lib().icua_read_kv(self._h, layer, kind, slot0, nslots, _p(out)))
        return out

    def write_kv(self, layer: int, kind: int, slot0: int, data: np.ndarray) -> None:
        d = np.ascontiguousarray(data, dtype=np.float16)
        assert d.ndim == 3 and d.shape[0] == NKV and d.shape[2] == HD
        _check(lib().icua_write_kv(self._h, layer, kind, slot0, d.shape[1], _p(d)))
