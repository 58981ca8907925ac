"""Qwen2 tokenizer: compile step (Python) and the native tokenizer of ``libicua.so`` (ctypes).

``compile`` mirrors ``Tokenizer.compile(tokenizerJSON:output:)`` (Sources/Tokenizer/
Compile.swift:20-258): it checks that a Hugging Face ``tokenizer.json`` is the Qwen2 pipeline
(Compile.swift:260-291), decodes the byte-level alphabet back to raw bytes, and writes one
binary file (layout below) that the native tokenizer reads:

* the vocabulary and added tokens as raw bytes, the token id of every single byte;
* every merge as (left id, right id, result id) in rank order;
* the added tokens (id, content), matched leftmost-longest on the raw text;
* the Unicode tables: a two-stage property table (split-pattern class, contraction letters,
  canonical combining class), full canonical decompositions and primary compositions, from
  Python's ``unicodedata``.

``Tokenizer`` and ``TextStream`` mirror the reference's ``Tokenizer`` and ``TextStream``
(Tokenizer.swift:36-462) over ``include/icua_tok.h``.
"""
from __future__ import annotations

import ctypes as C
import json
import struct
import unicodedata
from typing import List, Tuple

import numpy as np

from . import engine as eng

QWEN2_SPLIT = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|"
               r"\s*[\r\n]+|\s+(?!\S)|\s+")
MAGIC, VERSION = 0x31544349, 1
VISION_START, VISION_END, IMAGE_PAD = 151652, 151653, 151655

# Unicode White_Space (PropList.txt): the characters \s matches.
WHITE_SPACE = set(range(0x09, 0x0E)) | {0x20, 0x85, 0xA0, 0x1680, 0x2028, 0x2029, 0x202F, 0x205F, 0x3000} \
    | set(range(0x2000, 0x200B))
C_L, C_N, C_O, C_WS, C_SP, C_NL = 0, 1, 2, 3, 4, 5
F_C1, F_RV, F_E, F_LL = 1 << 4, 1 << 5, 1 << 6, 1 << 7


class TokenizerError(RuntimeError):
    pass


def bytes_to_unicode() -> dict:
    """GPT-2's byte-level alphabet: byte -> character (printable bytes map to themselves)."""
    bs = list(range(0x21, 0x7F)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    cs = list(bs)
    n = 0
    for b in range(256):
        if b not in bs:
            bs.append(b)
            cs.append(256 + n)
            n += 1
    return {b: chr(c) for b, c in zip(bs, cs)}


def check_pipeline(root: dict) -> None:
    """The Qwen2 pipeline, the only one the tokenizer implements (Compile.swift:260-291)."""
    def no(what):
        raise TokenizerError(f"unsupported tokenizer.json: {what}")
    norm = root.get("normalizer") or {}
    if norm.get("type") != "NFC":
        no("normalizer must be NFC")
    pre = root.get("pre_tokenizer") or {}
    lst = pre.get("pretokenizers") or []
    if pre.get("type") != "Sequence" or len(lst) != 2:
        no("pre_tokenizer must be Sequence[Split, ByteLevel]")
    sp, bl = lst
    if sp.get("type") != "Split" or (sp.get("pattern") or {}).get("Regex") != QWEN2_SPLIT \
            or sp.get("behavior") != "Isolated" or sp.get("invert", False):
        no("Split must be the Qwen2 pattern with behavior Isolated")
    if bl.get("type") != "ByteLevel" or bl.get("add_prefix_space", False) or bl.get("use_regex", True):
        no("ByteLevel pre-tokenizer must have add_prefix_space=false, use_regex=false")
    model = root.get("model") or {}
    if model.get("type") != "BPE":
        no("model must be BPE")
    if model.get("dropout") is not None:
        no("BPE dropout")
    if model.get("byte_fallback"):
        no("byte_fallback")
    if model.get("continuing_subword_prefix") or model.get("end_of_word_suffix"):
        no("subword prefix / suffix")
    if model.get("ignore_merges"):
        no("ignore_merges")
    dec = root.get("decoder")
    if dec is not None and dec.get("type") != "ByteLevel":
        no("decoder must be ByteLevel")


_UNICODE = None


def unicode_tables():
    """(uni1 u16[4352], uni2 u16[blocks * 256], decomposition keys / values / data, composition
    keys / values) from the interpreter's unicodedata."""
    global _UNICODE
    if _UNICODE is not None:
        return _UNICODE
    fold = {"s": F_C1, "t": F_C1, "m": F_C1, "d": F_C1, "r": F_RV, "v": F_RV, "e": F_E, "l": F_LL}
    prop = np.zeros(0x110000, dtype=np.uint16)
    dkeys, dvals, ddata, comp = [], [], [], {}
    for cp in range(0x110000):
        ch = chr(cp)
        cat = unicodedata.category(ch)
        if cp in (0x0A, 0x0D):
            c = C_NL
        elif cp == 0x20:
            c = C_SP
        elif cp in WHITE_SPACE:
            c = C_WS
        elif cat[0] == "L":
            c = C_L
        elif cat[0] == "N":
            c = C_N
        else:
            c = C_O
        f = fold.get(ch.casefold(), 0) if cat[0] == "L" else 0
        prop[cp] = c | f | (unicodedata.combining(ch) << 8)
        if 0xD800 <= cp <= 0xDFFF:
            continue
        nfd = unicodedata.normalize("NFD", ch)
        if nfd != ch:
            dkeys.append(cp)
            dvals.append(len(ddata) << 5 | len(nfd))
            ddata.extend(ord(x) for x in nfd)
        d = unicodedata.decomposition(ch)
        if d and not d.startswith("<"):
            parts = [int(x, 16) for x in d.split()]
            if len(parts) == 2 and unicodedata.normalize("NFC", ch) == ch:
                comp[parts[0] << 21 | parts[1]] = cp
    # Hangul syllables compose algorithmically (L V -> LV, LV T -> LVT).
    for l in range(19):
        for v in range(21):
            lv = 0xAC00 + (l * 21 + v) * 28
            comp[(0x1100 + l) << 21 | (0x1161 + v)] = lv
            for t in range(1, 28):
                comp[lv << 21 | (0x11A7 + t)] = lv + t
    blocks, uni1 = {}, np.zeros(4352, dtype=np.uint16)
    for b in range(4352):
        key = prop[b * 256:(b + 1) * 256].tobytes()
        uni1[b] = blocks.setdefault(key, len(blocks))
    uni2 = np.frombuffer(b"".join(sorted(blocks, key=blocks.get)), dtype=np.uint16)
    ck = np.array(sorted(comp), dtype=np.uint64)
    _UNICODE = (uni1, uni2, np.array(dkeys, np.uint32), np.array(dvals, np.uint32), np.array(ddata, np.uint32),
                ck, np.array([comp[int(k)] for k in ck], np.uint32))
    return _UNICODE


def compile(tokenizer_json: str, output: str) -> int:  # noqa: A001  (mirrors Tokenizer.compile)
    """tokenizer.json -> compiled file; returns its size."""
    with open(tokenizer_json, encoding="utf-8") as f:
        root = json.load(f)
    check_pipeline(root)
    model = root["model"]
    vocab, merges = model.get("vocab"), model.get("merges")
    if not isinstance(vocab, dict) or merges is None:
        raise TokenizerError("model.vocab / model.merges missing")
    b2u = bytes_to_unicode()
    u2b = {c: b for b, c in b2u.items()}
    added = [(int(a["id"]), a["content"].encode("utf-8")) for a in root.get("added_tokens") or []]
    n_total = max([int(i) for i in vocab.values()] + [i for i, _ in added]) + 1
    tok = [b""] * n_total
    for s, i in vocab.items():
        try:
            tok[int(i)] = bytes(u2b[ch] for ch in s)
        except KeyError as e:
            raise TokenizerError(f"vocab entry {s!r} is not in the byte-level alphabet") from e
    for i, content in added:
        tok[i] = content
    byte_tok = np.array([vocab[b2u[b]] for b in range(256)], dtype=np.int32)
    mtab = np.zeros((len(merges), 3), dtype=np.uint32)
    for r, m in enumerate(merges):
        a, b = m.split(" ", 1) if isinstance(m, str) else m
        if a not in vocab or b not in vocab or a + b not in vocab:
            raise TokenizerError(f"merge {r} ({a!r}, {b!r}) names a token outside the vocabulary")
        mtab[r] = (vocab[a], vocab[b], vocab[a + b])
    tok_off = np.zeros(n_total + 1, dtype=np.uint32)
    tok_off[1:] = np.cumsum([len(t) for t in tok])
    tok_bytes = b"".join(tok)
    spec_tab = np.zeros((len(added), 3), dtype=np.uint32)
    spec_bytes = b""
    for k, (i, content) in enumerate(added):
        spec_tab[k] = (i, len(spec_bytes), len(content))
        spec_bytes += content
    uni1, uni2, dk, dv, dd, ck, cv = unicode_tables()

    sections = [tok_off.tobytes(), tok_bytes, byte_tok.tobytes(), mtab.tobytes(), spec_tab.tobytes(), spec_bytes,
                uni1.tobytes(), uni2.tobytes(), dk.tobytes(), dv.tobytes(), dd.tobytes(), ck.tobytes(), cv.tobytes()]
    hdr_fmt = "<8I14Q"
    offs, cur = [], (struct.calcsize(hdr_fmt) + 63) // 64 * 64
    for sec in sections:
        offs.append(cur)
        cur = (cur + len(sec) + 63) // 64 * 64
    header = struct.pack(hdr_fmt, MAGIC, VERSION, n_total, len(merges), len(added), uni2.size // 256, dk.size, ck.size,
                         *offs, cur)
    buf = bytearray(cur)
    buf[:len(header)] = header
    for o, sec in zip(offs, sections):
        buf[o:o + len(sec)] = sec
    with open(output, "wb") as f:
        f.write(buf)
    return cur


_bound = False


def _lib():
    global _bound
    L = eng.lib()
    if not _bound:
        vp, sz, i32 = C.c_void_p, C.c_size_t, C.c_int
        L.icua_tok_last_error.restype = C.c_char_p
        L.icua_tok_open.argtypes = [C.c_char_p, C.POINTER(vp)]
        L.icua_tok_close.argtypes = [vp]
        L.icua_tok_vocab_size.argtypes = [vp]
        L.icua_tok_special_id.argtypes = [vp, C.c_char_p]
        L.icua_tok_special_id.restype = C.c_int32
        L.icua_tok_encode.argtypes = [vp, C.c_char_p, sz, i32, vp, sz, C.POINTER(sz)]
        L.icua_tok_encode_chat.argtypes = [vp, C.c_char_p, sz, C.c_char_p, sz, vp, sz, C.POINTER(sz)]
        L.icua_tok_encode_vision_chat.argtypes = [vp, C.c_char_p, sz, C.c_char_p, sz, i32, vp, sz, C.POINTER(sz),
                                                  C.POINTER(C.c_int)]
        L.icua_tok_token_bytes.argtypes = [vp, C.c_int32, C.POINTER(C.POINTER(C.c_uint8)), C.POINTER(sz)]
        L.icua_tok_decode.argtypes = [vp, vp, sz, C.c_char_p, sz, C.POINTER(sz)]
        L.icua_tok_stream_new.restype = vp
        L.icua_tok_stream_free.argtypes = [vp]
        L.icua_tok_stream_push.argtypes = [vp, vp, C.c_int32, i32, C.c_char_p, sz, C.POINTER(sz)]
        _bound = True
    return L


def _check(rc: int) -> None:
    if rc != 0:
        raise TokenizerError(_lib().icua_tok_last_error().decode())


class Tokenizer:
    """Tokenizer(path:) over a compiled file (Tokenizer.swift:36-395)."""

    def __init__(self, path: str):
        h = C.c_void_p()
        _check(_lib().icua_tok_open(path.encode(), C.byref(h)))
        self._h = h.value
        self.vocab_size = _lib().icua_tok_vocab_size(self._h)
        sid = lambda s: int(_lib().icua_tok_special_id(self._h, s.encode()))  # noqa: E731
        self.im_start, self.im_end, self.end_of_text = sid("<|im_start|>"), sid("<|im_end|>"), sid("<|endoftext|>")
        self.vision_start, self.vision_end, self.image_pad = VISION_START, VISION_END, IMAGE_PAD

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib().icua_tok_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def _ids(self, fn, *args) -> List[int]:
        cap = 256
        while True:
            out = np.empty(cap, dtype=np.int32)
            n = C.c_size_t(0)
            rc = fn(self._h, *args, out.ctypes.data_as(C.c_void_p), cap, C.byref(n))
            if rc == 0:
                return out[:n.value].tolist()
            if n.value <= cap:
                _check(rc)
            cap = n.value

    def encode(self, text: str) -> List[int]:
        """Plain text: added tokens are not matched (Tokenizer.swift:153)."""
        b = text.encode("utf-8")
        return self._ids(_lib().icua_tok_encode, b, len(b), 0)

    def encode_with_specials(self, text: str) -> List[int]:
        """Added tokens matched leftmost-longest on the raw text, like HF encode (159)."""
        b = text.encode("utf-8")
        return self._ids(_lib().icua_tok_encode, b, len(b), 1)

    def encode_chat(self, system: str, user: str) -> List[int]:
        s, u = system.encode("utf-8"), user.encode("utf-8")
        return self._ids(_lib().icua_tok_encode_chat, s, len(s), u, len(u))

    def encode_vision_chat(self, system: str, user: str, num_image_tokens: int) -> Tuple[List[int], int]:
        """(tokens, index of the first image pad) (Tokenizer.swift:192-204)."""
        s, u = system.encode("utf-8"), user.encode("utf-8")
        off = C.c_int(0)
        cap = 256 + num_image_tokens
        while True:
            out = np.empty(cap, dtype=np.int32)
            n = C.c_size_t(0)
            rc = _lib().icua_tok_encode_vision_chat(self._h, s, len(s), u, len(u), num_image_tokens,
                                                    out.ctypes.data_as(C.c_void_p), cap, C.byref(n), C.byref(off))
            if rc == 0:
                return out[:n.value].tolist(), off.value
            if n.value <= cap:
                _check(rc)
            cap = n.value

    def token_bytes(self, tid: int) -> bytes:
        p = C.POINTER(C.c_uint8)()
        n = C.c_size_t(0)
        _check(_lib().icua_tok_token_bytes(self._h, tid, C.byref(p), C.byref(n)))
        return C.string_at(p, n.value) if n.value else b""

    def decode(self, ids) -> str:
        a = np.ascontiguousarray(ids, dtype=np.int32)
        cap = 16 + 3 * sum(len(self.token_bytes(int(i))) for i in a)
        out = C.create_string_buffer(cap)
        n = C.c_size_t(0)
        _check(_lib().icua_tok_decode(self._h, a.ctypes.data_as(C.c_void_p), a.size, out, cap, C.byref(n)))
        return out.raw[:n.value].decode("utf-8")


class TextStream:
    """Incremental detokenizer (Tokenizer.swift:400-462)."""

    def __init__(self, tok: Tokenizer):
        self._tok = tok
        self._s = _lib().icua_tok_stream_new()

    def _push(self, tid: int, final: int) -> str:
        cap = 64
        while True:
            out = C.create_string_buffer(cap)
            n = C.c_size_t(0)
            rc = _lib().icua_tok_stream_push(self._tok._h, self._s, tid, final, out, cap, C.byref(n))
            if rc == 0:
                return out.raw[:n.value].decode("utf-8")
            if n.value <= cap:
                _check(rc)
            cap = n.value

    def push(self, tid: int) -> str:
        return self._push(int(tid), 0)

    def finish(self) -> str:
        return self._push(-1, 1)

    def __del__(self):
        if getattr(self, "_s", None):
            _lib().icua_tok_stream_free(self._s)
            self._s = None
