"""Qwen2 tokenizer: compile step (Python) and the native tokenizer of ``libicua.so`` (ctypes).

``compile`` takes the place of ``Tokenizer.compile(tokenizerJSON:output:)`` (Sources/Tokenizer/
Compile.swift:20-258).  It checks a Hugging Face ``tokenizer.json`` against ``REQUIREMENTS`` (the
pipeline the native tokenizer runs: NFC, one regex Split, byte-level BPE), decodes the
byte-level alphabet back to raw bytes, compiles the Split regex (``split_pattern``) and writes one
file of tagged sections that ``icua_tok_open`` reads:

====  =====  ===========================================================================
tag   elem   contents
====  =====  ===========================================================================
TOFF  u32    byte offset of every token in TBYT, n_tokens + 1 entries
TBYT  u8     the tokens' raw bytes (vocabulary and added tokens)
BYTK  i32    the token of every single byte, 256 entries
MRGE  3xu32  merges in rank order: (left id, right id, result id)
SPEC  3xu32  added tokens: (id, offset in SBYT, length), matched leftmost-longest
SBYT  u8     the added tokens' bytes
PROG  4xi32  the split program (op, a, b, guard)
CIDX  u16    per class, the block of each 256-code-point range (classes x 4352)
CBIT  32xu8  256-bit membership blocks, LSB first
CCCI  u16    the block of each 256-code-point range of the canonical combining classes
CCCD  256xu8 combining-class blocks
DKEY  u32    code points with a canonical decomposition, ascending
DVAL  u32    offset << 5 | length of each decomposition in DDAT
DDAT  u32    full canonical decompositions
CKEY  u64    first << 21 | second of every primary composition, ascending
CVAL  u32    the composed code point
====  =====  ===========================================================================

The file starts with (magic, version, number of sections, 0) as u32, then one 24-byte entry per
section (tag, element size u32, offset u64, element count u64); sections are 64-byte aligned.

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
from .split_pattern import PatternError, SplitProgram

# The Split regex of the Qwen2 / Qwen3 tokenizer.json.
QWEN2_SPLIT = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|"
               r"\s*[\r\n]+|\s+(?!\S)|\s+")
FILE_MAGIC, FILE_VERSION = 0x32544349, 2
VISION_START, VISION_END, IMAGE_PAD = 151652, 151653, 151655


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


_MISSING = object()


def _lookup(root, path: str):
    """Value at a dotted path ("pre_tokenizer.pretokenizers.0.type"), or _MISSING."""
    node = root
    for key in path.split("."):
        if isinstance(node, list) and key.isdigit() and int(key) < len(node):
            node = node[int(key)]
        elif isinstance(node, dict) and key in node:
            node = node[key]
        else:
            return _MISSING
    return node


def _is(*allowed):
    return lambda v: v in allowed


def _absent_or(*allowed):
    return lambda v: v is _MISSING or v in allowed


# What the native tokenizer runs, as (path in tokenizer.json, test of the value found there, the
# requirement in words).  The reference accepts the same pipeline (Compile.swift:260-291); here
# the Split regex may be any pattern split_pattern compiles, not only the Qwen2 one.
REQUIREMENTS = (
    ("normalizer.type", _is("NFC"), "NFC normalisation"),
    ("pre_tokenizer.type", _is("Sequence"), "a Sequence pre-tokenizer"),
    ("pre_tokenizer.pretokenizers", lambda v: isinstance(v, list) and len(v) == 2, "exactly two pre-tokenizers"),
    ("pre_tokenizer.pretokenizers.0.type", _is("Split"), "a Split first"),
    ("pre_tokenizer.pretokenizers.0.behavior", _is("Isolated"), "Split behaviour Isolated"),
    ("pre_tokenizer.pretokenizers.0.invert", _absent_or(False), "a Split that is not inverted"),
    ("pre_tokenizer.pretokenizers.0.pattern",
     lambda v: isinstance(v, dict) and len(v) == 1 and ("Regex" in v or "String" in v), "a Regex or String pattern"),
    ("pre_tokenizer.pretokenizers.1.type", _is("ByteLevel"), "a ByteLevel second"),
    ("pre_tokenizer.pretokenizers.1.add_prefix_space", _absent_or(False), "ByteLevel without a prefix space"),
    ("pre_tokenizer.pretokenizers.1.use_regex", _is(False), "ByteLevel without its own regex"),
    ("model.type", _is("BPE"), "a BPE model"),
    ("model.dropout", _absent_or(None), "no BPE dropout"),
    ("model.byte_fallback", _absent_or(False, None), "no byte fallback"),
    ("model.continuing_subword_prefix", _absent_or(None, ""), "no continuing-subword prefix"),
    ("model.end_of_word_suffix", _absent_or(None, ""), "no end-of-word suffix"),
    ("model.ignore_merges", _absent_or(False, None), "merges always applied"),
    ("model.vocab", lambda v: isinstance(v, dict), "a vocabulary"),
    ("model.merges", lambda v: isinstance(v, list), "a merge list"),
    ("decoder.type", _absent_or("ByteLevel"), "a ByteLevel decoder"),
)


def check_pipeline(root: dict) -> None:
    """Raise TokenizerError naming every requirement the tokenizer.json does not meet."""
    unmet = []
    for path, ok, want in REQUIREMENTS:
        v = _lookup(root, path)
        if not ok(v):
            found = "absent" if v is _MISSING else json.dumps(v)[:60]
            unmet.append(f"{path} is {found}; needed: {want}")
    if unmet:
        raise TokenizerError("tokenizer.json describes a pipeline this tokenizer does not run:\n  "
                             + "\n  ".join(unmet))


def split_program(root: dict) -> SplitProgram:
    pat = root["pre_tokenizer"]["pretokenizers"][0]["pattern"]
    regex = pat["Regex"] if "Regex" in pat else "".join("\\" + c if not c.isalnum() else c for c in pat["String"])
    try:
        return SplitProgram(regex)
    except PatternError as e:
        raise TokenizerError(f"pre_tokenizer.pretokenizers.0.pattern: {e}") from e


_NFC = None


def nfc_tables():
    """Canonical combining classes as a two-stage table (CCCI u16[4352], CCCD u8[blocks, 256]) and
    the canonical decompositions / primary compositions, from the interpreter's unicodedata."""
    global _NFC
    if _NFC is not None:
        return _NFC
    ccc = np.zeros(0x110000, dtype=np.uint8)
    dkeys, dvals, ddata, comp = [], [], [], {}
    for cp in range(0x110000):
        ch = chr(cp)
        ccc[cp] = unicodedata.combining(ch)
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
    blocks, index = np.unique(ccc.reshape(4352, 256), axis=0, return_inverse=True)
    ck = np.array(sorted(comp), dtype=np.uint64)
    _NFC = (index.reshape(4352).astype(np.uint16), np.ascontiguousarray(blocks, dtype=np.uint8),
            np.array(dkeys, np.uint32), np.array(dvals, np.uint32), np.array(ddata, np.uint32),
            ck, np.array([comp[int(k)] for k in ck], np.uint32))
    return _NFC


def _write_sections(path: str, sections) -> int:
    """sections: [(tag, element size, array or bytes)] -> file; returns its size."""
    head = struct.calcsize("<4I") + struct.calcsize("<4sIQQ") * len(sections)
    entries, cur = [], (head + 63) // 64 * 64
    for tag, elem, data in sections:
        raw = data.tobytes() if isinstance(data, np.ndarray) else bytes(data)
        assert len(raw) % elem == 0, tag
        entries.append((tag, elem, cur, len(raw) // elem, raw))
        cur = (cur + len(raw) + 63) // 64 * 64
    buf = bytearray(cur)
    struct.pack_into("<4I", buf, 0, FILE_MAGIC, FILE_VERSION, len(sections), 0)
    for k, (tag, elem, off, count, raw) in enumerate(entries):
        struct.pack_into("<4sIQQ", buf, 16 + 24 * k, tag.encode(), elem, off, count)
        buf[off:off + len(raw)] = raw
    with open(path, "wb") as f:
        f.write(buf)
    return cur


def compile(tokenizer_json: str, output: str) -> int:  # noqa: A001  (mirrors Tokenizer.compile)
    """tokenizer.json -> compiled file; returns its size."""
    with open(tokenizer_json, encoding="utf-8") as f:
        root = json.load(f)
    check_pipeline(root)
    prog = split_program(root)
    model = root["model"]
    vocab, merges = model["vocab"], model["merges"]
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
    try:
        byte_tok = np.array([vocab[b2u[b]] for b in range(256)], dtype=np.int32)
    except KeyError as e:
        raise TokenizerError(f"the vocabulary lacks the single byte {e}") from e
    mtab = np.zeros((len(merges), 3), dtype=np.uint32)
    for r, m in enumerate(merges):
        a, b = m.split(" ", 1) if isinstance(m, str) else m
        if a not in vocab or b not in vocab or a + b not in vocab:
            raise TokenizerError(f"merge {r} ({a!r}, {b!r}) names a token outside the vocabulary")
        mtab[r] = (vocab[a], vocab[b], vocab[a + b])
    tok_off = np.zeros(n_total + 1, dtype=np.uint32)
    tok_off[1:] = np.cumsum([len(t) for t in tok])
    spec_tab = np.zeros((len(added), 3), dtype=np.uint32)
    spec_bytes = b""
    for k, (i, content) in enumerate(added):
        spec_tab[k] = (i, len(spec_bytes), len(content))
        spec_bytes += content
    cidx, cbits = prog.tables()
    ccci, cccd, dk, dv, dd, ck, cv = nfc_tables()
    return _write_sections(output, [
        ("TOFF", 4, tok_off), ("TBYT", 1, b"".join(tok)), ("BYTK", 4, byte_tok), ("MRGE", 12, mtab),
        ("SPEC", 12, spec_tab), ("SBYT", 1, spec_bytes), ("PROG", 16, prog.code), ("CIDX", 2, cidx),
        ("CBIT", 32, cbits), ("CCCI", 2, ccci), ("CCCD", 256, cccd), ("DKEY", 4, dk), ("DVAL", 4, dv),
        ("DDAT", 4, dd), ("CKEY", 8, ck), ("CVAL", 4, cv)])


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

    def _ids(self, fn, *args, cap: int = 256) -> List[int]:
        """Every token holds at least one byte of the text (an added token too), so a buffer of the
        input's length plus the template's tokens is enough the first time."""
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
        return self._ids(_lib().icua_tok_encode, b, len(b), 0, cap=len(b) + 1)

    def encode_with_specials(self, text: str) -> List[int]:
        """Added tokens matched leftmost-longest on the raw text, like HF encode (159)."""
        b = text.encode("utf-8")
        return self._ids(_lib().icua_tok_encode, b, len(b), 1, cap=len(b) + 1)

    def encode_chat(self, system: str, user: str) -> List[int]:
        s, u = system.encode("utf-8"), user.encode("utf-8")
        return self._ids(_lib().icua_tok_encode_chat, s, len(s), u, len(u), cap=len(s) + len(u) + 64)

    def encode_vision_chat(self, system: str, user: str, num_image_tokens: int) -> Tuple[List[int], int]:
        """(tokens, index of the first image pad) (Tokenizer.swift:192-204)."""
        s, u = system.encode("utf-8"), user.encode("utf-8")
        off = C.c_int(0)
        cap = len(s) + len(u) + 64 + num_image_tokens
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
