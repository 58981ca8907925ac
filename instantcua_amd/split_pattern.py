"""Compiler of a tokenizer.json ``Split`` pattern into the program the native pre-tokenizer runs.

Hugging Face ``tokenizers`` splits text with an Oniguruma regex (the Qwen2 pattern is
``QWEN2_SPLIT`` in tokenizer.py; the reference hard-codes it as ``qwen2SplitRegex``,
Sources/Tokenizer/Tokenizer.swift).  Here the pattern is not re-implemented by hand: it is parsed,
checked and lowered to a small instruction set, and its character classes are evaluated once
over every code point.  The native side (``tokenizer.cpp``) runs the program with a memoised
backtracking matcher, which has Oniguruma's leftmost-first semantics and runs in time linear in
(program length x text length).

Supported syntax (a subset of Oniguruma's Ruby syntax; anything else is rejected, so a pattern
that compiles means what Oniguruma means by it):

* alternation ``|``, groups ``(...)``, ``(?:...)``, ``(?i:...)``, ``(?-i:...)``;
* quantifiers ``? * + {m} {m,} {m,n} {,n}``, each greedy or lazy (``??`` ...);
* lookahead ``(?=c)`` / ``(?!c)`` of one character class ``c``;
* character classes ``[...]`` and ``[^...]`` with ranges, ``.``, and the escapes ``\\s \\S \\d
  \\D \\p{..} \\P{..} \\p{^..} \\r \\n \\t \\f \\v \\a \\e \\xHH \\x{H..} \\uHHHH`` and escaped
  punctuation.  ``\\p`` takes a general category (``L``, ``Lu``, ``N``, ``Nd``, ...) or its long
  name (``Letter``, ``Number``, ...).  ``\\s`` is Unicode White_Space and ``\\d`` is ``Nd``.
  ``\\w`` is refused: Oniguruma builds it on the Alphabetic property, which unicodedata lacks.
* Case-insensitive groups match a character when its simple case folding equals that of a
  member: ``(?i:'s)`` matches ``'s``, ``'S`` and ``'\\u017f``.

A pattern that can match the empty string is rejected: Split would then have to choose what an
empty match means, and the reference's pattern never does.

Program (four int32 per instruction, ``op, a, b, guard``):

====  ===========  ==========================================================================
 op   name         meaning at text position p
====  ===========  ==========================================================================
 0    MATCH        the match ends at p
 1    CLASS a      the code point at p is in class a: advance past it, else fail
 2    SPLIT a b g  try a; if that fails, try b (a is preferred: leftmost-first priority).
                   g >= 0 is the class of every code point that can begin a match through a:
                   when the code point at p is not in it (or the text has ended), go to b
 3    JMP a        continue at a
 4    AHEAD a      zero-width: a code point follows p and is in class a
 5    NOT_AHEAD a  zero-width: no code point follows p, or it is not in class a
====  ===========  ==========================================================================

``guard`` is -1 for every other instruction, and for a SPLIT whose branch a can reach MATCH
without consuming a code point.
"""
from __future__ import annotations

import unicodedata
from typing import List, Tuple

import numpy as np

MATCH, CLASS, SPLIT, JMP, AHEAD, NOT_AHEAD = range(6)
MAX_PROGRAM = 4096
N_CODEPOINTS = 0x110000

CATEGORIES = ("Lu", "Ll", "Lt", "Lm", "Lo", "Mn", "Mc", "Me", "Nd", "Nl", "No", "Pc", "Pd", "Ps", "Pe", "Pi", "Pf",
              "Po", "Sm", "Sc", "Sk", "So", "Zs", "Zl", "Zp", "Cc", "Cf", "Cs", "Co", "Cn")
_LONG_NAMES = {"Letter": "L", "Mark": "M", "Number": "N", "Punctuation": "P", "Symbol": "S", "Separator": "Z",
               "Other": "C", "Uppercase_Letter": "Lu", "Lowercase_Letter": "Ll", "Decimal_Number": "Nd"}
# Unicode White_Space (PropList.txt), the set Oniguruma's \s matches.
WHITE_SPACE = (tuple(range(0x09, 0x0E)) + (0x20, 0x85, 0xA0, 0x1680) + tuple(range(0x2000, 0x200B))
               + (0x2028, 0x2029, 0x202F, 0x205F, 0x3000))


class PatternError(ValueError):
    """The split pattern uses syntax the native pre-tokenizer does not run."""


# --- character data -------------------------------------------------------------------------

_UCD = None


def unicode_data():
    """(general category index u8, simple case fold i32) for every code point, from unicodedata.

    The simple fold of c is ``c.casefold()`` when that is one character, else c itself: Python's
    casefold is Unicode full folding, which agrees with the simple (C) folding wherever the full
    result is a single character."""
    global _UCD
    if _UCD is None:
        cat_index = {c: i for i, c in enumerate(CATEGORIES)}
        gc = np.empty(N_CODEPOINTS, dtype=np.uint8)
        fold = np.arange(N_CODEPOINTS, dtype=np.int32)
        for cp in range(N_CODEPOINTS):
            ch = chr(cp)
            gc[cp] = cat_index[unicodedata.category(ch)]
            f = ch.casefold()
            if len(f) == 1 and f != ch:
                fold[cp] = ord(f)
        _UCD = (gc, fold)
    return _UCD


# --- parser -----------------------------------------------------------------------------------
# Set expressions (evaluated later over every code point):
#   ("range", lo, hi) | ("gc", (cat, ...)) | ("ws",) | ("or", [s, ...]) | ("not", s) | ("fold", s)
# Pattern nodes:
#   ("set", s) | ("seq", [n, ...]) | ("alt", [n, ...]) | ("rep", n, lo, hi_or_None, greedy)
#   | ("ahead", negated, s)

_SIMPLE_ESCAPES = {"r": 0x0D, "n": 0x0A, "t": 0x09, "f": 0x0C, "v": 0x0B, "a": 0x07, "e": 0x1B}


def _gc_set(name: str):
    name = _LONG_NAMES.get(name, name)
    cats = tuple(c for c in CATEGORIES if c == name or (len(name) == 1 and c[0] == name))
    if not cats:
        raise PatternError(f"unknown property \\p{{{name}}}")
    return ("gc", cats)


_DIGIT = ("gc", ("Nd",))
_SPACE = ("ws",)


class _Parser:
    def __init__(self, pattern: str):
        self.s, self.i = pattern, 0

    def fail(self, what: str):
        raise PatternError(f"{what} (offset {self.i} of {self.s!r})")

    def peek(self, k: int = 0):
        j = self.i + k
        return self.s[j] if j < len(self.s) else None

    def eat(self, text: str) -> bool:
        if self.s.startswith(text, self.i):
            self.i += len(text)
            return True
        return False

    def parse(self):
        node = self.alternation(False)
        if self.i < len(self.s):
            self.fail("unbalanced ')'")
        return node

    def alternation(self, icase: bool):
        branches = [self.sequence(icase)]
        while self.eat("|"):
            branches.append(self.sequence(icase))
        return branches[0] if len(branches) == 1 else ("alt", branches)

    def sequence(self, icase: bool):
        items = []
        while self.peek() not in (None, "|", ")"):
            items.append(self.repeat(icase))
        return items[0] if len(items) == 1 else ("seq", items)

    def interval(self):
        """{m}, {m,}, {m,n}, {,n} at the cursor as (lo, hi), or None (then '{' is a literal)."""
        j = self.s.find("}", self.i)
        if j < 0:
            return None
        body = self.s[self.i + 1:j]
        parts = body.split(",")
        if len(parts) > 2 or not all(p.isdigit() or p == "" for p in parts) or parts[0] == "" and len(parts) == 1:
            return None
        if len(parts) == 1:
            lo = hi = int(parts[0])
        else:
            lo = int(parts[0]) if parts[0] else 0
            hi = int(parts[1]) if parts[1] else None
            if parts[0] == "" and parts[1] == "":
                return None
        if hi is not None and hi < lo:
            self.fail("interval with max < min")
        self.i = j + 1
        return lo, hi

    def repeat(self, icase: bool):
        node = self.atom(icase)
        while True:
            c = self.peek()
            if c in ("?", "*", "+"):
                self.i += 1
                lo, hi = {"?": (0, 1), "*": (0, None), "+": (1, None)}[c]
            elif c == "{" and (iv := self.interval()) is not None:
                lo, hi = iv
            else:
                return node
            greedy = not self.eat("?")
            if self.peek() == "+":
                self.fail("possessive quantifiers are not supported")
            if node[0] == "ahead":
                self.fail("a lookahead cannot be repeated")
            node = ("rep", node, lo, hi, greedy)

    def atom(self, icase: bool):
        c = self.peek()
        if c is None:
            self.fail("pattern ends early")
        self.i += 1
        if c == "(":
            if self.eat("?:"):
                inner = self.alternation(icase)
            elif self.eat("?i:"):
                inner = self.alternation(True)
            elif self.eat("?-i:"):
                inner = self.alternation(False)
            elif self.peek() == "?" and self.peek(1) in ("=", "!"):
                negated = self.peek(1) == "!"
                self.i += 2
                inner = self.alternation(icase)
                if inner[0] != "set":
                    self.fail("a lookahead must hold one character class")
                inner = ("ahead", negated, inner[1])
            elif self.peek() == "?":
                self.fail("unsupported group syntax")
            else:  # a capturing group: Split uses only the whole match
                inner = self.alternation(icase)
            if not self.eat(")"):
                self.fail("missing ')'")
            return inner
        if c == "[":
            return ("set", self.bracket(icase))
        if c == ".":
            return ("set", ("not", ("range", 0x0A, 0x0A)))
        if c == "\\":
            return ("set", self.escape(icase))
        if c in "^$":
            self.fail("anchors are not supported")
        if c in "*+?":
            self.fail("nothing to repeat")
        return ("set", self.literal(ord(c), icase))

    @staticmethod
    def literal(cp: int, icase: bool):
        s = ("range", cp, cp)
        return ("fold", s) if icase else s

    def hex_digits(self, n=None) -> int:
        if n is None:  # \x{...}
            j = self.s.find("}", self.i)
            txt = self.s[self.i:j] if j > self.i else ""
            self.i = j + 1 if j > self.i else self.i
        else:
            txt = self.s[self.i:self.i + n]
            self.i += len(txt)
        try:
            v = int(txt, 16)
        except ValueError:
            self.fail("bad hexadecimal escape")
        if not (0 <= v < N_CODEPOINTS) or len(txt) == 0:
            self.fail("bad hexadecimal escape")
        return v

    def escape(self, icase: bool):
        """The escape after a backslash: a set expression (one code point or a class)."""
        c = self.peek()
        if c is None:
            self.fail("pattern ends in a backslash")
        self.i += 1
        if c in _SIMPLE_ESCAPES:
            return self.literal(_SIMPLE_ESCAPES[c], icase)
        if c == "x":
            v = self.hex_digits(None) if self.eat("{") else self.hex_digits(2)
            return self.literal(v, icase)
        if c == "u":
            return self.literal(self.hex_digits(4), icase)
        classes = {"s": _SPACE, "d": _DIGIT}
        if c.lower() in classes:
            s = classes[c.lower()]
            return ("not", s) if c.isupper() else s
        if c in "pP":
            if not self.eat("{"):
                self.fail("\\p needs {name}")
            neg = c == "P"
            if self.eat("^"):
                neg = not neg
            j = self.s.find("}", self.i)
            if j < 0:
                self.fail("unterminated \\p{")
            s = _gc_set(self.s[self.i:j])
            self.i = j + 1
            if icase:
                s = ("fold", s)
            return ("not", s) if neg else s
        if c.isalnum():
            self.fail(f"unsupported escape \\{c}")
        return self.literal(ord(c), icase)

    def bracket(self, icase: bool):
        neg = self.eat("^")
        items = []
        first = True
        while True:
            c = self.peek()
            if c is None:
                self.fail("unterminated character class")
            if c == "]":
                if first:
                    self.fail("empty character class")
                self.i += 1
                break
            first = False
            if c == "[" or self.s.startswith("&&", self.i):
                self.fail("nested classes and class intersection are not supported")
            lo = self.bracket_item()
            if self.peek() == "-" and self.peek(1) not in ("]", None):
                self.i += 1
                hi = self.bracket_item()
                if lo[0] != "range" or hi[0] != "range" or lo[1] != lo[2] or hi[1] != hi[2] or hi[1] < lo[1]:
                    self.fail("bad range in character class")
                lo = ("range", lo[1], hi[1])
            items.append(lo)
        s = ("or", items)
        if icase:
            s = ("fold", s)
        return ("not", s) if neg else s

    def bracket_item(self):
        c = self.peek()
        self.i += 1
        if c == "\\":
            return self.escape(False)
        return ("range", ord(c), ord(c))


def parse(pattern: str):
    return _Parser(pattern).parse()


def _nullable(node) -> bool:
    kind = node[0]
    if kind == "set":
        return False
    if kind == "ahead":
        return True
    if kind == "seq":
        return all(_nullable(n) for n in node[1])
    if kind == "alt":
        return any(_nullable(n) for n in node[1])
    return node[2] == 0 or _nullable(node[1])


# --- set evaluation -------------------------------------------------------------------------

def _members(s, memo: dict) -> np.ndarray:
    key = repr(s)
    if key in memo:
        return memo[key]
    gc, fold = unicode_data()
    kind = s[0]
    if kind == "range":
        m = np.zeros(N_CODEPOINTS, dtype=bool)
        m[s[1]:s[2] + 1] = True
    elif kind == "gc":
        m = np.isin(gc, [CATEGORIES.index(c) for c in s[1]])
    elif kind == "ws":
        m = np.zeros(N_CODEPOINTS, dtype=bool)
        m[list(WHITE_SPACE)] = True
    elif kind == "or":
        m = np.zeros(N_CODEPOINTS, dtype=bool)
        for x in s[1]:
            m |= _members(x, memo)
    elif kind == "not":
        m = ~_members(s[1], memo)
    elif kind == "fold":
        inner = _members(s[1], memo)
        m = inner | np.isin(fold, np.unique(fold[inner]))
    else:
        raise AssertionError(kind)
    memo[key] = m
    return m


# --- lowering ---------------------------------------------------------------------------------

class SplitProgram:
    """A compiled pattern: ``code`` int32[n, 4] and ``classes`` bool[n_classes, 0x110000]."""

    def __init__(self, pattern: str):
        self.pattern = pattern
        tree = parse(pattern)
        if _nullable(tree):
            raise PatternError(f"the pattern can match the empty string: {pattern!r}")
        self._code: List[Tuple[int, int, int]] = []
        self._class_ids = {}
        self._memo = {}
        self._sets: List[np.ndarray] = []
        self._emit(tree)
        self._code.append((MATCH, 0, 0))
        guards = [self._guard(at) if op == SPLIT else -1 for at, (op, _, _) in enumerate(self._code)]
        self.code = np.array([c + (g,) for c, g in zip(self._code, guards)], dtype=np.int32).reshape(-1, 4)
        self.classes = np.stack(self._sets) if self._sets else np.zeros((0, N_CODEPOINTS), bool)
        del self._memo

    def _class(self, s) -> int:
        return self._class_of(_members(s, self._memo))

    def _guard(self, split_at: int) -> int:
        """Class of the code points that can begin a path from the preferred target of the SPLIT at
        split_at (zero-width instructions are passed through), or -1 when MATCH is reachable
        without consuming one."""
        todo, seen, first = [self._code[split_at][1]], set(), []
        while todo:
            pc = todo.pop()
            if pc in seen:
                continue
            seen.add(pc)
            op, a, b = self._code[pc]
            if op == MATCH:
                return -1
            if op == CLASS:
                first.append(a)
            elif op == SPLIT:
                todo += [a, b]
            elif op == JMP:
                todo.append(a)
            else:
                todo.append(pc + 1)
        m = np.zeros(N_CODEPOINTS, dtype=bool)
        for k in set(first):
            m |= self._sets[k]
        return self._class_of(m)

    def _class_of(self, m: np.ndarray) -> int:
        key = np.packbits(m).tobytes()
        if key not in self._class_ids:
            self._class_ids[key] = len(self._sets)
            self._sets.append(m)
        return self._class_ids[key]

    def _put(self, op, a=0, b=0) -> int:
        if len(self._code) >= MAX_PROGRAM:
            raise PatternError(f"the pattern needs more than {MAX_PROGRAM} instructions")
        self._code.append((op, a, b))
        return len(self._code) - 1

    def _patch(self, at: int, a=None, b=None):
        op, a0, b0 = self._code[at]
        self._code[at] = (op, a0 if a is None else a, b0 if b is None else b)

    def _set_choice(self, at: int, enter: int, skip: int, greedy: bool):
        self._patch(at, *((enter, skip) if greedy else (skip, enter)))

    def _emit(self, node):
        kind = node[0]
        if kind == "set":
            self._put(CLASS, self._class(node[1]))
        elif kind == "ahead":
            self._put(NOT_AHEAD if node[1] else AHEAD, self._class(node[2]))
        elif kind == "seq":
            for n in node[1]:
                self._emit(n)
        elif kind == "alt":
            exits = []
            for n in node[1][:-1]:
                at = self._put(SPLIT)
                self._emit(n)
                exits.append(self._put(JMP))
                self._patch(at, at + 1, len(self._code))
            self._emit(node[1][-1])
            for at in exits:
                self._patch(at, len(self._code))
        else:
            _, body, lo, hi, greedy = node
            for _ in range(lo):
                self._emit(body)
            if hi is None:  # loop: L: SPLIT body, out; body; JMP L
                at = self._put(SPLIT)
                self._emit(body)
                self._put(JMP, at)
                self._set_choice(at, at + 1, len(self._code), greedy)
            else:  # hi - lo nested optional copies, every skip leaving the whole construct
                outs = []
                for _ in range(hi - lo):
                    outs.append(self._put(SPLIT))
                    self._emit(body)
                for at in outs:
                    self._set_choice(at, at + 1, len(self._code), greedy)

    def tables(self):
        """Two-stage bitmaps of the classes: (index u16[n_classes, 4352], blocks u8[n_blocks, 32]),
        class k holds cp when bit (cp & 255) of blocks[index[k, cp >> 8]] is set (LSB first)."""
        nk = self.classes.shape[0]
        rows = np.packbits(self.classes.reshape(nk * 4352, 256), axis=1, bitorder="little")
        uniq, inverse = np.unique(rows, axis=0, return_inverse=True)
        if uniq.shape[0] > 0xFFFF:
            raise PatternError("character classes too irregular for the bitmap tables")
        return inverse.reshape(nk, 4352).astype(np.uint16), np.ascontiguousarray(uniq, dtype=np.uint8)
