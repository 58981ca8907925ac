"""Parity of the native Qwen2 tokenizer (include/icua_tok.h; Sources/Tokenizer/Tokenizer.swift,
Core.swift, Compile.swift) with Hugging Face `tokenizers` on the same tokenizer.json.

The reference tokenizer restates HF's Qwen2 pipeline ("exactly like HF", Tokenizer.swift:157-165,
340-341): NFC, the Qwen2 split pattern, byte-level BPE, added tokens matched on the raw text,
ByteLevel decoding.  The real Qwen tokenizer.json is not available offline, so the vocabularies
here are BPE models trained by `tokenizers` on a synthetic multilingual corpus, with the Qwen
added tokens.  Text is drawn from characters of Unicode 13 or older (the interpreter's
unicodedata version), so both sides share their character properties."""
import json
import random

import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

tokenizers = pytest.importorskip("tokenizers")
from tokenizers import Regex, decoders, models, normalizers, pre_tokenizers, trainers  # noqa: E402

from instantcua_amd import tokenizer as itok  # noqa: E402

WORDS = ["hello", "world", "click", "button", "the", "Menu", "café", "naïve", "Ångström", "日本語", "テスト", "中文字",
         "한국어", "Ωmega", "Привет", "مرحبا", "12345", "x=3;", "a+=b", "don't", "we'll", "I'M", "they're", "YOU'VE",
         "it'd", "(10, 20)", "click(x, y)", "<div>", "   ", "\n\n", "\r\n", "\t", "naïveté", "½", "²", "٣", "Ⅻ",
         "emoji🙂", "🙂🙂", "ﬁ", "ǅ", "İstanbul", "straße"]
SPECIALS = ["<|endoftext|>", "<|im_start|>", "<|im_end|>", "<|vision_start|>", "<|vision_end|>", "<|image_pad|>",
            "<tool_call>"]
# Characters for fuzzing: every split-pattern class and NFC case (combining marks in both orders,
# Hangul jamo, singletons, compatibility characters NFC keeps).
PALETTE = list("abcXYZ éèÅ日本語한국ΩЖ0123456789٣²Ⅻ.,;:!?'\"()[]{}<>+-*/=_#@$%^&~|\\`") + \
    ["́", "̈", "̣", "̧", "é", "ậ", "각", "가",
     "Å", "Ω", "ﬁ", " ", "  ", "\t", "\n", "\r\n", " ", "　", " ", "\u0085", "'s", "'S",
     "'ll", "'LL", "'re", "'VE", "'d", "'m", "'t", "'x", "🙂", "​", "­"]


# Split patterns of other byte-level BPE tokenizers (GPT-2's, and the one of Llama 3 / GPT-4 with
# digit runs of at most three), plus constructs the compiler supports beyond them.
GPT2_SPLIT = r"""'s|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+"""
LLAMA3_SPLIT = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}{1,3}| ?[^\s\p{L}\p{N}]+[\r\n]*|"
                r"\s*[\r\n]+|\s+(?!\S)|\s+")
EXTRA_SPLITS = [r"\p{Lu}?\p{Ll}+|\d{2,}?|[\x{4e00}-\x{9fff}]|(?i:[a-c]+x)|\S", r"[\p{L}\p{M}]+(?=\s)|\P{L}|.",
                r"(?:ab|a)+?c|\P{L}+|\p{^N}"]


def _train(vocab_size, seed, pattern=None):
    tok = tokenizers.Tokenizer(models.BPE())
    tok.normalizer = normalizers.NFC()
    tok.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(pattern or itok.QWEN2_SPLIT), behavior="isolated"),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    tok.decoder = decoders.ByteLevel()
    rng = random.Random(seed)
    corpus = ["".join(rng.choice(WORDS) + rng.choice([" ", "", "  ", "\n", ", "]) for _ in range(24))
              for _ in range(3000)]
    trainer = trainers.BpeTrainer(vocab_size=vocab_size, initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                                  show_progress=False)
    tok.train_from_iterator(corpus, trainer)
    tok.add_special_tokens(SPECIALS)
    return tokenizers.Tokenizer.from_str(tok.to_str())


@pytest.fixture(scope="module", params=[(700, 1), (3000, 2), (700, 3, LLAMA3_SPLIT)],
                ids=["v700", "v3000", "llama3-split"])
def pair(request, tmp_path_factory):
    hf = _train(*request.param)
    d = tmp_path_factory.mktemp("tok")
    js = str(d / "tokenizer.json")
    hf.save(js)
    out = str(d / "tokenizer.ict")
    itok.compile(js, out)
    ours = itok.Tokenizer(out)
    yield hf, ours
    ours.close()


def hf_ids(hf, text):
    return hf.encode(text, add_special_tokens=False).ids


SAMPLES = ["", "hello world", "  leading and trailing  ", "a\n\n\nb", "x \n y\t\tz ", "line\r\n\r\nnext",
           "don't we'll I'M they're YOU'VE it'd 'sun 'LLama", "café naïve Ångström", "é ậ ö́",
           "각가 한국어", "ÅΩ ﬁ ǅ", "12345 ٣² Ⅻ", "click(120, 45)", "a+=b; x==y",
           "日本語テスト中文字", "emoji🙂🙂 done", " nbsp　ideo em", "tab\tword", "end with spaces   ",
           "x" * 200, "abc" * 50 + " " + "日本" * 40, "́ leading mark", "'", "''s", "a'", "123abc456",
           "İstanbul straße ΣΑΣ"]


def test_encode_matches_hf(pair):
    hf, ours = pair
    for s in SAMPLES:
        assert ours.encode(s) == hf_ids(hf, s), repr(s)


def test_added_tokens_match_hf(pair):
    hf, ours = pair
    for s in ["<|im_start|>system\nYou are a GUI agent.<|im_end|>\n<|im_start|>user\n",
              "text<|im_end|><|im_end|>x<tool_call>y", "<|im_start", "<|image_pad|>" * 3, "a<|endoftext|>b"]:
        assert ours.encode_with_specials(s) == hf_ids(hf, s), repr(s)
    # Plain encode does not match them (a literal special is text).
    assert ours.encode("<|im_end|>") != hf_ids(hf, "<|im_end|>")
    assert ours.im_end == hf.token_to_id("<|im_end|>") and ours.im_start == hf.token_to_id("<|im_start|>")
    assert ours.end_of_text == hf.token_to_id("<|endoftext|>")
    assert ours.vocab_size == hf.get_vocab_size()


def test_chat_templates(pair):
    hf, ours = pair
    system, user = "You are a helpful GUI agent. café", "Click the 'OK' button<|im_end|>?"
    text = f"<|im_start|>system\n{system}<|im_end|>\n<|im_start|>user\n{user}<|im_end|>\n<|im_start|>assistant\n"
    assert ours.encode_chat(system, user) == hf_ids(hf, text)
    toks, off = ours.encode_vision_chat(system, user, 12)
    pre = hf_ids(hf, f"<|im_start|>system\n{system}<|im_end|>\n<|im_start|>user\n")
    suf = hf_ids(hf, f"{user}<|im_end|>\n<|im_start|>assistant\n")
    assert toks == pre + [itok.VISION_START] + [itok.IMAGE_PAD] * 12 + [itok.VISION_END] + suf
    assert off == len(pre) + 1 and toks[off:off + 12] == [itok.IMAGE_PAD] * 12


def test_decode_and_stream_match_hf(pair):
    hf, ours = pair
    rng = random.Random(5)
    n = hf.get_vocab_size()
    cases = [hf_ids(hf, s) for s in SAMPLES] + [[rng.randrange(n) for _ in range(rng.randrange(1, 30))]
                                               for _ in range(200)]
    for ids in cases:
        want = hf.decode(ids, skip_special_tokens=False)
        assert ours.decode(ids) == want, ids
        stream = itok.TextStream(ours)
        got = "".join(stream.push(i) for i in ids) + stream.finish()
        assert got == want, ids
    assert ours.decode([-1, 10 ** 9]) == ""


@settings(max_examples=400, deadline=None, suppress_health_check=[HealthCheck.function_scoped_fixture])
@given(parts=st.lists(st.sampled_from(PALETTE), max_size=40))
def test_fuzz_encode_matches_hf(pair, parts):
    hf, ours = pair
    s = "".join(parts)
    assert ours.encode(s) == hf_ids(hf, s), repr(s)


def test_rejects_other_pipelines(tmp_path, pair):
    hf, _ = pair
    root = json.loads(hf.to_str())
    root["normalizer"] = {"type": "NFKC"}
    p = tmp_path / "bad.json"
    p.write_text(json.dumps(root))
    with pytest.raises(itok.TokenizerError, match="NFC"):
        itok.compile(str(p), str(tmp_path / "bad.ict"))
    root = json.loads(hf.to_str())
    root["model"]["ignore_merges"] = True
    p.write_text(json.dumps(root))
    with pytest.raises(itok.TokenizerError, match="ignore_merges"):
        itok.compile(str(p), str(tmp_path / "bad.ict"))
    with pytest.raises(itok.TokenizerError):
        itok.Tokenizer(str(p))  # not a compiled file


_RUN_SCRIPT = r"""
import ctypes as C, resource, sys
import numpy as np
sys.path.insert(0, sys.argv[2])
from instantcua_amd import tokenizer as itok
tok = itok.Tokenizer(sys.argv[1])
text = b" " * (4 << 20)
out = np.zeros(len(text) + 1, dtype=np.int32)  # touched: its pages count before the call
n = C.c_size_t(0)
fn = itok._lib().icua_tok_encode
assert fn(tok._h, b"a b", 3, 0, out.ctypes.data_as(C.c_void_p), out.size, C.byref(n)) == 0
before = resource.getrusage(resource.RUSAGE_SELF).ru_maxrss
assert fn(tok._h, text, len(text), 0, out.ctypes.data_as(C.c_void_p), out.size, C.byref(n)) == 0
after = resource.getrusage(resource.RUSAGE_SELF).ru_maxrss
print(n.value, after - before)
"""


def test_long_runs_are_cut_into_bounded_pieces(pair, tmp_path):
    """A match reads at most 16 KiB past its start (tokenizer.cpp MAX_PIECE): below that the pieces
    are HF's; a longer run becomes pieces of 16 KiB, the text still round-trips, and the memory an
    encode takes does not grow with the run (a visited set and stack per byte of a 4 MiB run would
    take ~100 MB; the limit here is the output buffers')."""
    hf, ours = pair
    for s in [" " * 5000 + "x", "a" * 9000, "7" * 12000, "\n" * 3000 + "y", "日" * 5000]:
        assert ours.encode(s) == hf_ids(hf, s)
    for s in [" " * 70000, "b" * 50000 + " c", "x" + "\t" * 40000]:
        assert ours.decode(ours.encode(s)) == s
    import os
    import subprocess
    import sys
    js = str(tmp_path / "tokenizer.json")
    hf.save(js)
    ict = str(tmp_path / "tokenizer.ict")
    itok.compile(js, ict)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _RUN_SCRIPT, ict, root], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    n_tokens, grew_kib = (int(v) for v in r.stdout.split())
    assert 0 < n_tokens <= 4 << 20
    assert grew_kib < 48 * 1024, grew_kib


def test_invalid_utf8_is_rejected(pair):
    import ctypes as C
    _, ours = pair
    n = C.c_size_t(0)
    L = itok._lib()
    assert L.icua_tok_encode(ours._h, b"\xff\xfe", 2, 0, None, 0, C.byref(n)) == -1
    assert b"UTF-8" in L.icua_tok_last_error()


# --- the split program against HF's Split -----------------------------------------------------

def _run_program(prog, text, start):
    """End (code-point index) of the leftmost-first match of a compiled split program at start, or
    -1: a plain backtracking interpreter of the instruction set of split_pattern, written from its
    table, with no memo and no guards (so it also checks that both only skip dead paths)."""
    from instantcua_amd import split_pattern as sp
    stack = [(0, start)]
    while stack:
        pc, p = stack.pop()
        while True:
            op, a, b, _ = (int(x) for x in prog.code[pc])
            if op == sp.MATCH:
                return p
            if op == sp.SPLIT:
                stack.append((b, p))
                pc = a
                continue
            if op == sp.JMP:
                pc = a
                continue
            inside = p < len(text) and bool(prog.classes[a, ord(text[p])])
            if op == sp.CLASS:
                if not inside:
                    break
                p += 1
            elif inside != (op == sp.AHEAD):
                break
            pc += 1
    return -1


def _program_split(prog, text):
    out, gap, i = [], 0, 0
    while i < len(text):
        e = _run_program(prog, text, i)
        if e > i:
            out += [text[gap:i]] if gap < i else []
            out.append(text[i:e])
            i = gap = e
        else:
            i += 1
    return out + ([text[gap:]] if gap < len(text) else [])


ALL_SPLITS = [itok.QWEN2_SPLIT, GPT2_SPLIT, LLAMA3_SPLIT] + EXTRA_SPLITS


@pytest.fixture(scope="module")
def programs():
    from instantcua_amd.split_pattern import SplitProgram
    return [(SplitProgram(p), pre_tokenizers.Split(Regex(p), behavior="isolated")) for p in ALL_SPLITS]


def test_split_program_matches_hf_split(programs):
    rng = random.Random(11)
    texts = SAMPLES + ["".join(rng.choice(PALETTE) for _ in range(rng.randrange(1, 30))) for _ in range(300)] + \
        ["abcabx ABX aBcX abababc 12345 1 x", "ſ 'ſ 'ſt 'K 'k", "aaab ab abc ababc", "日本 語x  \u000b\u000c\u001c"]
    for prog, hf_split in programs:
        for t in texts:
            want = [piece for piece, _ in hf_split.pre_tokenize_str(t)]
            assert _program_split(prog, t) == want, (prog.pattern, t)


@pytest.mark.parametrize("pattern,why", [
    (r"a|", "empty"), (r"x*", "empty"), (r"(?=a)", "empty"), (r"^a", "anchor"), (r"a$", "anchor"),
    (r"(a)\1", "escape"), (r"a++", "possessive"), (r"(?<=a)b", "group"), (r"\p{Foo}", "property"),
    (r"[[a]]", "nested"), (r"[a&&b]", "intersection"), (r"(?!ab)c", "lookahead"), (r"(a", "missing"),
    (r"a)", "unbalanced"), (r"*a", "repeat"), (r"a{3,2}", "max < min"), (r"\w+", "escape"), (r"(?=a)+b", "repeated"),
])
def test_split_patterns_outside_the_compiler_are_refused(pattern, why):
    from instantcua_amd.split_pattern import PatternError, SplitProgram
    with pytest.raises(PatternError, match=why):
        SplitProgram(pattern)


def test_pipeline_report_names_every_unmet_requirement(tmp_path, pair):
    hf, _ = pair
    root = json.loads(hf.to_str())
    root["pre_tokenizer"]["pretokenizers"][1]["add_prefix_space"] = True
    root["model"]["dropout"] = 0.1
    root["decoder"] = {"type": "Metaspace"}
    with pytest.raises(itok.TokenizerError) as e:
        itok.check_pipeline(root)
    msg = str(e.value)
    for path in ("pretokenizers.1.add_prefix_space", "model.dropout", "decoder.type"):
        assert path in msg
    assert "normalizer" not in msg
    root = json.loads(hf.to_str())
    root["pre_tokenizer"]["pretokenizers"][0]["pattern"] = {"Regex": r"\s*"}
    p = tmp_path / "empty.json"
    p.write_text(json.dumps(root))
    with pytest.raises(itok.TokenizerError, match="empty string"):
        itok.compile(str(p), str(tmp_path / "x.ict"))


def test_corrupt_compiled_files_are_refused(tmp_path, pair):
    import struct
    hf, _ = pair
    js, good = tmp_path / "t.json", tmp_path / "t.ict"
    hf.save(str(js))
    itok.compile(str(js), str(good))
    raw = bytearray(good.read_bytes())
    n_sec = struct.unpack_from("<I", raw, 8)[0]
    entries = {struct.unpack_from("<4s", raw, 16 + 24 * k)[0].decode(): struct.unpack_from("<IQQ", raw, 20 + 24 * k)
               for k in range(n_sec)}

    def refused(buf, what):
        p = tmp_path / "bad.ict"
        p.write_bytes(bytes(buf))
        with pytest.raises(itok.TokenizerError, match=what):
            itok.Tokenizer(str(p))

    refused(raw[:len(raw) // 2], "section")
    _, off, count = entries["PROG"]
    bad = bytearray(raw)
    struct.pack_into("<i", bad, off + 16 * 0 + 4, count + 5)  # SPLIT target past the end
    refused(bad, "split program")
    bad = bytearray(raw)
    struct.pack_into("<i", bad, off + 16 * (count - 1), 1)  # last instruction no longer MATCH
    refused(bad, "split program|instruction")
    _, off, _ = entries["MRGE"]
    bad = bytearray(raw)
    struct.pack_into("<I", bad, off, 10 ** 8)
    refused(bad, "merge")
    bad = bytearray(raw)
    struct.pack_into("<I", bad, 4, 1)
    refused(bad, "version")
