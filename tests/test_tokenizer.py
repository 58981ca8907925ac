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


def _train(vocab_size, seed):
    tok = tokenizers.Tokenizer(models.BPE())
    tok.normalizer = normalizers.NFC()
    tok.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(itok.QWEN2_SPLIT), behavior="isolated"),
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


@pytest.fixture(scope="module", params=[(700, 1), (3000, 2)], ids=["v700", "v3000"])
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


def test_invalid_utf8_is_rejected(pair):
    import ctypes as C
    _, ours = pair
    n = C.c_size_t(0)
    L = itok._lib()
    assert L.icua_tok_encode(ours._h, b"\xff\xfe", 2, 0, None, 0, C.byref(n)) == -1
    assert b"UTF-8" in L.icua_tok_last_error()
