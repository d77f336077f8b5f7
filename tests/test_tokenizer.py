"""The checkpoint tokenizer (include/hai_tokenizer.h) on the CPU.

Checked against the HF `tokenizers` library -- the library Qwen checkpoints'
tokenizer.json files are written for, and the one the reference's own
tokenizer-debug scripts compare with -- on a byte-level BPE tokenizer.json
that library trains here (tests/tok.py): token ids, the pre-tokenizer's
pieces, and decoding, over fixed multilingual strings and seeded random
strings from tricky and from arbitrary codepoints.  The reference's own
tokenizer tests (tests/qwen_tokenizer_test.cc:46-94) are restated, and its
chat layout and load errors (qwen_tokenizer.cc:59-187, 490-503) checked.
Inputs are NFC strings: the reference applies no normalizer, and neither
does this tokenizer."""
import json
import random
import time

import pytest

import tok

FILE_NOT_FOUND, INVALID_MODEL = 7, 8

FIXED = [
    "", " ", "\n", "'", "''", "'s", "a'", "x'S'", "I'M here, you'RE not; they'LL've gone, he'D know.",
    "don't DON'T Don'T it'ſ a'ſx 'll'LL'Ll", "It’s a curly apostrophe’s case",
    "a  b", "a   \n\n  b", "\t\tx", "trailing   ", "  leading", "\r\n\r\n", "x \u00a0y", "\u3000全角スペース",
    "line\u2028sep\u2029para", "a\u0085b", "  \n\t hi", "a  ", "\n\n\nword", " \n word", "x\r\r\ny",
    "12345 ٣٤٥ ４５ x² Ⅻ ½", "12,3.5e-7", "e\u0301 \u0301start a\u0301\u0302b", "नमस्ते दुनिया", "สวัสดีครับ",
    "你好，世界！", "こんにちは、世界。カタカナ", "안녕하세요", "Привет, мир!", "¿Qué tal? «quote» ‘x’",
    "👍🏽 family: 👨‍👩‍👧 🙂🙂🙂", "a+b=c; x->y || z&&w", "====", "...!!!???", "@user #tag $100 C:\\path\\file",
    "def f(x):\n    return x**2\n", "for (int i = 0; i < n; ++i) {\n\t sum += a[i];\n}",
    "\u0870\u0871 \U00010D40\U00010D41 \u0897",  # letters / marks / digits of Unicode 14-16
    "<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n<think>\n\n</think>\n\n",
    "<think>inline</think>", "partial <|im_sta", "<|im_end|><|im_end|>", "x<tool_call>y", "<|endoftext|>",
]

TRICKY = (list(" \n\r\t'sSſtTrReEvVmMlLdD") + ["\u00a0", "\u3000", "\u0301", "\u0300", "1", "٣", "²", ".", ",", "!",
          "-", "_", "(", "é", "ß", "中", "文", "ア", "한", "я", "🙂", "\u200b", "\u2028", "<think>", "<|im_end|>"])


def random_strings(seed, n, alphabet=None):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        k = rng.randint(1, 40)
        if alphabet is not None:
            out.append("".join(rng.choice(alphabet) for _ in range(k)))
        else:
            cps = []
            while len(cps) < k:
                c = rng.randrange(0x110000) if rng.random() < 0.5 else rng.randrange(0x3000)
                if not 0xD800 <= c <= 0xDFFF:
                    cps.append(chr(c))
            out.append("".join(cps))
    return out


@pytest.fixture(scope="module")
def T():
    from hybridai_amd import tokenizer
    return tokenizer


@pytest.fixture(scope="module")
def tdir(tmp_path_factory):
    return tok.write_tokenizer(tmp_path_factory.mktemp("tok"),
                               generation={"bos_token_id": 1075, "eos_token_id": [1077, 1075], "pad_token_id": 1075})


@pytest.fixture(scope="module")
def pair(T, tdir):
    return T.QwenTokenizer(tdir), tok.hf(tdir)


@pytest.mark.parametrize("strings", ["fixed", "tricky", "codepoints"])
def test_encode_matches_hf(pair, strings):
    ours, hf = pair
    cases = {"fixed": FIXED, "tricky": random_strings(1, 1500, TRICKY), "codepoints": random_strings(2, 400)}[strings]
    for s in cases:
        assert ours.encode(s) == hf.encode(s).ids, repr(s)


@pytest.mark.parametrize("strings", ["fixed", "tricky", "codepoints"])
def test_pieces_match_hf_split(pair, strings):
    """The pre-tokenizer pattern alone, on texts without added tokens."""
    ours, _ = pair
    from tokenizers import Regex, pre_tokenizers
    split = pre_tokenizers.Split(Regex(tok.QWEN_PATTERN), behavior="isolated")
    cases = {"fixed": FIXED, "tricky": random_strings(3, 1500, TRICKY[:-2]), "codepoints": random_strings(4, 400)}
    for s in cases[strings]:
        if "<" in s:
            continue
        b = s.encode()
        assert [b[x:y].decode() for x, y in ours.pieces(s)] == [p for p, _ in split.pre_tokenize_str(s)], repr(s)


def test_decode_matches_hf_and_round_trips(pair):
    ours, hf = pair
    for s in FIXED + random_strings(5, 300, TRICKY) + random_strings(6, 100):
        ids = hf.encode(s).ids
        assert ours.decode(ids) == hf.decode(ids, skip_special_tokens=False) == s, repr(s)
        assert ours.decode(ids, skip_special_tokens=True) == hf.decode(ids, skip_special_tokens=True), repr(s)


def test_bytes_that_are_not_utf8_are_kept(pair):
    """Ill-formed UTF-8 (a lone continuation byte, a truncated sequence, an
    overlong form, a surrogate) is tokenized byte by byte and decodes back."""
    ours, _ = pair
    for b in [b"\x80", b"ab\xe4\xbd", b"\xc0\xaf", b"\xed\xa0\x80x", b"ok \xff\xfe end", b"\xf0\x9f\x99"]:
        assert ours.decode_bytes(ours.encode(b)) == b


def test_special_ids_and_chat_layout(T, pair):
    ours, _ = pair
    assert ours.eos_token_ids() == [1077, 1075] and ours.pad_token_id() == 1075 and ours.bos_token_id() == 1075
    msgs = [("system", "Be brief."), ("user", "2+2?")]
    body = "<|im_start|>system\nBe brief.<|im_end|>\n<|im_start|>user\n2+2?<|im_end|>\n"
    assert T.QwenTokenizer.build_chat_prompt(msgs, False, True) == body
    assert T.QwenTokenizer.build_chat_prompt(msgs, True, True) == body + "<|im_start|>assistant\n<think>\n"
    assert T.QwenTokenizer.build_chat_prompt(msgs, True, False) == \
        body + "<|im_start|>assistant\n<think>\n\n</think>\n\n"
    # the chat prompt's markers are added tokens, encoded whole
    ids = ours.encode(T.QwenTokenizer.build_chat_prompt([("user", "hi")], True, False))
    assert ids[0] == 1076 and ids.count(1077) == 1 and ids.count(1076) == 2


@pytest.mark.parametrize("merges_as,ignore_merges", [("strings", None), ("pairs", None), ("default", True)])
def test_merges_forms_and_ignore_merges(T, tmp_path, merges_as, ignore_merges):
    d = tok.write_tokenizer(tmp_path, merges_as=merges_as, ignore_merges=ignore_merges)
    ours, hf = T.QwenTokenizer(d), tok.hf(d)
    for s in FIXED + random_strings(7, 300, TRICKY):
        assert ours.encode(s) == hf.encode(s).ids, repr(s)


def test_long_text_is_fast(pair):
    ours, hf = pair
    text = "\n".join(tok.corpus()) * 2
    t0 = time.perf_counter()
    ids = ours.encode(text)
    dt = time.perf_counter() - t0
    assert ids == hf.encode(text).ids
    assert dt < 2.0, f"{len(text)} chars in {dt:.2f} s"


# -- the reference's tests (tests/qwen_tokenizer_test.cc) -------------------

def ref_dir(path, added, generation=None):
    path.mkdir(parents=True, exist_ok=True)
    (path / "tokenizer.json").write_text(json.dumps(
        {"model": {"type": "BPE", "vocab": {"a": 0, "b": 1}, "merges": []}, "added_tokens": added}))
    if generation is not None:
        (path / "generation_config.json").write_text(json.dumps(
            {"bos_token_id": 100, "eos_token_id": generation, "pad_token_id": 101}))
    return path


def test_ref_added_tokens_above_vocabulary_decode_verbatim(T, tmp_path):
    d = ref_dir(tmp_path, [{"id": 100, "content": "<|im_end|>", "special": True},
                           {"id": 102, "content": "<think>", "special": False}], [100, 103])
    t = T.QwenTokenizer(d)
    assert t.decode([0, 100, 102, 1]) == "a<|im_end|><think>b"
    assert t.decode([0, 100, 102, 1], skip_special_tokens=True) == "a<think>b"


def test_ref_scalar_and_array_generation_ids(T, tmp_path):
    d = ref_dir(tmp_path, [], [100, 103])
    t = T.QwenTokenizer(d)
    assert t.eos_token_ids() == [100, 103] and t.is_eos_token(100) and t.is_eos_token(103)
    assert not t.is_eos_token(101) and t.bos_token_id() == 100 and t.pad_token_id() == 101
    ref_dir(tmp_path, [], 102)
    assert T.QwenTokenizer(d).eos_token_ids() == [102]


def test_ref_reload_clears_added_tokens(T, tmp_path):
    d = ref_dir(tmp_path, [{"id": 100, "content": "<old>", "special": False}])
    assert T.QwenTokenizer(d).decode([100]) == "<old>"
    ref_dir(tmp_path, [{"id": 101, "content": "<new>", "special": False}])
    t = T.QwenTokenizer(d)
    assert t.decode([100]) == "" and t.decode([101]) == "<new>"


def test_ref_non_special_added_token_encodes_whole(T, tmp_path):
    d = ref_dir(tmp_path, [{"id": 102, "content": "<think>", "special": False}])
    assert T.QwenTokenizer(d).encode("a<think>b") == [0, 102, 1]


def test_longest_added_token_wins(T, tmp_path):
    d = ref_dir(tmp_path, [{"id": 10, "content": "<a>", "special": False},
                           {"id": 11, "content": "<a><b>", "special": True}])
    assert T.QwenTokenizer(d).encode("a<a><b>b<a>") == [0, 11, 1, 10]


@pytest.mark.parametrize("case,code", [
    ("missing", FILE_NOT_FOUND), ("not_json", INVALID_MODEL), ("no_model", INVALID_MODEL),
    ("wordpiece", INVALID_MODEL), ("merge_not_in_vocab", INVALID_MODEL), ("bad_id", INVALID_MODEL),
    ("eos_string", INVALID_MODEL), ("eos_array_string", INVALID_MODEL), ("eos_null", INVALID_MODEL),
    ("generation_not_json", INVALID_MODEL)])
def test_load_errors(T, tmp_path, case, code):
    model = {"type": "BPE", "vocab": {"a": 0, "b": 1, "ab": 2}, "merges": ["a b"]}
    gen = None
    if case == "not_json":
        (tmp_path / "tokenizer.json").write_text('{"model": ')
    elif case != "missing":
        root = {"model": model}
        if case == "no_model":
            root = {"added_tokens": []}
        elif case == "wordpiece":
            model["type"] = "WordPiece"
        elif case == "merge_not_in_vocab":
            model["merges"] = ["a c"]
        elif case == "bad_id":
            model["vocab"]["c"] = "3"
        gen = {"eos_string": '{"eos_token_id": "2"}', "eos_array_string": '{"eos_token_id": [1, "2"]}',
               "eos_null": '{"eos_token_id": null}', "generation_not_json": "{eos"}.get(case)
        (tmp_path / "tokenizer.json").write_text(json.dumps(root))
        if gen is not None:
            (tmp_path / "generation_config.json").write_text(gen)
    with pytest.raises(T.TokenizerError) as e:
        T.QwenTokenizer(tmp_path)
    assert e.value.code == code
