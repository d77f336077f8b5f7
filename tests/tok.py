"""A small Qwen-style tokenizer.json for tests, made by the HF `tokenizers`
library (the library Qwen checkpoints' tokenizer.json files are written
for): a byte-level BPE trained on a fixed multilingual corpus, split by the
Qwen pre-tokenizer pattern, with Qwen's special tokens (<|endoftext|>,
<|im_start|>, <|im_end|>) and non-special added tokens (<think>, </think>,
<tool_call>).  Test helper only."""
import json
from pathlib import Path

from tokenizers import AddedToken, Regex, Tokenizer, decoders, models, pre_tokenizers, trainers

QWEN_PATTERN = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?[\p{L}\p{M}]+|\p{N}"
                r"| ?[^\s\p{L}\p{M}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+")
SPECIAL = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]
ADDED = ["<think>", "</think>", "<tool_call>"]

_BASE = [
    "The quick brown fox jumps over the lazy dog. It's a dog's life, isn't it? We'll see; they've gone.",
    "I'M SURE YOU'RE RIGHT, BUT HE'D SAY IT'S NOT. Don't worry: we're fine, you'll manage.",
    "Speculative decoding drafts tokens with a small head and verifies them with the target model.",
    "def forward(x, cache):\n    h = self.norm(x)\n    return h @ self.weight.T + self.bias\n",
    "for (int i = 0; i < n; ++i) {\n\tsum += a[i] * b[i];\n}\n",
    "Numbers: 3.14159, 2,718, 1e-6, 0x7fff, 42%, $100.00, 2026-12-02 04:10:58.",
    "你好，世界！今天的天气很好。我们一起去公园散步吧。机器学习和深度学习。",
    "こんにちは、世界。カタカナとひらがなと漢字を混ぜた文章です。",
    "안녕하세요, 세계! 한국어 문장도 포함되어 있습니다.",
    "Привет, мир! Это предложение на русском языке с числами 123 и знаками.",
    "Ελληνικά: Καλημέρα κόσμε. Français : « où est la bibliothèque ? » Español: ¿Qué tal?",
    "नमस्ते दुनिया। यह हिंदी वाक्य है। สวัสดีครับ ภาษาไทย العربية: مرحبا بالعالم",
    "Emoji 🙂🙂 👍🏽 and symbols → ⇒ ≤ ≥ ∑ ∫ ©®™ … — – ‘quoted’ “double”.",
    "    indented line\n\n\n  two blank lines above\r\nwindows line\r\n\ttab\tseparated\tvalues\n",
    "<|im_start|>user\nWhat is 2+2?<|im_end|>\n<|im_start|>assistant\n<think>\nsimple\n</think>\n\n4<|im_end|>",
]


def corpus():
    lines = []
    for k in range(40):
        for i, s in enumerate(_BASE):
            lines.append(s if (k + i) % 3 else s.lower())
            lines.append(" ".join(reversed(s.split(" "))))
    return lines


def write_tokenizer(path, vocab_size=1500, merges_as="default", ignore_merges=None, generation=None):
    """Writes <path>/tokenizer.json (and generation_config.json when
    generation is a dict); merges_as "strings" or "pairs" rewrites the merges
    list in that form."""
    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(QWEN_PATTERN), behavior="isolated"),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=vocab_size, initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                                  show_progress=False)
    tok.train_from_iterator(corpus(), trainer)
    tok.add_special_tokens([AddedToken(t, special=True, normalized=False) for t in SPECIAL])
    tok.add_tokens([AddedToken(t, special=False, normalized=False) for t in ADDED])
    f = path / "tokenizer.json"
    tok.save(str(f))
    if merges_as != "default" or ignore_merges is not None:
        raw = json.loads(f.read_text())
        m = raw["model"]["merges"]
        pairs = [x.split(" ", 1) if isinstance(x, str) else x for x in m]
        if merges_as == "strings":
            raw["model"]["merges"] = [" ".join(p) for p in pairs]
        elif merges_as == "pairs":
            raw["model"]["merges"] = pairs
        if ignore_merges is not None:
            raw["model"]["ignore_merges"] = ignore_merges
        f.write_text(json.dumps(raw, ensure_ascii=False))
    if generation is not None:
        (path / "generation_config.json").write_text(json.dumps(generation))
    return path


def hf(path):
    return Tokenizer.from_file(str(Path(path) / "tokenizer.json"))
