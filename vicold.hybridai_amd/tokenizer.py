"""ctypes binding of the checkpoint tokenizer (include/hai_tokenizer.h), with
the reference's QwenTokenizer interface (src/tokenizer/qwen_tokenizer.h:
15-104): load a checkpoint directory, encode, decode, build_chat_prompt and
the generation config's eos / pad / bos ids.  Host code only."""
from __future__ import annotations

import ctypes

VP, I32, I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
I64P = ctypes.POINTER(ctypes.c_int64)
OK, INVALID_ARGUMENT = 0, 1

_bound = None


def _lib():
    global _bound
    if _bound is None:
        from . import host
        lib = host()
        lib.hai_tokenizer_open.restype = VP
        lib.hai_tokenizer_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(I32), ctypes.c_char_p, I64]
        lib.hai_tokenizer_close.restype = None
        lib.hai_tokenizer_close.argtypes = [VP]
        lib.hai_tokenizer_encode.restype = I32
        lib.hai_tokenizer_encode.argtypes = [VP, ctypes.c_char_p, I64, I64P, I64, I64P]
        lib.hai_tokenizer_decode.restype = I32
        lib.hai_tokenizer_decode.argtypes = [VP, I64P, I64, I32, ctypes.c_char_p, I64, I64P]
        lib.hai_tokenizer_chat_prompt.restype = I32
        lib.hai_tokenizer_chat_prompt.argtypes = [ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_char_p),
                                                  I64, I32, I32, ctypes.c_char_p, I64, I64P]
        lib.hai_tokenizer_special_ids.restype = I32
        lib.hai_tokenizer_special_ids.argtypes = [VP, I64P, I64, I64P, I64P, I64P]
        lib.hai_tokenizer_pieces.restype = I32
        lib.hai_tokenizer_pieces.argtypes = [VP, ctypes.c_char_p, I64, I64P, I64, I64P]
        _bound = lib
    return _bound


class TokenizerError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"({code}) {message}")
        self.code = code


def _sized(call, ctype, per_item=1):
    """Runs call(buffer, capacity, n_out) with a size query first."""
    n = I64(0)
    rc = call(None, 0, ctypes.byref(n))
    if rc == OK:
        return (ctype * 0)(), 0
    if rc != INVALID_ARGUMENT or n.value <= 0:
        raise TokenizerError(rc, "tokenizer call failed")
    buf = (ctype * (n.value * per_item + 1))()
    rc = call(buf, len(buf), ctypes.byref(n))
    if rc != OK:
        raise TokenizerError(rc, "tokenizer call failed")
    return buf, n.value


class QwenTokenizer:
    """tokenizer::QwenTokenizer over a checkpoint directory."""

    def __init__(self, model_dir):
        lib = _lib()
        status, msg = I32(0), ctypes.create_string_buffer(512)
        self._h = lib.hai_tokenizer_open(str(model_dir).encode(), ctypes.byref(status), msg, len(msg))
        if not self._h:
            raise TokenizerError(status.value, msg.value.decode(errors="replace"))
        self._lib = lib

    def close(self):
        if getattr(self, "_h", None):
            self._lib.hai_tokenizer_close(self._h)
            self._h = None

    __del__ = close

    @staticmethod
    def _bytes(text):
        return text.encode() if isinstance(text, str) else bytes(text)

    def encode(self, text, add_special_tokens=True):
        """Token ids of text (str or UTF-8 bytes); add_special_tokens is
        accepted as the reference's is and adds nothing."""
        del add_special_tokens
        b = self._bytes(text)
        buf, n = _sized(lambda out, cap, n: self._lib.hai_tokenizer_encode(self._h, b, len(b), out, cap, n),
                        ctypes.c_int64)
        return list(buf[:n])

    def decode_bytes(self, ids, skip_special_tokens=False):
        arr = (ctypes.c_int64 * max(1, len(ids)))(*ids)
        buf, n = _sized(lambda out, cap, nn: self._lib.hai_tokenizer_decode(
            self._h, arr, len(ids), int(skip_special_tokens), out, cap, nn), ctypes.c_char)
        return bytes(buf[:n])

    def decode(self, ids, skip_special_tokens=False):
        """Text of ids (bytes that are not UTF-8 decode as U+FFFD)."""
        return self.decode_bytes(ids, skip_special_tokens).decode(errors="replace")

    def pieces(self, text):
        """Byte ranges of the pre-tokenizer's pieces of text."""
        b = self._bytes(text)
        buf, n = _sized(lambda out, cap, nn: self._lib.hai_tokenizer_pieces(self._h, b, len(b), out, cap, nn),
                        ctypes.c_int64, per_item=2)
        return [(buf[2 * k], buf[2 * k + 1]) for k in range(n)]

    @staticmethod
    def build_chat_prompt(messages, add_generation_prompt=True, enable_thinking=True):
        lib = _lib()
        roles = (ctypes.c_char_p * max(1, len(messages)))(*[r.encode() for r, _ in messages])
        contents = (ctypes.c_char_p * max(1, len(messages)))(*[c.encode() for _, c in messages])
        buf, n = _sized(lambda out, cap, nn: lib.hai_tokenizer_chat_prompt(
            roles, contents, len(messages), int(add_generation_prompt), int(enable_thinking), out, cap, nn),
            ctypes.c_char)
        return bytes(buf[:n]).decode()

    def _special(self):
        eos, n, pad, bos = (ctypes.c_int64 * 64)(), I64(0), I64(0), I64(0)
        rc = self._lib.hai_tokenizer_special_ids(self._h, eos, 64, ctypes.byref(n), ctypes.byref(pad),
                                                 ctypes.byref(bos))
        if rc != OK:
            raise TokenizerError(rc, "special ids")
        return list(eos[:n.value]), pad.value, bos.value

    def eos_token_ids(self):
        return self._special()[0]

    def is_eos_token(self, token_id):
        return token_id in self.eos_token_ids()

    def pad_token_id(self):
        return self._special()[1]

    def bos_token_id(self):
        return self._special()[2]
