"""ctypes binding of the C++ verify engine (include/hai_engine.h)."""
from __future__ import annotations

import ctypes

import numpy as np

VP = ctypes.c_void_p
I64 = ctypes.c_int64
I32P = ctypes.POINTER(ctypes.c_int32)
U16P = ctypes.POINTER(ctypes.c_uint16)
ROUND_RECORD = 16


class ModelConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "hidden", "num_layers", "full_attention_interval", "num_q_heads", "num_kv_heads", "head_dim",
        "rope_dim", "lin_qk_heads", "lin_v_heads", "lin_k_dim", "lin_v_dim", "conv_kernel", "ffn", "vocab",
        "mtp_layers")] + [("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float)]


WEIGHTS_BF16, WEIGHTS_FP8_BLOCK128 = 0, 1


class EngineOptions(ctypes.Structure):
    _fields_ = [("max_context", ctypes.c_int32), ("max_verify_tokens", ctypes.c_int32),
                ("device", ctypes.c_int32), ("use_graphs", ctypes.c_int32), ("weight_format", ctypes.c_int32),
                ("max_batch", ctypes.c_int32), ("mfma", ctypes.c_int32), ("prefill_rows", ctypes.c_int32)]


class SpecStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in (
        "rounds", "proposed", "accepted", "rejected", "corrections", "replay_tokens", "mtp_recovery_tokens",
        "max_proposal_width", "emitted")] + [(n, ctypes.c_double) for n in (
            "prefill_seconds", "decode_seconds", "draft_seconds", "verify_seconds", "correction_seconds")] + [
                ("host_syncs", ctypes.c_int64)]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


class VerifyProfile(ctypes.Structure):
    _fields_ = [(n, ctypes.c_double) for n in (
        "verify_ms", "gemm_ms", "gemm_bytes", "gemm_launches", "step_bytes", "draft_ms", "draft_bytes")]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


TINY = dict(hidden=256, num_layers=4, full_attention_interval=4, num_q_heads=4, num_kv_heads=2, head_dim=64,
            rope_dim=16, lin_qk_heads=4, lin_v_heads=4, lin_k_dim=64, lin_v_dim=64, conv_kernel=4, ffn=768,
            vocab=4096, mtp_layers=1, rms_eps=1e-6, rope_theta=1e7)
QWEN27B = dict(hidden=5120, num_layers=64, full_attention_interval=4, num_q_heads=24, num_kv_heads=4,
               head_dim=256, rope_dim=64, lin_qk_heads=16, lin_v_heads=48, lin_k_dim=128, lin_v_dim=128,
               conv_kernel=4, ffn=17408, vocab=248320, mtp_layers=1, rms_eps=1e-6, rope_theta=1e7)


def bind(lib: ctypes.CDLL) -> ctypes.CDLL:
    lib.hai_engine_create.restype = VP
    lib.hai_engine_create.argtypes = [ctypes.POINTER(ModelConfig), ctypes.POINTER(EngineOptions)]
    lib.hai_engine_destroy.restype = None
    lib.hai_engine_destroy.argtypes = [VP]
    lib.hai_engine_last_error.restype = ctypes.c_char_p
    lib.hai_engine_last_error.argtypes = [VP]
    lib.hai_engine_init_synthetic.argtypes = [VP, ctypes.c_uint64, ctypes.c_float]
    lib.hai_engine_read_tensor.restype = I64
    lib.hai_engine_read_tensor.argtypes = [VP, ctypes.c_uint32, U16P, I64]
    lib.hai_engine_weight_bytes.restype = ctypes.c_uint64
    lib.hai_engine_weight_bytes.argtypes = [VP]
    lib.hai_engine_forward.argtypes = [VP, I32P, I64, U16P, U16P]
    lib.hai_engine_generate_greedy.argtypes = [VP, I32P, I64, I64, I32P, I64, I32P]
    lib.hai_engine_generate_speculative.argtypes = [VP, I32P, I64, I64, I64, I32P, I64, I32P, I64, I32P,
                                                    ctypes.POINTER(SpecStats), I32P, I64]
    lib.hai_engine_prefill.argtypes = [VP, I32P, I64, I64]
    lib.hai_engine_spec_rounds.argtypes = [VP, I64, I64, I32P, I64, ctypes.POINTER(ctypes.c_int64),
                                           ctypes.POINTER(SpecStats)]
    lib.hai_engine_profile_verify.argtypes = [VP, I64, I64, ctypes.POINTER(VerifyProfile)]
    lib.hai_engine_set_draft_override.argtypes = [VP, I32P, I64]
    lib.hai_engine_set_prefill_rows.argtypes = [VP, I64]
    lib.hai_model_config_load.argtypes = [ctypes.c_char_p, ctypes.POINTER(ModelConfig), ctypes.POINTER(ctypes.c_int64),
                                          I64, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int32),
                                          ctypes.c_char_p, I64]
    lib.hai_model_config_load.restype = ctypes.c_int
    lib.hai_engine_load_checkpoint.argtypes = [VP, ctypes.c_char_p]
    lib.hai_engine_load_checkpoint.restype = ctypes.c_int
    lib.hai_engine_forward_batch.argtypes = [VP, I32P, I64, U16P, U16P]
    lib.hai_engine_generate_speculative_batch.argtypes = [VP, I32P, I64, I64, I64, I32P, I64, I32P, I64, I32P,
                                                          ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(SpecStats),
                                                          I32P, I64]
    lib.hai_engine_batch.restype = I64
    lib.hai_engine_batch.argtypes = [VP]
    for n in ("hai_engine_init_synthetic", "hai_engine_forward", "hai_engine_generate_greedy",
              "hai_engine_generate_speculative", "hai_engine_prefill", "hai_engine_spec_rounds",
              "hai_engine_profile_verify", "hai_engine_forward_batch", "hai_engine_generate_speculative_batch",
              "hai_engine_set_draft_override", "hai_engine_set_prefill_rows"):
        getattr(lib, n).restype = ctypes.c_int
    return lib


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


class CheckpointError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"({code}) {message}")
        self.code = code


def model_config_load(model_dir, weight_format=True):
    """<model_dir>/config.json (and, with weight_format, the checkpoint's
    Linear format) -> (config dict as TINY / QWEN27B, eos ids, format)."""
    from . import host
    lib = host()
    c = ModelConfig()
    eos = (ctypes.c_int64 * 64)()
    n_eos = ctypes.c_int64(0)
    fmt = ctypes.c_int32(-1)
    msg = ctypes.create_string_buffer(1024)
    rc = lib.hai_model_config_load(str(model_dir).encode(), ctypes.byref(c), eos, 64, ctypes.byref(n_eos),
                                   ctypes.byref(fmt) if weight_format else None, msg, 1024)
    if rc != 0:
        raise CheckpointError(rc, msg.value.decode())
    cfg = {n: getattr(c, n) for n, _ in ModelConfig._fields_}
    return cfg, [int(eos[i]) for i in range(min(64, n_eos.value))], (fmt.value if weight_format else None)


class Engine:
    """One verify engine on one GPU (synthetic weights, or a checkpoint
    through load_checkpoint)."""

    def __init__(self, cfg: dict, max_context: int, max_verify_tokens: int = 16, device: int = 0,
                 use_graphs: bool = False, fp8: bool = False, batch: int = 1, mfma: bool = False,
                 prefill_rows: int = 0):
        from . import host
        self.lib = host()
        self.cfg = dict(cfg)
        self.fp8 = fp8
        self.batch = batch
        c = ModelConfig(**cfg)
        o = EngineOptions(max_context, max_verify_tokens, device, int(use_graphs),
                          WEIGHTS_FP8_BLOCK128 if fp8 else WEIGHTS_BF16, batch, int(mfma), int(prefill_rows))
        self.h = self.lib.hai_engine_create(ctypes.byref(c), ctypes.byref(o))
        if not self.h:
            raise RuntimeError("hai_engine_create: " + self.lib.hai_engine_last_error(None).decode())

    def _check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} ({rc}): " + self.lib.hai_engine_last_error(self.h).decode())

    def close(self):
        if getattr(self, "h", None):
            self.lib.hai_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def init_synthetic(self, seed=0, std=0.02):
        self._check(self.lib.hai_engine_init_synthetic(self.h, seed, std), "init_synthetic")

    def load_checkpoint(self, model_dir):
        self._check(self.lib.hai_engine_load_checkpoint(self.h, str(model_dir).encode()), "load_checkpoint")

    def weight_bytes(self) -> int:
        return int(self.lib.hai_engine_weight_bytes(self.h))

    def read_tensor(self, tid: int) -> np.ndarray:
        n = self.lib.hai_engine_read_tensor(self.h, tid, None, 0)
        if n < 0:
            raise KeyError(tid)
        out = np.empty(n, np.uint16)
        got = self.lib.hai_engine_read_tensor(self.h, tid, out.ctypes.data_as(U16P), n)
        if got != n:
            raise RuntimeError("read_tensor failed")
        return out

    def forward(self, ids):
        ids = _i32(ids)
        T = ids.size
        H, V = self.cfg["hidden"], self.cfg["vocab"]
        hid = np.empty((T, H), np.uint16)
        lg = np.empty((T, V), np.uint16)
        self._check(self.lib.hai_engine_forward(self.h, ids.ctypes.data_as(I32P), T, hid.ctypes.data_as(U16P),
                                                lg.ctypes.data_as(U16P)), "forward")
        return hid, lg

    def greedy(self, prompt, max_new, eos=()):
        p = _i32(prompt)
        e = _i32(list(eos))
        out = np.empty(max_new, np.int32)
        n = self.lib.hai_engine_generate_greedy(self.h, p.ctypes.data_as(I32P), p.size, max_new,
                                                e.ctypes.data_as(I32P), e.size, out.ctypes.data_as(I32P))
        if n < 0:
            self._check(-n, "generate_greedy")
        return out[:n]

    def speculative(self, prompt, max_new, width=1, eos=(), draft_override=None, max_rounds=4096):
        p = _i32(prompt)
        e = _i32(list(eos))
        out = np.empty(max_new, np.int32)
        st = SpecStats()
        log = np.full((max_rounds, ROUND_RECORD), -1, np.int32)
        if draft_override is not None:
            ov = _i32(draft_override)
            ovp, nov = ov.ctypes.data_as(I32P), ov.size
        else:
            ovp, nov = None, 0
        n = self.lib.hai_engine_generate_speculative(self.h, p.ctypes.data_as(I32P), p.size, max_new, width,
                                                     e.ctypes.data_as(I32P), e.size, ovp, nov,
                                                     out.ctypes.data_as(I32P), ctypes.byref(st),
                                                     log.ctypes.data_as(I32P), max_rounds)
        if n < 0:
            self._check(-n, "generate_speculative")
        return out[:n], st.as_dict(), log[:st.rounds]

    def forward_batch(self, ids):
        """ids [B][T] -> hidden [B][T][H], logits [B][T][V] (bf16 bits)."""
        ids = _i32(ids).reshape(self.batch, -1)
        T = ids.shape[1]
        H, V = self.cfg["hidden"], self.cfg["vocab"]
        hid = np.empty((self.batch, T, H), np.uint16)
        lg = np.empty((self.batch, T, V), np.uint16)
        self._check(self.lib.hai_engine_forward_batch(self.h, ids.ctypes.data_as(I32P), T,
                                                      hid.ctypes.data_as(U16P), lg.ctypes.data_as(U16P)),
                    "forward_batch")
        return hid, lg

    def speculative_batch(self, prompts, max_new, width=1, eos=(), draft_override=None, max_rounds=4096):
        """prompts [B][P] -> per sequence (tokens, stats, round log)."""
        p = _i32(prompts).reshape(self.batch, -1)
        e = _i32(list(eos))
        B = self.batch
        out = np.empty((B, max_new), np.int32)
        n = np.zeros(B, np.int64)
        st = (SpecStats * B)()
        log = np.full((B, max_rounds, ROUND_RECORD), -1, np.int32)
        if draft_override is not None:
            ov = _i32(draft_override).reshape(B, -1)
            ovp, nov = ov.ctypes.data_as(I32P), ov.shape[1]
        else:
            ovp, nov = None, 0
        rc = self.lib.hai_engine_generate_speculative_batch(
            self.h, p.ctypes.data_as(I32P), p.shape[1], max_new, width, e.ctypes.data_as(I32P), e.size, ovp, nov,
            out.ctypes.data_as(I32P), n.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), st,
            log.ctypes.data_as(I32P), max_rounds)
        if rc < 0:
            self._check(-rc, "generate_speculative_batch")
        return [(out[b, :n[b]], st[b].as_dict(), log[b, :st[b].rounds]) for b in range(B)]

    def prefill(self, prompt, max_new):
        """prompt [P] (one sequence) or [B][P]."""
        p = _i32(prompt).reshape(self.batch, -1)
        self._check(self.lib.hai_engine_prefill(self.h, p.ctypes.data_as(I32P), p.shape[1], max_new), "prefill")

    def spec_rounds(self, rounds, width, out: np.ndarray):
        """out [cap] or [B][cap]; returns (tokens emitted so far, summed over
        the sequences) and the summed stats of these rounds."""
        out2 = out.reshape(self.batch, -1)
        n = np.zeros(self.batch, np.int64)
        st = SpecStats()
        self._check(self.lib.hai_engine_spec_rounds(self.h, rounds, width, out2.ctypes.data_as(I32P),
                                                    out2.shape[1], n.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                                    ctypes.byref(st)), "spec_rounds")
        return int(n.sum()), st.as_dict()

    def set_draft_override(self, tokens):
        """tokens [n] or [B][n]: drafts of spec_rounds for output positions
        < n (None clears)."""
        if tokens is None:
            self._check(self.lib.hai_engine_set_draft_override(self.h, None, 0), "set_draft_override")
            return
        t = _i32(tokens).reshape(self.batch, -1)
        self._check(self.lib.hai_engine_set_draft_override(self.h, t.ctypes.data_as(I32P), t.shape[1]),
                    "set_draft_override")

    def set_prefill_rows(self, rows):
        """Prefill mode of the next prompts (0: through the verify step)."""
        self._check(self.lib.hai_engine_set_prefill_rows(self.h, int(rows)), "set_prefill_rows")

    def profile_verify(self, T, iters):
        pr = VerifyProfile()
        self._check(self.lib.hai_engine_profile_verify(self.h, T, iters, ctypes.byref(pr)), "profile_verify")
        return pr.as_dict()


def _splitmix64(x: np.ndarray) -> np.ndarray:
    x = x + np.uint64(0x9E3779B97F4A7C15)
    x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return x ^ (x >> np.uint64(31))


def synthetic_prompt(seed: int, n: int, vocab: int) -> np.ndarray:
    """Uniform prompt ids: splitmix64 counter stream 0xFFFF of the seed, mod
    vocab (the same stream the CPU oracle uses for its prompts)."""
    with np.errstate(over="ignore"):
        key = _splitmix64(np.array([np.uint64(seed) ^ (np.uint64(0xFFFF) << np.uint64(32))], np.uint64))[0]
        h = _splitmix64(key + np.arange(n, dtype=np.uint64))
    return (h % np.uint64(vocab)).astype(np.int32)
