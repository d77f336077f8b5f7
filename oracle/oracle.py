"""ctypes binding of the CPU parity oracle -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.  It restates Dustray/Vicold.HybridAI's MTP speculative decode
path on the CPU (see oracle.h for the per-function reference citations).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
_lib = None

F32P = ctypes.POINTER(ctypes.c_float)
I64P = ctypes.POINTER(ctypes.c_int64)
I32P = ctypes.POINTER(ctypes.c_int32)


class OrcConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "hidden", "num_layers", "full_attention_interval", "num_q_heads",
        "num_kv_heads", "head_dim", "rope_dim", "lin_qk_heads", "lin_v_heads",
        "lin_k_dim", "lin_v_dim", "conv_kernel", "ffn", "vocab", "mtp_layers")] + [
        ("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float)]


class OrcSpecStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in (
        "rounds", "proposed", "accepted", "rejected", "corrections",
        "replay_tokens", "mtp_recovery_tokens", "max_proposal_width",
        "mtp_cache_clones", "target_cache_clones")]

    def as_dict(self):
        return {n: int(getattr(self, n)) for n, _ in self._fields_}


ROUND_RECORD = 16


def build(force: bool = False) -> Path:
    """Compile liboracle.so with the committed Makefile."""
    cmd = ["make", "-C", str(_HERE)] + (["-B"] if force else [])
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        _lib.orc_model_create.restype = ctypes.c_void_p
        _lib.orc_model_create.argtypes = [ctypes.POINTER(OrcConfig), ctypes.c_uint64, ctypes.c_float]
        _lib.orc_model_destroy.argtypes = [ctypes.c_void_p]
        _lib.orc_model_tensor.restype = ctypes.c_int64
        _lib.orc_model_tensor.argtypes = [ctypes.c_void_p, ctypes.c_uint32, F32P, ctypes.c_int64]
        _lib.orc_forward.argtypes = [ctypes.c_void_p, I32P, ctypes.c_int64, F32P, F32P]
        _lib.orc_generate_greedy.argtypes = [ctypes.c_void_p, I32P, ctypes.c_int64, ctypes.c_int64,
                                             I32P, ctypes.c_int64, I32P]
        _lib.orc_generate_speculative.argtypes = [
            ctypes.c_void_p, I32P, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            I32P, ctypes.c_int64, I32P, ctypes.c_int64, I32P,
            ctypes.POINTER(OrcSpecStats), I32P, ctypes.c_int64]
        _lib.orc_synthetic_weight_bits.restype = ctypes.c_uint16
        _lib.orc_synthetic_weight_bits.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint64,
                                                   ctypes.c_float]
        _lib.orc_synthetic_prompt.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_int64, I32P]
        _lib.orc_set_threads.argtypes = [ctypes.c_int]
        _lib.orc_set_threads.restype = ctypes.c_int
        _lib.orc_model_quantize_fp8.argtypes = [ctypes.c_void_p]
        _lib.orc_fp8_synthetic_scales.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int64, F32P]
        _lib.orc_model_set_tensor.argtypes = [ctypes.c_void_p, ctypes.c_uint32, F32P, ctypes.c_int64]
        _lib.orc_mtp_forward.argtypes = [ctypes.c_void_p, I32P, F32P, ctypes.c_int64, F32P, F32P, F32P]
        _lib.orc_last_mtp_cache.restype = ctypes.c_int64
        _lib.orc_last_mtp_cache.argtypes = [ctypes.c_void_p, F32P, F32P, ctypes.c_int64]
    return _lib


def _f(a):
    return a.ctypes.data_as(F32P)


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- bf16 helpers
def bf16_bits_to_f32(bits) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bits (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r[nan] = ((u[nan] >> 16) | np.uint32(0x40)).astype(np.uint16)
    return r


def round_bf16(x) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ---------------------------------------------------------------- primitives
def cexp(x):
    x = _c32(x); y = np.empty_like(x)
    lib().orc_exp_array(_f(x), _f(y), ctypes.c_int64(x.size)); return y


def clog1p(x):
    x = _c32(x); y = np.empty_like(x)
    lib().orc_log1p_array(_f(x), _f(y), ctypes.c_int64(x.size)); return y


# ---------------------------------------------------------------- ops
def gemm(x, w, round_out=True):
    x = _c32(x); w = _c32(w)
    M, K = x.shape; N = w.shape[0]
    y = np.empty((M, N), np.float32)
    lib().orc_gemm(_f(x), _f(w), _f(y), ctypes.c_int64(M), ctypes.c_int64(N), ctypes.c_int64(K),
                   ctypes.c_int(int(round_out)))
    return y


def rmsnorm(x, w, eps=1e-6, unit_offset=True, round_out=True):
    x = _c32(x); w = _c32(w)
    rows, H = x.shape
    y = np.empty_like(x)
    lib().orc_rmsnorm(_f(x), _f(w), _f(y), ctypes.c_int64(rows), ctypes.c_int64(H),
                      ctypes.c_float(eps), ctypes.c_int(int(unit_offset)), ctypes.c_int(int(round_out)))
    return y


def add(a, b, round_out=True):
    a = _c32(a); b = _c32(b); y = np.empty_like(a)
    lib().orc_add(_f(a), _f(b), _f(y), ctypes.c_int64(a.size), ctypes.c_int(int(round_out)))
    return y


def silu_mul(g, u, round_out=True):
    g = _c32(g); u = _c32(u); y = np.empty_like(g)
    lib().orc_silu_mul(_f(g), _f(u), _f(y), ctypes.c_int64(g.size), ctypes.c_int(int(round_out)))
    return y


def embedding(table, ids):
    table = _c32(table); ids = np.ascontiguousarray(ids, dtype=np.int64)
    V, H = table.shape
    y = np.empty((ids.size, H), np.float32)
    lib().orc_embedding(_f(table), ids.ctypes.data_as(I64P), _f(y), ctypes.c_int64(ids.size),
                        ctypes.c_int64(V), ctypes.c_int64(H))
    return y


def rope_table(pos0, npos, R, base):
    c = np.empty((npos, R // 2), np.float32); s = np.empty_like(c)
    lib().orc_rope_table(_f(c), _f(s), ctypes.c_int64(pos0), ctypes.c_int64(npos), ctypes.c_int64(R),
                         ctypes.c_float(base))
    return c, s


def q_gate_rmsnorm_rope(src, w, T, nq, D, R, pos0, base, eps=1e-6, unit_offset=True, round_out=True):
    src = _c32(src); w = _c32(w)
    q = np.empty((T, nq, D), np.float32); g = np.empty_like(q)
    lib().orc_q_gate_rmsnorm_rope(_f(src), _f(w), _f(q), _f(g), *map(ctypes.c_int64, (T, nq, D, R, pos0)),
                                  ctypes.c_float(base), ctypes.c_float(eps), ctypes.c_int(int(unit_offset)),
                                  ctypes.c_int(int(round_out)))
    return q, g


def k_rmsnorm_rope(src, w, T, nkv, D, R, pos0, base, eps=1e-6, round_out=True):
    src = _c32(src); w = _c32(w)
    k = np.empty((T, nkv, D), np.float32)
    lib().orc_k_rmsnorm_rope(_f(src), _f(w), _f(k), *map(ctypes.c_int64, (T, nkv, D, R, pos0)),
                             ctypes.c_float(base), ctypes.c_float(eps), ctypes.c_int(int(round_out)))
    return k


def partial_rope(src, T, heads, D, R, pos0, base, round_out=False):
    src = _c32(src); dst = np.empty_like(src)
    lib().orc_partial_rope(_f(src), _f(dst), *map(ctypes.c_int64, (T, heads, D, R, pos0)),
                           ctypes.c_float(base), ctypes.c_int(int(round_out)))
    return dst


def attention(q, gate, kc, vc, T, cache_len, nq, nkv, D, round_out=True):
    q = _c32(q); kc = _c32(kc); vc = _c32(vc)
    gp = None
    if gate is not None:
        gate = _c32(gate); gp = _f(gate)
    out = np.empty((T, nq, D), np.float32)
    lib().orc_attention(_f(q), gp, _f(kc), _f(vc), _f(out), *map(ctypes.c_int64, (T, cache_len, nq, nkv, D)),
                        ctypes.c_int(int(round_out)))
    return out


def deltanet_conv(qkv, w, conv_state, T, nk, nv, dk, dv, Kc, round_out=True):
    qkv = _c32(qkv); w = _c32(w)
    st = np.array(conv_state, dtype=np.float32, copy=True)
    q = np.empty((T, nk * dk), np.float32); k = np.empty_like(q); v = np.empty((T, nv * dv), np.float32)
    lib().orc_deltanet_conv(_f(qkv), _f(w), _f(st), _f(q), _f(k), _f(v),
                            *map(ctypes.c_int64, (T, nk, nv, dk, dv, Kc)), ctypes.c_int(int(round_out)))
    return q, k, v, st


def deltanet_recurrent(q, k, v, a, b, z, a_log, dt_bias, norm_w, state, T, nk, nv, dk, dv, eps=1e-6,
                       round_out=True):
    args = [_c32(t) for t in (q, k, v, a, b, z, a_log, dt_bias, norm_w)]
    st = np.array(state, dtype=np.float32, copy=True)
    out = np.empty((T, nv * dv), np.float32)
    lib().orc_deltanet_recurrent(*[_f(t) for t in args], _f(st), _f(out),
                                 *map(ctypes.c_int64, (T, nk, nv, dk, dv)), ctypes.c_float(eps),
                                 ctypes.c_int(int(round_out)))
    return out, st


def argmax_rows(x):
    x = _c32(x)
    rows, cols = x.shape
    out = np.empty(rows, np.int64)
    lib().orc_argmax_rows(_f(x), out.ctypes.data_as(I64P), ctypes.c_int64(rows), ctypes.c_int64(cols))
    return out


# ---------------------------------------------------------------- FP8
U8P = ctypes.POINTER(ctypes.c_uint8)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def fp8_decode(q):
    q = _u8(q); y = np.empty(q.shape, np.float32)
    lib().orc_fp8_decode_array(q.ctypes.data_as(U8P), _f(y), ctypes.c_int64(q.size)); return y


def fp8_encode(x):
    x = _c32(x); q = np.empty(x.shape, np.uint8)
    lib().orc_fp8_encode_array(_f(x), q.ctypes.data_as(U8P), ctypes.c_int64(x.size)); return q


def fp8_dequant_2d(q, s, block_rows, block_cols):
    q = _u8(q); s = _c32(s); rows, cols = q.shape
    w = np.empty((rows, cols), np.float32)
    lib().orc_fp8_dequant_2d(q.ctypes.data_as(U8P), _f(s), _f(w), ctypes.c_int64(rows), ctypes.c_int64(cols),
                             ctypes.c_int64(block_rows), ctypes.c_int64(block_cols))
    return w


def gemm_fp8(x, q, s, round_out=True):
    x = _c32(x); q = _u8(q); s = _c32(s)
    M, K = x.shape; N = q.shape[0]
    y = np.empty((M, N), np.float32)
    lib().orc_gemm_fp8(_f(x), q.ctypes.data_as(U8P), _f(s), _f(y), ctypes.c_int64(M), ctypes.c_int64(N),
                       ctypes.c_int64(K), ctypes.c_int(int(round_out)))
    return y


def fp8_synthetic_scales(seed, tensor_id, n):
    out = np.empty(n, np.float32)
    lib().orc_fp8_synthetic_scales(ctypes.c_uint64(seed), ctypes.c_uint32(tensor_id), ctypes.c_int64(n), _f(out))
    return out


# ---------------------------------------------------------------- model
TINY = dict(hidden=256, num_layers=4, full_attention_interval=4, num_q_heads=4, num_kv_heads=2,
            head_dim=64, rope_dim=16, lin_qk_heads=4, lin_v_heads=4, lin_k_dim=64, lin_v_dim=64,
            conv_kernel=4, ffn=768, vocab=4096, mtp_layers=1, rms_eps=1e-6, rope_theta=1e7)

QWEN27B = dict(hidden=5120, num_layers=64, full_attention_interval=4, num_q_heads=24, num_kv_heads=4,
               head_dim=256, rope_dim=64, lin_qk_heads=16, lin_v_heads=48, lin_k_dim=128, lin_v_dim=128,
               conv_kernel=4, ffn=17408, vocab=248320, mtp_layers=1, rms_eps=1e-6, rope_theta=1e7)


def make_config(d: dict) -> OrcConfig:
    return OrcConfig(**d)


def set_threads(n: int) -> int:
    """OpenMP threads of the oracle's loops (n <= 0 only queries); returns
    the count in effect.  Results do not depend on it."""
    return int(lib().orc_set_threads(int(n)))


def synthetic_prompt(seed, n, vocab):
    out = np.empty(n, np.int32)
    lib().orc_synthetic_prompt(ctypes.c_uint64(seed), ctypes.c_int64(n), ctypes.c_int64(vocab),
                               out.ctypes.data_as(I32P))
    return out


def tensor_id(slot, kind):
    return slot * 64 + kind


class Model:
    """Synthetic hybrid model held by the oracle."""

    def __init__(self, cfg: dict, seed: int = 0, std: float = 0.02, fp8: bool = False):
        self.cfg = dict(cfg)
        self._c = make_config(cfg)
        self.h = lib().orc_model_create(ctypes.byref(self._c), ctypes.c_uint64(seed), ctypes.c_float(std))
        if fp8 and lib().orc_model_quantize_fp8(self.h) != 0:
            raise RuntimeError("orc_model_quantize_fp8 failed")

    def close(self):
        if self.h:
            lib().orc_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor(self, tid: int) -> np.ndarray:
        n = lib().orc_model_tensor(self.h, ctypes.c_uint32(tid), None, ctypes.c_int64(0))
        if n < 0:
            raise KeyError(tid)
        out = np.empty(n, np.float32)
        lib().orc_model_tensor(self.h, ctypes.c_uint32(tid), _f(out), ctypes.c_int64(n))
        return out

    def set_tensor(self, tid: int, values) -> None:
        v = _c32(np.asarray(values).ravel())
        if lib().orc_model_set_tensor(self.h, ctypes.c_uint32(tid), _f(v), ctypes.c_int64(v.size)) != 0:
            raise KeyError(f"tensor {tid}: unknown id or wrong size {v.size}")

    def mtp_forward(self, ids, hidden):
        """MTP forward over rows (emb(ids[r]), hidden[r]) on a fresh MTP
        cache: returns (out [rows, H], K rows, V rows [rows, nkv, D])."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        hidden = _c32(hidden)
        rows = ids.size
        H, nkv, D = self.cfg["hidden"], self.cfg["num_kv_heads"], self.cfg["head_dim"]
        out = np.empty((rows, H), np.float32)
        k = np.empty((rows, nkv, D), np.float32); v = np.empty_like(k)
        if lib().orc_mtp_forward(self.h, ids.ctypes.data_as(I32P), _f(hidden), ctypes.c_int64(rows), _f(out), _f(k),
                                 _f(v)) != 0:
            raise RuntimeError("orc_mtp_forward failed")
        return out, k, v

    def last_mtp_cache(self):
        """(K, V) rows [len, nkv, D] of the MTP cache the last speculative
        decode left."""
        n = lib().orc_last_mtp_cache(self.h, None, None, ctypes.c_int64(0))
        nkv, D = self.cfg["num_kv_heads"], self.cfg["head_dim"]
        k = np.empty((n, nkv, D), np.float32); v = np.empty_like(k)
        lib().orc_last_mtp_cache(self.h, _f(k), _f(v), ctypes.c_int64(n))
        return k, v

    def forward(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        T = ids.size
        H, V = self.cfg["hidden"], self.cfg["vocab"]
        hid = np.empty((T, H), np.float32); lg = np.empty((T, V), np.float32)
        rc = lib().orc_forward(self.h, ids.ctypes.data_as(I32P), ctypes.c_int64(T), _f(hid), _f(lg))
        if rc != 0:
            raise RuntimeError("orc_forward failed")
        return hid, lg

    def greedy(self, prompt, max_new, eos=()):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        e = np.ascontiguousarray(list(eos), dtype=np.int32)
        out = np.empty(max_new, np.int32)
        n = lib().orc_generate_greedy(self.h, prompt.ctypes.data_as(I32P), ctypes.c_int64(prompt.size),
                                      ctypes.c_int64(max_new), e.ctypes.data_as(I32P), ctypes.c_int64(e.size),
                                      out.ctypes.data_as(I32P))
        if n < 0:
            raise RuntimeError("orc_generate_greedy failed")
        return out[:n]

    def speculative(self, prompt, max_new, width=1, eos=(), draft_override=None, max_rounds=4096):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        e = np.ascontiguousarray(list(eos), dtype=np.int32)
        out = np.empty(max_new, np.int32)
        st = OrcSpecStats()
        log = np.full((max_rounds, ROUND_RECORD), -1, np.int32)
        if draft_override is not None:
            ov = np.ascontiguousarray(draft_override, dtype=np.int32)
            ovp, nov = ov.ctypes.data_as(I32P), ov.size
        else:
            ovp, nov = None, 0
        n = lib().orc_generate_speculative(
            self.h, prompt.ctypes.data_as(I32P), ctypes.c_int64(prompt.size), ctypes.c_int64(max_new),
            ctypes.c_int64(width), e.ctypes.data_as(I32P), ctypes.c_int64(e.size), ovp, ctypes.c_int64(nov),
            out.ctypes.data_as(I32P), ctypes.byref(st), log.ctypes.data_as(I32P), ctypes.c_int64(max_rounds))
        if n < 0:
            raise RuntimeError("orc_generate_speculative failed")
        rounds = st.rounds
        return out[:n], st.as_dict(), log[:rounds]
