"""vicold.hybridai_amd -- MI355X-native MTP speculative verify path.

Python access to the two in-tree libraries through their C ABIs:
  * libhai_kernels.so  gfx950 kernels + runtime wrappers (include/hai_kernels.h)
  * libhybridai.so     C++ host: verify engine, Backend, Generator
                       (include/hai_engine.h)

The directory name contains a dot, so load it with load_package() from
__graft_entry__ / tests rather than a plain import.  There is no CPU fallback:
every compute call goes to the HIP library and fails loudly when it is missing.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
LIB_DIR = PKG_DIR / "lib"
KERNELS_SO = LIB_DIR / "libhai_kernels.so"
HOST_SO = LIB_DIR / "libhybridai.so"

VP = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int32
F32 = ctypes.c_float
I32P = ctypes.POINTER(ctypes.c_int32)
I64P = ctypes.POINTER(ctypes.c_int64)
F32P = ctypes.POINTER(ctypes.c_float)

EPI_STORE, EPI_RESIDUAL, EPI_SILU_MUL = 0, 1, 2
FP8_NO_SPECIAL_CODES = 0x100  # hai_gemm_fp8_bf16 epilogue flag: weights hold no 0x7F / 0xFF code
MFMA_KEEP_PARTIALS = 0x200  # MFMA GEMM residual epilogue flag: leave the K-split partials
# hai_status codes (include/hai_kernels.h)
OK, ERR_INVALID, ERR_OOM, ERR_NOT_IMPLEMENTED, ERR_INVALID_DEVICE, ERR_BACKEND = 0, 1, 2, 3, 5, 9

# name -> argtypes (restype int unless noted)
_KERNEL_SIGS = {
    "hai_device_count": [I32P],
    "hai_set_device": [ctypes.c_int],
    "hai_get_device": [I32P],
    "hai_malloc": [ctypes.POINTER(VP), ctypes.c_size_t],
    "hai_free": [VP],
    "hai_memcpy_h2d": [VP, VP, ctypes.c_size_t, VP],
    "hai_memcpy_d2h": [VP, VP, ctypes.c_size_t, VP],
    "hai_memcpy_d2d": [VP, VP, ctypes.c_size_t, VP],
    "hai_memcpy_h2d_2d": [VP, ctypes.c_size_t, VP, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, VP],
    "hai_memset": [VP, ctypes.c_int, ctypes.c_size_t, VP],
    "hai_memcpy": [VP, VP, ctypes.c_size_t, VP],
    "hai_host_malloc": [ctypes.POINTER(VP), ctypes.c_size_t],
    "hai_host_free": [VP],
    "hai_stream_wait_event": [VP, VP],
    "hai_stream_create": [ctypes.POINTER(VP)],
    "hai_stream_destroy": [VP],
    "hai_stream_synchronize": [VP],
    "hai_device_synchronize": [],
    "hai_event_create": [ctypes.POINTER(VP)],
    "hai_event_destroy": [VP],
    "hai_event_record": [VP, VP],
    "hai_event_synchronize": [VP],
    "hai_event_elapsed_ms": [VP, VP, F32P],
    "hai_graph_begin_capture": [VP],
    "hai_graph_end_capture": [VP, ctypes.POINTER(VP)],
    "hai_graph_launch": [VP, VP],
    "hai_graph_destroy": [VP],
    "hai_gemm_bf16": [VP, I64, VP, I64, VP, I64, I64, I64, ctypes.c_int, VP, I64, VP],
    "hai_gemm_rmsnorm_bf16": [VP, I64, VP, I64, VP, F32, ctypes.c_int, VP, I64, VP, I64, I64, I64, ctypes.c_int,
                              VP, I64, VP],
    "hai_gemm_fp8_bf16": [VP, I64, VP, I64, VP, VP, VP, I64, I64, I64, ctypes.c_int, VP, I64, VP],
    "hai_gemm_rmsnorm_fp8_bf16": [VP, I64, VP, I64, VP, F32, ctypes.c_int, VP, I64, VP, VP, VP, I64, I64, I64,
                                  ctypes.c_int, VP, I64, VP],
    "hai_fp8_quantize_bf16": [VP, I64, VP, I64, VP, I64, I64, VP],
    "hai_fill_synthetic_scales_f32": [VP, I64, ctypes.c_uint64, ctypes.c_uint32, VP],
    "hai_rmsnorm_bf16": [VP, I64, VP, I64, VP, I64, I64, F32, ctypes.c_int, VP],
    "hai_add_bf16": [VP, VP, VP, I64, VP],
    "hai_silu_mul_bf16": [VP, VP, VP, I64, VP],
    "hai_embedding_gather_bf16": [VP, VP, VP, I64, I64, I64, VP],
    "hai_q_gate_rmsnorm_rope_bf16": [VP, VP, VP, I64, VP, VP, VP, I64, I64, I64, I64, I64, I64, VP, I32, F32,
                                     VP],
    "hai_kv_rmsnorm_rope_append_bf16": [VP, VP, I64, VP, VP, I64, VP, VP, VP, I64, I64, I64, I64, I64, I64, VP,
                                        I32, F32, VP],
    "hai_append_kv_bf16": [VP, VP, I64, VP, VP, I64, I64, I64, VP, I32, VP],
    "hai_partial_rope_bf16": [VP, VP, I64, I64, I64, I64, VP, VP, I64, I64, VP],
    "hai_deltanet_conv_bf16": [VP, VP, VP, VP, VP, VP, I64, I64, I64, I64, I64, I64, VP],
    "hai_deltanet_recurrent_bf16": [VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, I64, I64, I64, I64, I64, F32, VP],
    "hai_qkv_rmsnorm_rope_append_bf16": [VP, VP, VP, VP, I64, VP, I64, VP, VP, VP, VP, I64, I64, I64, I64, I64, I64,
                                         I64, VP, I32, F32, VP],
    "hai_gqa_verify_bf16": [VP, VP, VP, VP, VP, I64, VP, I64, I64, I64, I64, I64, VP, I32, I64, VP],
    "hai_gqa_verify_fused_bf16": [VP, VP, VP, I64, VP, VP, VP, VP, I64, I64, F32, VP, VP, I64, VP, I64, I64, I64, I64,
                                  I64, VP, I32, I64, VP],
    "hai_gqa_verify_mfma_bf16": [VP, VP, VP, VP, VP, I64, VP, I64, I64, I64, I64, I64, VP, I32, I64, VP],
    "hai_gqa_verify_noalloc_bf16": [VP, VP, VP, VP, VP, I64, I64, I64, I64, I64, I64, VP, I32, I64, VP],
    "hai_deltanet_verify_bf16": [VP, I64, VP, I64, I64, I64, I64, I64, VP, VP, I64, VP, I64, ctypes.c_int, VP, VP,
                                 VP, VP, I32, I64, I64, I64, I64, I64, I64, I64, F32, VP],
    "hai_deltanet_verify_ws_bf16": [VP, I64, VP, I64, I64, I64, I64, I64, VP, VP, I64, VP, I64, ctypes.c_int, VP,
                                    VP, VP, VP, I32, I64, I64, I64, I64, I64, I64, I64, F32, VP, I64, VP],
    "hai_deltanet_verify_ab_bf16": [VP, I64, VP, I64, I64, I64, VP, I64, VP, I64, VP, VP, I64, VP, I64, ctypes.c_int,
                                    VP, VP, VP, VP, I32, I64, I64, I64, I64, I64, I64, I64, F32, VP],
    "hai_deltanet_verify_rec_bf16": [VP, I64, VP, I64, I64, I64, I64, I64, VP, I64, VP, I64, VP, VP, I64, VP, I64, VP,
                                     VP, ctypes.c_int, VP, VP, VP, VP, I32, I64, I64, I64, I64, I64, I64, I64, F32, VP],
    "hai_deltanet_prefill_bf16": [VP, I64, VP, I64, I64, I64, I64, I64, VP, VP, I64, VP, I64, VP, VP, VP, VP, I32,
                                  I64, I64, I64, I64, I64, I64, I64, F32, VP, I64, VP],
    "hai_argmax_rows_bf16": [VP, VP, I64, I64, I64, VP, VP],
    "hai_verify_argmax_accept_bf16": [VP, I64, VP, I64, VP, VP, I64, I64, VP, VP, VP, VP, VP, VP, VP, VP, VP],
    "hai_add_i32": [VP, VP, I32, I64, VP],
    "hai_draft_chain_count": [I64, VP, I64, VP, VP, I64, VP, I64, VP],
    "hai_copy_i64_strided": [VP, I64, VP, I64, I64, VP],
    "hai_correction_commit_bf16": [VP, VP, VP, I64, I64, VP, VP, VP, VP, VP],
    "hai_gemm_bf16_mfma": [VP, I64, VP, I64, VP, I64, I64, I64, ctypes.c_int, VP, I64, VP, ctypes.c_size_t, VP],
    "hai_gemm_bf16_tiled": [VP, I64, VP, I64, VP, I64, I64, I64, ctypes.c_int, VP, I64, VP],
    "hai_gemm_fp8_tiled": [VP, I64, VP, I64, VP, VP, VP, I64, I64, I64, ctypes.c_int, VP, I64, VP],
    "hai_gemm_fp8_mfma": [VP, I64, VP, I64, VP, VP, VP, I64, I64, I64, ctypes.c_int, VP, I64, VP, ctypes.c_size_t,
                          VP],
    "hai_gemm_mfma_splits": [I64, I64, I64, VP, ctypes.c_size_t],
    "hai_mfma_residual_rmsnorm_bf16": [VP, I64, VP, ctypes.c_size_t, I64, I64, I64, VP, F32, ctypes.c_int, VP, I64,
                                       VP],
    "hai_fill_synthetic_bf16": [VP, I64, I64, I64, ctypes.c_uint64, ctypes.c_uint32, F32, VP],
    "hai_debug_math_f32": [VP, VP, I64, ctypes.c_int, VP],
    "hai_debug_check_extent": [VP, ctypes.c_size_t],
}
_SIZE_SIGS = {
    "hai_gemm_mfma_workspace_bytes": [I64, I64],
    "hai_gqa_scratch_bytes": [I64, I64, I64, I64, I64],
    "hai_gqa_mfma_scratch_bytes": [I64, I64, I64, I64, I64],
    "hai_gqa_mfma_plan_scratch_bytes": [I64, I64, I64, I64, I64, I64],
    "hai_argmax_scratch_bytes": [I64, I64],
    "hai_deltanet_workspace_bytes": [I64, I64, I64],
    "hai_deltanet_prefill_workspace_bytes": [I64, I64, I64, I64],
    "hai_deltanet_records_bytes": [I64, I64, I64, I64, I64],
}

_kern = None


class HaiError(RuntimeError):
    pass


def _check_fresh(so: Path) -> None:
    """Refuses a library whose sources changed after it was built: build.py
    records a digest of the sources of each library, recomputed here from the
    tree, so a stale .so can never run silently against newer sources."""
    import importlib.util
    import json
    manifest = LIB_DIR / "build_manifest.json"
    if not manifest.exists():
        raise HaiError(f"{manifest} is missing: run __graft_entry__.build()")
    spec = importlib.util.spec_from_file_location("_hai_build", PKG_DIR / "build.py")
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    inputs = build.kernel_inputs() if so.name == KERNELS_SO.name else build.host_inputs()
    recorded = json.loads(manifest.read_text()).get(so.name)
    if recorded != build.source_digest(inputs):
        raise HaiError(f"{so.name} is older than its sources: run __graft_entry__.build()")


def kernels() -> ctypes.CDLL:
    """Load libhai_kernels.so (raises when it has not been built or is
    older than its sources)."""
    global _kern
    if _kern is None:
        if not KERNELS_SO.exists():
            raise HaiError(f"{KERNELS_SO} is missing: run __graft_entry__.build()")
        _check_fresh(KERNELS_SO)
        lib = ctypes.CDLL(str(KERNELS_SO))
        for name, args in _KERNEL_SIGS.items():
            f = getattr(lib, name)
            f.argtypes = args
            f.restype = ctypes.c_int
        for name, args in _SIZE_SIGS.items():
            f = getattr(lib, name)
            f.argtypes = args
            f.restype = ctypes.c_size_t
        lib.hai_last_error.restype = ctypes.c_char_p
        lib.hai_last_error.argtypes = []
        _kern = lib
    return _kern


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = kernels().hai_last_error().decode(errors="replace")
        raise HaiError(f"{what} failed ({rc}): {msg}")


def device_count() -> int:
    n = ctypes.c_int32(0)
    rc = kernels().hai_device_count(ctypes.byref(n))
    return int(n.value) if rc == 0 else 0


def synchronize() -> None:
    check(kernels().hai_device_synchronize(), "hai_device_synchronize")


class DeviceBuffer:
    """A raw device allocation owned by Python (freed on close/GC)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = VP()
        check(kernels().hai_malloc(ctypes.byref(p), ctypes.c_size_t(max(self.nbytes, 1))), "hai_malloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(kernels().hai_memcpy_h2d(self.ptr, a.ctypes.data, ctypes.c_size_t(a.nbytes), None), "h2d")
        synchronize()

    def download(self, dtype, count=None) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else int(count)
        out = np.empty(n, dtype)
        synchronize()
        check(kernels().hai_memcpy_d2h(out.ctypes.data, self.ptr, ctypes.c_size_t(out.nbytes), None), "d2h")
        synchronize()
        return out

    def zero(self) -> None:
        check(kernels().hai_memset(self.ptr, 0, ctypes.c_size_t(self.nbytes), None), "memset")

    def close(self) -> None:
        if getattr(self, "ptr", None):
            kernels().hai_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __int__(self):
        return int(self.ptr)


def bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r[nan] = ((u[nan] >> 16) | np.uint32(0x40)).astype(np.uint16)
    return r


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------------ host library
_host = None


def host() -> ctypes.CDLL:
    """Load libhybridai.so (the C++ engine); raises when missing."""
    global _host
    if _host is None:
        kernels()
        if not HOST_SO.exists():
            raise HaiError(f"{HOST_SO} is missing: run __graft_entry__.build()")
        _check_fresh(HOST_SO)
        from . import engine as _engine  # noqa: F401  (sets signatures)
        _host = _engine.bind(ctypes.CDLL(str(HOST_SO)))
    return _host
