"""The C ABI without a GPU: both shared libraries load, export every entry
point that include/*.h declares, and the argument checks that run before any
device call reject bad shapes with HAI_ERR_INVALID_ARGUMENT."""
import ctypes
import re

import pytest

from _hai import ROOT, hai

HEADERS = sorted((ROOT / "include").glob("*.h"))
DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(hai_[a-z0-9_]+)\s*\(", re.M)


def declared(header):
    return sorted(set(DECL.findall(header.read_text())))


def test_headers_declare_entry_points():
    names = {h.name: declared(h) for h in HEADERS}
    assert names["hai_kernels.h"] and names["hai_engine.h"]


@pytest.mark.parametrize("header", HEADERS, ids=lambda p: p.name)
def test_every_declared_symbol_is_exported(header):
    libs = [ctypes.CDLL(str(hai.KERNELS_SO)), ctypes.CDLL(str(hai.HOST_SO))]
    missing = [n for n in declared(header) if not any(hasattr(lib, n) for lib in libs)]
    assert not missing, f"{header.name}: not exported by the built libraries: {missing}"


def test_kernel_signatures_cover_the_header():
    """Every kernels-header entry point has a ctypes signature in the package."""
    sigs = set(hai._KERNEL_SIGS) | set(hai._SIZE_SIGS) | {"hai_last_error"}
    missing = [n for n in declared(ROOT / "include" / "hai_kernels.h") if n not in sigs]
    assert not missing, missing


def test_argument_checks_need_no_device():
    k = hai.kernels()
    p = ctypes.c_void_p(16)  # never dereferenced: every call below fails its host-side checks
    assert k.hai_gemm_bf16(p, 4, p, 12, p, 2, 4, 12, 0, None, 0, None) == hai.ERR_INVALID  # K % 8
    assert k.hai_gemm_bf16(p, 4, p, 8, p, -1, 4, 8, 0, None, 0, None) == hai.ERR_INVALID   # M < 0
    assert k.hai_gemm_rmsnorm_bf16(p, 8, p, 8, p, 1e-6, 1, None, 0, p, 17, 8, 8, 0, None, 0,
                                   None) == hai.ERR_INVALID  # more than 16 rows without xn_out
    assert k.hai_gemm_bf16(None, 4, p, 8, p, 1, 4, 8, 0, None, 0, None) == hai.ERR_INVALID
    assert k.hai_gemm_rmsnorm_bf16(p, 8, p, 5120, p, 1e-6, 1, None, 0, p, 4, 8, 5120, 0, None, 0,
                                   None) == hai.ERR_INVALID  # above the fused limit without xn_out
    assert k.hai_deltanet_verify_bf16(p, 8, p, 8, 0, 0, 0, 0, p, p, 4, p, 1, 1, p, p, p, None, 0, 1, 17, 1, 1,
                                      128, 128, 4, 1e-6, None) == hai.ERR_INVALID  # T > 16
    assert k.hai_gqa_verify_bf16(p, p, p, p, p, 8, p, 1, 4, 4, 3, 64, None, 4, 8, None) == hai.ERR_INVALID
    assert b"gqa_verify" in k.hai_last_error()
    # the prefill's conv reads channel pairs as dwords: proj and the ring 4-byte aligned, ld_proj and
    # off_qkv even (B = 1, T = 4, one 128 x 128 head, 4 taps; the workspace size is checked after)
    def prefill(proj, ld_proj, off_qkv, ring_ptr):
        return k.hai_deltanet_prefill_bf16(p, 128, proj, ld_proj, off_qkv, 384, 512, 513, p, ring_ptr, 4, p, 1, p,
                                           p, p, None, 0, 1, 4, 1, 1, 128, 128, 4, 1e-6, p, 1 << 30, None)
    for args in ((ctypes.c_void_p(18), 514, 0, p), (p, 515, 0, p), (p, 514, 1, p), (p, 514, 0, ctypes.c_void_p(18))):
        assert prefill(*args) == hai.ERR_INVALID
        assert b"4-byte aligned" in k.hai_last_error(), k.hai_last_error()


def test_deltanet_records_checks_need_no_device():
    """hai_deltanet_verify_rec_bf16 rejects, before any device call: no
    records or base buffer, unaligned records, nslots <= T (the final state
    would overwrite the replay's start slot), replay outside {0, 1} and a
    replay call of more than 4 tokens; the records size is
    nslots x B x nv x (dk + dv + 4) floats, SIZE_MAX on overflow."""
    k = hai.kernels()
    p = ctypes.c_void_p(16)  # never dereferenced
    assert k.hai_deltanet_records_bytes(5, 2, 48, 128, 128) == 5 * 2 * 48 * 260 * 4
    assert k.hai_deltanet_records_bytes(1 << 40, 1 << 40, 48, 128, 128) == 2 ** 64 - 1

    def call(records, base, replay, T, nslots):
        return k.hai_deltanet_verify_rec_bf16(p, 512, p, 1280, 0, 768, 1024, 1028, None, 0, None, 0, p, p, 8, p,
                                              nslots, records, base, replay, p, p, p, p, 0, 1, T, 2, 4, 64, 64, 4,
                                              1e-6, None)
    for args, what in (((None, p, 0, 2, 5), b"null records"), ((p, None, 0, 2, 5), b"null base"),
                       ((ctypes.c_void_p(24), p, 0, 2, 5), b"records alignment"),
                       ((p, p, 0, 5, 5), b"nslots > T"), ((p, p, 2, 2, 5), b"replay must be"),
                       ((p, p, 1, 5, 8), b"at most 4 tokens")):
        assert call(*args) == hai.ERR_INVALID, what
        assert what in k.hai_last_error(), (what, k.hai_last_error())


def test_noalloc_attention_bounds_its_shape_before_sizing():
    """hai_gqa_verify_noalloc_bf16 checks every operand of the scratch size
    before computing it: a batch past int32, a bad head_dim or nkv, or a
    size above the fixed 16 MiB array is refused on the host, before the
    device array is looked up; the size function reports overflow as
    SIZE_MAX instead of wrapping."""
    k = hai.kernels()
    p = ctypes.c_void_p(16)  # never dereferenced
    big = 1 << 40
    for B, nkv, D, what in ((big, 4, 256, b"shape"), (1, 0, 256, b"shape"), (1, 4, 100, b"head_dim"),
                            (100000, 4, 256, b"16 MiB")):
        assert k.hai_gqa_verify_noalloc_bf16(p, p, p, p, p, 4096, B, 2, 24, nkv, D, None, 2, 4096,
                                             None) == hai.ERR_INVALID, (B, nkv, D)
        assert what in k.hai_last_error(), k.hai_last_error()
    assert k.hai_gqa_scratch_bytes(big, big, 24, 256, 4096) == 2 ** 64 - 1
    # 2 rows x 24 heads x 64 chunks of 64 keys x (256 + 2) floats
    assert k.hai_gqa_scratch_bytes(1, 2, 24, 256, 4096) == 2 * 24 * 64 * 258 * 4


def test_fused_attention_checks_need_no_device():
    """hai_gqa_verify_fused_bf16 rejects on the host, before any device
    call: a null operand, projection rows narrower than [q+gate | k | v],
    an odd rotary width or one wider than the head, no rotation table, a
    cache window past the capacity, a host-side length that does not cover
    the T new rows, unaligned caches or projection rows, and a head_dim
    other than 64, 128 or 256."""
    k = hai.kernels()
    p = ctypes.c_void_p(16)  # never dereferenced

    def call(proj=p, ld=14336, R=64, rope_pos=4096, kc=p, max_len=4096, len_add=2, D=256):
        return k.hai_gqa_verify_fused_bf16(p, p, proj, ld, p, p, p, p, rope_pos, R, 1e-6, kc, p, 4096, p, 1, 2,
                                           24, 4, D, None, len_add, max_len, None)
    for kw, what in (({"proj": None}, b"null pointer"), ({"ld": 14335}, b"shape"), ({"R": 63}, b"shape"),
                     ({"R": 512}, b"shape"), ({"rope_pos": 0}, b"shape"), ({"max_len": 5000}, b"shape"),
                     ({"len_add": 1}, b"cache length"), ({"kc": ctypes.c_void_p(24)}, b"alignment"),
                     ({"ld": 14340}, b"alignment"), ({"D": 100, "ld": 5600}, b"head_dim")):
        assert call(**kw) == hai.ERR_INVALID, kw
        assert what in k.hai_last_error(), (kw, k.hai_last_error())
