"""Kernel-level parity: every hai_* entry point against the CPU oracle on the
same seeded inputs, bit-exact on the bf16 outputs (the oracle follows the
same canonical reduction order, see oracle/oracle_numerics.h)."""
import ctypes

import numpy as np
import pytest

from _hai import assert_bits_equal, hai, orc, rand_bf16

pytestmark = pytest.mark.gpu
K = None


def kern():
    global K
    if K is None:
        K = hai.kernels()
    return K


def dev(a):
    return hai.DeviceBuffer.from_array(np.ascontiguousarray(a))


def out_buf(nbytes):
    b = hai.DeviceBuffer(nbytes)
    b.zero()
    return b


# ----------------------------------------------------------------- primitives
def _special_inputs(rng):
    xs = [rng.standard_normal(200000).astype(np.float32) * s for s in (0.1, 1.0, 5.0, 30.0, 100.0)]
    xs.append(np.array([0.0, -0.0, 1e-45, -1e-45, 1e-38, 88.7, 88.72, 88.73, -87.3, -103.9, -104.0,
                        -110.0, 1e30, -1e30, np.inf, -np.inf, np.nan, 0.5, -0.5, 1.0, -1.0, 2.0,
                        0.693147, -0.693147, 1e-7, -1e-7], np.float32))
    return np.concatenate(xs)


@pytest.mark.parametrize("fn,name", [(0, "exp"), (1, "log1p"), (2, "sigmoid"), (3, "silu"), (4, "sqrt"),
                                     (5, "recip"), (6, "bf16")])
def test_primitives_bit_exact(fn, name):
    rng = np.random.default_rng(100 + fn)
    x = _special_inputs(rng)
    if name == "log1p":
        x = np.concatenate([np.abs(x) % 1.0, x[x > -1.0], rng.uniform(-0.999, 1.0, 100000).astype(np.float32)])
    if name == "sqrt":
        x = np.abs(x)
    x = x.astype(np.float32)
    dx, dy = dev(x), out_buf(x.nbytes)
    hai.check(kern().hai_debug_math_f32(dy.ptr, dx.ptr, x.size, fn, None), "debug_math")
    got = dy.download(np.float32)
    if name == "exp":
        want = orc.cexp(x)
    elif name == "log1p":
        want = orc.clog1p(x)
    elif name == "sigmoid":
        want = (np.float32(1.0) / (np.float32(1.0) + orc.cexp(-x))).astype(np.float32)
    elif name == "silu":
        want = (x / (np.float32(1.0) + orc.cexp(-x))).astype(np.float32)
    elif name == "sqrt":
        want = np.sqrt(x)
    elif name == "recip":
        with np.errstate(divide="ignore"):
            want = (np.float32(1.0) / x).astype(np.float32)
    else:
        want = orc.round_bf16(x)
    gb, wb = got.view(np.uint32), want.view(np.uint32)
    nan_ok = np.isnan(got) & np.isnan(want)
    bad = np.nonzero((gb != wb) & ~nan_ok)[0]
    assert bad.size == 0, f"{name}: {bad.size} mismatches, e.g. x={x[bad[:5]]} got={got[bad[:5]]} want={want[bad[:5]]}"


def test_bf16_rounding_bits_with_nans():
    """The device's f32 -> bf16 rounding (gfx950 v_cvt_pk_bf16_f32 in every
    kernel) equals the oracle's integer round-to-nearest-even bit for bit,
    NaNs included (sign and upper payload kept, quiet bit set): NaN classes,
    exact ties to even and odd, denormals, values that round up to inf."""
    rng = np.random.default_rng(77)
    pats = []
    for s in (0, 0x80000000):
        for m in (1, 0x10000, 0x8000, 0x18000, 0x3FFFFF, 0x400000, 0x7FFFFF, 0x1FFFF, 0x55AA55):
            pats.append(s | 0x7F800000 | m)                       # NaNs, signalling and quiet
        for x in (0x7F800000, 0, 1, 0x7FFF, 0x8000, 0x18000, 0x10000, 0x7F7FFFFF, 0x7F7F8000,
                  0x7F7F7FFF, 0x3F808000, 0x3F818000, 0x3F80FFFF, 0x007FFFFF, 0x00008000, 0x00018000):
            pats.append(s | x)                                    # inf, ties, denormals, overflow
    pats = np.array(pats, np.uint32)
    rand = rng.integers(0, 1 << 32, 1 << 18, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([pats, rand]).view(np.float32)
    dx, dy = dev(x), out_buf(x.nbytes)
    hai.check(kern().hai_debug_math_f32(dy.ptr, dx.ptr, x.size, 6, None), "debug_math bf16")
    got = dy.download(np.uint32)
    want = orc.round_bf16(x).view(np.uint32)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (f"{bad.size} mismatches, e.g. x={x.view(np.uint32)[bad[:4]]} got={got[bad[:4]]} "
                           f"want={want[bad[:4]]}")


# ----------------------------------------------------------------- gemm
@pytest.mark.parametrize("M,N,K_", [(1, 37, 8), (2, 256, 256), (2, 1536, 256), (3, 4096, 256),
                                    (4, 100, 1000), (7, 64, 520), (16, 512, 768), (2, 5120, 17408),
                                    (1, 16480, 5120), (2, 9, 1024), (2, 1030, 2056), (2, 8192, 20480)])
def test_gemm_store(M, N, K_):
    rng = np.random.default_rng(M * 1000 + N + K_)
    x, xb = rand_bf16(rng, (M, K_))
    w, wb = rand_bf16(rng, (N, K_), 0.05)
    dx, dw, dy = dev(xb), dev(wb), out_buf(M * N * 2)
    hai.check(kern().hai_gemm_bf16(dy.ptr, N, dx.ptr, K_, dw.ptr, M, N, K_, hai.EPI_STORE, None, 0, None), "gemm")
    assert_bits_equal(dy.download(np.uint16), orc.gemm(x, w), f"gemm {M}x{N}x{K_}")


@pytest.mark.parametrize("M,N,K_", [(2, 256, 256), (4, 5120, 6144), (16, 300, 512), (1, 5120, 6144),
                                    (2, 5120, 17408), (1, 77, 9000), (2, 130, 8192), (2, 2050, 8200),
                                    (2, 1031, 6152)])
def test_gemm_residual(M, N, K_):
    rng = np.random.default_rng(7 + M + N)
    x, xb = rand_bf16(rng, (M, K_))
    w, wb = rand_bf16(rng, (N, K_), 0.05)
    h, hb = rand_bf16(rng, (M, N))
    dx, dw, dh = dev(xb), dev(wb), dev(hb)
    hai.check(kern().hai_gemm_bf16(dh.ptr, N, dx.ptr, K_, dw.ptr, M, N, K_, hai.EPI_RESIDUAL, dh.ptr, N, None),
              "gemm residual")
    want = orc.add(h, orc.gemm(x, w))
    assert_bits_equal(dh.download(np.uint16), want, "gemm residual")


def test_gemm_two_rows_with_row_pitch():
    """Two-row residual launch of the short layers (activation rows staged
    in LDS) with row pitches above the row lengths: x rows K + 24 apart,
    h rows N + 40 apart, only the first N columns of h touched."""
    M, N, K_, ldx, ldh = 2, 3000, 6144, 6168, 3040
    rng = np.random.default_rng(11)
    xp, xpb = rand_bf16(rng, (M, ldx))
    w, wb = rand_bf16(rng, (N, K_), 0.05)
    hp, hpb = rand_bf16(rng, (M, ldh))
    dx, dw, dh = dev(xpb), dev(wb), dev(hpb)
    hai.check(kern().hai_gemm_bf16(dh.ptr, ldh, dx.ptr, ldx, dw.ptr, M, N, K_, hai.EPI_RESIDUAL, dh.ptr, ldh, None),
              "gemm residual with pitch")
    got = dh.download(np.uint16).reshape(M, ldh)
    want = orc.add(hp[:, :N], orc.gemm(xp[:, :K_], w))
    assert_bits_equal(got[:, :N], want, "gemm residual with pitch")
    assert np.array_equal(got[:, N:], hpb.reshape(M, ldh)[:, N:])


@pytest.mark.parametrize("M,F,K_", [(2, 768, 256), (1, 17408, 5120), (5, 96, 512), (1, 2000, 9000), (2, 300, 8192)])
def test_gemm_silu_mul(M, F, K_):
    rng = np.random.default_rng(11 + M + F)
    x, xb = rand_bf16(rng, (M, K_))
    g, gb = rand_bf16(rng, (F, K_), 0.05)
    u, ub = rand_bf16(rng, (F, K_), 0.05)
    wb = np.empty((2 * F, K_), np.uint16)
    wb[0::2] = gb
    wb[1::2] = ub
    dx, dw, dy = dev(xb), dev(wb), out_buf(M * F * 2)
    hai.check(kern().hai_gemm_bf16(dy.ptr, F, dx.ptr, K_, dw.ptr, M, 2 * F, K_, hai.EPI_SILU_MUL, None, 0, None),
              "gemm silu")
    want = orc.silu_mul(orc.gemm(x, g), orc.gemm(x, u))
    assert_bits_equal(dy.download(np.uint16), want, "gemm silu_mul")


def test_gemm_rejects_bad_shapes():
    d = out_buf(64)
    assert kern().hai_gemm_bf16(d.ptr, 4, d.ptr, 12, d.ptr, 2, 4, 12, 0, None, 0, None) == 1  # K % 8
    assert kern().hai_gemm_bf16(d.ptr, 4, d.ptr, 4, d.ptr, 2, 4, 8, 0, None, 0, None) == 1    # ldx < K
    assert kern().hai_gemm_bf16(d.ptr, 4, d.ptr, 8, d.ptr, -1, 4, 8, 0, None, 0, None) == 1   # M < 0
    # a fused-norm launch of more than 16 rows needs xn_out for the two-kernel form
    assert kern().hai_gemm_rmsnorm_bf16(d.ptr, 4, d.ptr, 8, d.ptr, 1e-6, 1, None, 0, d.ptr, 17, 4, 8, 0,
                                        None, 0, None) == 1


@pytest.mark.parametrize("M,N,K_,epi,ldx", [(17, 300, 256, 0, 256), (37, 1000, 520, 1, 528), (300, 77, 8, 0, 8),
                                            (100, 1200, 1024, 2, 1024), (512, 1536, 2048, 0, 2048),
                                            (64, 8200, 1024, 1, 1040), (40, 5120, 17408, 1, 17408)])
def test_gemm_row_batches(M, N, K_, epi, ldx):
    """Launches of more than 16 rows (prompt-sized M through Backend::gemm,
    hip_backend.cc:697-809): one launch whose blocks each take a weight row
    group and a 16-row batch, ragged last batch and row pitches included;
    every row bit-identical to the oracle's canonical-order sum."""
    rng = np.random.default_rng(M * 7 + N + K_)
    xp, xpb = rand_bf16(rng, (M, ldx))
    x = xp[:, :K_]
    if epi == hai.EPI_SILU_MUL:
        F = N // 2
        g, gb = rand_bf16(rng, (F, K_), 0.05)
        u, ub = rand_bf16(rng, (F, K_), 0.05)
        wb = np.empty((N, K_), np.uint16)
        wb[0::2], wb[1::2] = gb, ub
        want = orc.silu_mul(orc.gemm(x, g), orc.gemm(x, u))
        ncols = F
    else:
        w, wb = rand_bf16(rng, (N, K_), 0.05)
        want = orc.gemm(x, w)
        ncols = N
    h, hb = rand_bf16(rng, (M, ncols))
    if epi == hai.EPI_RESIDUAL:
        want = orc.add(h, want)
    dx, dw, dy = dev(xpb), dev(wb), dev(hb)
    res = dy.ptr if epi == hai.EPI_RESIDUAL else None
    hai.check(kern().hai_gemm_bf16(dy.ptr, ncols, dx.ptr, ldx, dw.ptr, M, N, K_, epi, res, ncols, None),
              "gemm row batches")
    assert_bits_equal(dy.download(np.uint16), want, f"gemm {M}x{N}x{K_} epi {epi}")


def test_gemm_rmsnorm_row_batches():
    """The fused-norm entry with more than 16 rows: the norm into xn_out,
    then one batched launch, bit-identical to rmsnorm then gemm."""
    M, N, K_ = 48, 640, 1024
    rng = np.random.default_rng(5)
    x, xb = rand_bf16(rng, (M, K_))
    nw, nwb = rand_bf16(rng, (K_,), 0.02)
    w, wb = rand_bf16(rng, (N, K_), 0.05)
    dx, dn, dw, dy, dxn = dev(xb), dev(nwb), dev(wb), out_buf(M * N * 2), out_buf(M * K_ * 2)
    hai.check(kern().hai_gemm_rmsnorm_bf16(dy.ptr, N, dx.ptr, K_, dn.ptr, 1e-6, 1, dxn.ptr, K_, dw.ptr, M, N, K_,
                                           hai.EPI_STORE, None, 0, None), "gemm_rmsnorm 48 rows")
    xn = orc.rmsnorm(x, nw, 1e-6, True)
    assert_bits_equal(dxn.download(np.uint16), xn, "xn")
    assert_bits_equal(dy.download(np.uint16), orc.gemm(xn, w), "gemm after norm")


@pytest.mark.parametrize("M,N,K_,epi", [(1, 4096, 256, 0), (2, 16480, 5120, 0), (2, 17408, 5120, 2),
                                        (3, 520, 5120, 1), (16, 300, 1024, 0), (2, 77, 1000, 0),
                                        (4, 64, 5120, 0), (8, 512, 2048, 2), (2, 1030, 5120, 1)])
@pytest.mark.parametrize("with_xn", [False, True])
def test_gemm_rmsnorm_fused(M, N, K_, epi, with_xn):
    """hai_gemm_rmsnorm_bf16 == rmsnorm then gemm, on both sides of the fused
    limit (M*K <= 16384 runs the LDS prologue, above it the two kernels)."""
    rng = np.random.default_rng(31 + M * 7 + N + K_ + epi)
    x, xb = rand_bf16(rng, (M, K_))
    nw, nwb = rand_bf16(rng, (K_,), 0.02)
    w, wb = rand_bf16(rng, (N, K_), 0.05)
    xn_want = orc.rmsnorm(x, nw, 1e-6, True)
    y_lin = orc.gemm(xn_want, w)
    ncols = N // 2 if epi == hai.EPI_SILU_MUL else N
    need_xn = with_xn or M * K_ > 16384
    dx, dnw, dw = dev(xb), dev(nwb), dev(wb)
    dxn = out_buf(M * K_ * 2) if need_xn else None
    h, hb = rand_bf16(rng, (M, ncols))
    dy = dev(hb) if epi == hai.EPI_RESIDUAL else out_buf(M * ncols * 2)
    hai.check(kern().hai_gemm_rmsnorm_bf16(dy.ptr, ncols, dx.ptr, K_, dnw.ptr, 1e-6, 1,
                                           dxn.ptr if dxn else None, K_, dw.ptr, M, N, K_, epi,
                                           dy.ptr if epi == hai.EPI_RESIDUAL else None, ncols, None),
              "gemm_rmsnorm")
    if epi == hai.EPI_STORE:
        want = y_lin
    elif epi == hai.EPI_RESIDUAL:
        want = orc.add(h, y_lin)
    else:
        want = orc.silu_mul(y_lin[:, 0::2], y_lin[:, 1::2])
    assert_bits_equal(dy.download(np.uint16), want, f"gemm_rmsnorm {M}x{N}x{K_} epi {epi}")
    if dxn is not None:
        assert_bits_equal(dxn.download(np.uint16), xn_want, "normalised rows")


# The C3 verify step's weight streams at M = 2 rows, called as the engine
# calls them (fused input RMSNorm on in_proj / qkv / gate-up, residual on the
# out / o / down projections, lm_head after a separate norm); bit-exact.  Also
# the workload of the rocprofv3 FETCH_SIZE / WRITE_SIZE passes that give the
# HBM traffic per launch.
C3_VERIFY_GEMMS = [("deltanet_in_proj", 16480, 5120, 0, True), ("out_proj", 5120, 6144, 1, False),
                   ("gate_up", 34816, 5120, 2, True), ("down", 5120, 17408, 1, False),
                   ("attn_qkv", 14336, 5120, 0, True), ("lm_head", 248320, 5120, 0, False)]


@pytest.mark.parametrize("name,N,K_,epi,norm", C3_VERIFY_GEMMS)
def test_gemm_c3_verify_shapes(name, N, K_, epi, norm):
    M = 2
    rng = np.random.default_rng(N + K_ + epi)
    x, xb = rand_bf16(rng, (M, K_))
    w, wb = rand_bf16(rng, (N, K_), 0.02)
    ncols = N // 2 if epi == hai.EPI_SILU_MUL else N
    h, hb = rand_bf16(rng, (M, ncols))
    dx, dw = dev(xb), dev(wb)
    dy = dev(hb) if epi == hai.EPI_RESIDUAL else out_buf(M * ncols * 2)
    res = dy.ptr if epi == hai.EPI_RESIDUAL else None
    if norm:
        nw, nwb = rand_bf16(rng, (K_,), 0.02)
        dnw = dev(nwb)
        xin = orc.rmsnorm(x, nw, 1e-6, True)
        hai.check(kern().hai_gemm_rmsnorm_bf16(dy.ptr, ncols, dx.ptr, K_, dnw.ptr, 1e-6, 1, None, K_, dw.ptr, M, N,
                                               K_, epi, res, ncols, None), name)
    else:
        xin = x
        hai.check(kern().hai_gemm_bf16(dy.ptr, ncols, dx.ptr, K_, dw.ptr, M, N, K_, epi, res, ncols, None), name)
    y = orc.gemm(xin, w)
    want = {hai.EPI_STORE: lambda: y, hai.EPI_RESIDUAL: lambda: orc.add(h, y),
            hai.EPI_SILU_MUL: lambda: orc.silu_mul(y[:, 0::2], y[:, 1::2])}[epi]()
    assert_bits_equal(dy.download(np.uint16), want, name)


@pytest.mark.parametrize("N,K_,epi,ldx", [(8200, 5120, 0, 5120), (16480, 5120, 0, 5144), (34816, 5120, 2, 5120),
                                         (9000, 8192, 1, 8192), (12000, 5128, 1, 5136), (8194, 1000, 2, 1000)])
def test_gemm_two_rows_wide_staged(N, K_, epi, ldx):
    """Two-row launches of the wide layers (N > 8192) stage the rows in LDS
    once per resident block (rows already normalised, e.g. by a residual
    launch's norm tail): bit-exact for every epilogue, ragged K and N, row
    pitch above K."""
    M = 2
    rng = np.random.default_rng(N + K_ + 3 * epi)
    xp, xpb = rand_bf16(rng, (M, ldx))
    w, wb = rand_bf16(rng, (N, K_), 0.02)
    ncols = N // 2 if epi == hai.EPI_SILU_MUL else N
    h, hb = rand_bf16(rng, (M, ncols))
    dx, dw = dev(xpb), dev(wb)
    dy = dev(hb) if epi == hai.EPI_RESIDUAL else out_buf(M * ncols * 2)
    res = dy.ptr if epi == hai.EPI_RESIDUAL else None
    hai.check(kern().hai_gemm_bf16(dy.ptr, ncols, dx.ptr, ldx, dw.ptr, M, N, K_, epi, res, ncols, None), "gemm")
    y = orc.gemm(xp[:, :K_], w)
    want = {hai.EPI_STORE: lambda: y, hai.EPI_RESIDUAL: lambda: orc.add(h, y),
            hai.EPI_SILU_MUL: lambda: orc.silu_mul(y[:, 0::2], y[:, 1::2])}[epi]()
    assert_bits_equal(dy.download(np.uint16), want, f"two-row staged {N}x{K_} epi {epi}")


def test_copy_calibration():
    """One device-to-device copy of 256 MiB: the dispatch of known size that
    scales the rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes."""
    n = 256 << 20
    src, dst = out_buf(n), hai.DeviceBuffer(n)
    hai.check(kern().hai_memcpy_d2d(dst.ptr, src.ptr, n, None), "calibration copy")
    hai.synchronize()
    assert not dst.download(np.uint8)[:: 1 << 16].any()


def test_gemm_rmsnorm_needs_xn_above_fused_limit():
    d = out_buf(1 << 16)
    # M*K = 4*5120 > 16384 without an xn_out buffer
    assert kern().hai_gemm_rmsnorm_bf16(d.ptr, 8, d.ptr, 5120, d.ptr, 1e-6, 1, None, 0, d.ptr, 4, 8, 5120, 0,
                                        None, 0, None) == 1


# ----------------------------------------------------------------- norms
@pytest.mark.parametrize("rows,H", [(1, 256), (5, 256), (2, 5120), (3, 64)])
def test_rmsnorm(rows, H):
    rng = np.random.default_rng(rows + H)
    x, xb = rand_bf16(rng, (rows, H))
    w, wb = rand_bf16(rng, (H,), 0.02)
    dx, dw, dy = dev(xb), dev(wb), out_buf(rows * H * 2)
    hai.check(kern().hai_rmsnorm_bf16(dy.ptr, H, dx.ptr, H, dw.ptr, rows, H, 1e-6, 1, None), "rmsnorm")
    assert_bits_equal(dy.download(np.uint16), orc.rmsnorm(x, w, 1e-6, True), "rmsnorm")


@pytest.mark.parametrize("H,y_off", [(64, 0), (5120, 0), (8200, 0), (100, 0), (64, 1)],
                         ids=["vec", "vec_27b", "vec_two_passes", "scalar_ragged", "scalar_unaligned"])
def test_embedding_gather(H, y_off):
    """Rows of the table copied bit for bit; ids outside [0, V) give zero
    rows.  16-byte pieces when H % 8 == 0 and both pointers are 16-byte
    aligned (H = 8200: more pieces than one pass of the block covers),
    element copies otherwise (ragged H, an output offset by one element)."""
    rng = np.random.default_rng(5 + H)
    V = 50
    tab, tb = rand_bf16(rng, (V, H))
    ids = np.array([3, 0, 49, 50, -1, 7], np.int64)
    dt, di, dy = dev(tb), dev(ids), out_buf((ids.size * H + y_off) * 2)
    hai.check(kern().hai_embedding_gather_bf16(dy.ptr + 2 * y_off, dt.ptr, di.ptr, ids.size, V, H, None), "embedding")
    got = dy.download(np.uint16)[y_off:]
    assert_bits_equal(got, orc.embedding(tab, ids), "embedding")


def test_embedding_and_elementwise():
    rng = np.random.default_rng(5)
    a, ab = rand_bf16(rng, (1000,))
    b, bb = rand_bf16(rng, (1000,))
    da, db, dz = dev(ab), dev(bb), out_buf(2000)
    hai.check(kern().hai_add_bf16(dz.ptr, da.ptr, db.ptr, 1000, None), "add")
    assert_bits_equal(dz.download(np.uint16), orc.add(a, b), "add")
    hai.check(kern().hai_silu_mul_bf16(dz.ptr, da.ptr, db.ptr, 1000, None), "silu_mul")
    assert_bits_equal(dz.download(np.uint16), orc.silu_mul(a, b), "silu_mul")


def _rope_dev(npos, R, base):
    c, s = orc.rope_table(0, npos, R, base)
    return dev(c), dev(s)


@pytest.mark.parametrize("B,T,nq,D,R,base", [(1, 2, 4, 64, 16, 1e7), (1, 4, 24, 256, 64, 1e7),
                                               (2, 3, 2, 64, 64, 1e4)])
def test_q_gate_rmsnorm_rope(B, T, nq, D, R, base):
    rng = np.random.default_rng(B * 7 + T + D)
    src, sb = rand_bf16(rng, (B * T, nq * 2 * D))
    w, wb = rand_bf16(rng, (D,), 0.02)
    lens = np.array([5 + 11 * b for b in range(B)], np.int32)
    npos = 64
    cd, sd = _rope_dev(npos, R, base)
    dsrc, dw, dl = dev(sb), dev(wb), dev(lens)
    dq, dg = out_buf(B * T * nq * D * 2), out_buf(B * T * nq * D * 2)
    hai.check(kern().hai_q_gate_rmsnorm_rope_bf16(dq.ptr, dg.ptr, dsrc.ptr, nq * 2 * D, dw.ptr, cd.ptr, sd.ptr,
                                                  npos, B, T, nq, D, R, dl.ptr, 1, 1e-6, None), "q_gate")
    gq, gg = dq.download(np.uint16), dg.download(np.uint16)
    for b in range(B):
        q, g = orc.q_gate_rmsnorm_rope(src[b * T:(b + 1) * T], w, T, nq, D, R, int(lens[b]) + 1, base)
        n = T * nq * D
        assert_bits_equal(gq[b * n:(b + 1) * n], q, "q")
        assert_bits_equal(gg[b * n:(b + 1) * n], g, "gate")


@pytest.mark.parametrize("B,T,nkv,D,R", [(1, 2, 2, 64, 16), (1, 4, 4, 256, 64), (2, 1, 1, 64, 64)])
def test_kv_norm_rope_append(B, T, nkv, D, R):
    rng = np.random.default_rng(B + T * 3 + D)
    base = 1e7
    cap = 40
    ld = 2 * nkv * D + 8
    src, sb = rand_bf16(rng, (B * T, ld))
    w, wb = rand_bf16(rng, (D,), 0.02)
    lens = np.array([3 + 17 * b for b in range(B)], np.int32)
    cd, sd = _rope_dev(cap, R, base)
    dsrc, dw, dl = dev(sb), dev(wb), dev(lens)
    kc, vc = out_buf(B * cap * nkv * D * 2), out_buf(B * cap * nkv * D * 2)
    hai.check(kern().hai_kv_rmsnorm_rope_append_bf16(kc.ptr, vc.ptr, cap, dsrc.ptr, dsrc.ptr + nkv * D * 2, ld,
                                                     dw.ptr, cd.ptr, sd.ptr, cap, B, T, nkv, D, R, dl.ptr, 0,
                                                     1e-6, None), "kv append")
    K_ = kc.download(np.uint16).reshape(B, cap, nkv * D)
    V_ = vc.download(np.uint16).reshape(B, cap, nkv * D)
    for b in range(B):
        rows = src[b * T:(b + 1) * T]
        k = orc.k_rmsnorm_rope(rows[:, :nkv * D], w, T, nkv, D, R, int(lens[b]), base)
        p = int(lens[b])
        assert_bits_equal(K_[b, p:p + T], k, "k cache")
        assert_bits_equal(V_[b, p:p + T], rows[:, nkv * D:2 * nkv * D], "v cache")
        assert not K_[b, :p].any() and not K_[b, p + T:].any()


@pytest.mark.parametrize("B,T,nq,nkv,D,R", [(1, 2, 24, 4, 256, 64), (2, 3, 4, 2, 64, 16), (3, 1, 6, 1, 128, 128)])
def test_qkv_norm_rope_append_equals_the_two_launches(B, T, nq, nkv, D, R):
    """hai_qkv_rmsnorm_rope_append_bf16 on [q+gate | k | v] projection rows
    writes the same q, gate and cache rows as the q/gate and K/V launches."""
    rng = np.random.default_rng(B * 7 + T + nq + D)
    cap, base = 48, 1e7
    ld = (2 * nq + 2 * nkv) * D
    src, sb = rand_bf16(rng, (B * T, ld))
    wq, wqb = rand_bf16(rng, (D,), 0.02)
    wk, wkb = rand_bf16(rng, (D,), 0.02)
    lens = np.array([5 + 11 * b for b in range(B)], np.int32)
    cd, sd = _rope_dev(cap, R, base)
    dsrc, dwq, dwk, dl = dev(sb), dev(wqb), dev(wkb), dev(lens)
    outs = []
    for fused in (False, True):
        q, g = out_buf(B * T * nq * D * 2), out_buf(B * T * nq * D * 2)
        kc, vc = out_buf(B * cap * nkv * D * 2), out_buf(B * cap * nkv * D * 2)
        if fused:
            hai.check(kern().hai_qkv_rmsnorm_rope_append_bf16(q.ptr, g.ptr, kc.ptr, vc.ptr, cap, dsrc.ptr, ld,
                                                               dwq.ptr, dwk.ptr, cd.ptr, sd.ptr, cap, B, T, nq, nkv,
                                                               D, R, dl.ptr, 0, 1e-6, None), "qkv")
        else:
            hai.check(kern().hai_q_gate_rmsnorm_rope_bf16(q.ptr, g.ptr, dsrc.ptr, ld, dwq.ptr, cd.ptr, sd.ptr, cap,
                                                           B, T, nq, D, R, dl.ptr, 0, 1e-6, None), "q gate")
            ks = dsrc.ptr + 2 * nq * D * 2
            hai.check(kern().hai_kv_rmsnorm_rope_append_bf16(kc.ptr, vc.ptr, cap, ks, ks + nkv * D * 2, ld, dwk.ptr,
                                                             cd.ptr, sd.ptr, cap, B, T, nkv, D, R, dl.ptr, 0, 1e-6,
                                                             None), "kv")
        outs.append([buf.download(np.uint16) for buf in (q, g, kc, vc)])
    for name, a, b in zip(("q", "gate", "k cache", "v cache"), outs[0], outs[1]):
        assert np.array_equal(a, b), name


@pytest.mark.parametrize("B,T,nq,nkv,D,R,L0", [
    (1, 2, 24, 4, 256, 64, [1278]),       # C3 verify: both new rows in the last chunk
    (1, 2, 24, 4, 256, 64, [63]),         # new rows straddle chunks 0 and 1
    (2, 4, 4, 2, 64, 16, [100, 0]),       # a sequence whose new rows start the cache
    (1, 16, 4, 2, 128, 128, [200]),       # 16-row chunk over two key chunks, full rotation
    (3, 1, 24, 4, 256, 64, [4000, 5, 64]),  # correction rows; several query groups per block
    (1, 4, 24, 4, 256, 64, [1590]),       # 8 queries per block, 2 per wave
    (2, 4, 24, 4, 256, 64, [6390, 100]),  # all 24 per block, 3 per wave on 8 waves
])
def test_gqa_verify_fused_equals_norm_then_attention(B, T, nq, nkv, D, R, L0):
    """hai_gqa_verify_fused_bf16 against hai_qkv_rmsnorm_rope_append_bf16
    followed by hai_gqa_verify_bf16 on the same projection rows and caches:
    the attention output, the gate halves and both whole caches bit for bit
    (the new K / V rows are built inside the partial pass and appended by
    its first query group)."""
    rng = np.random.default_rng(B * 100 + T * 10 + D + L0[0])
    cap = max(L0) + T + 70
    base = 1e7
    ld = (2 * nq + 2 * nkv) * D + 8
    _, sb = rand_bf16(rng, (B * T, ld))
    _, wqb = rand_bf16(rng, (D,), 0.02)
    _, wkb = rand_bf16(rng, (D,), 0.02)
    _, kcb = rand_bf16(rng, (B * cap * nkv * D,))
    _, vcb = rand_bf16(rng, (B * cap * nkv * D,))
    lens = np.array(L0, np.int32)
    cd, sd = _rope_dev(cap, R, base)
    dsrc, dwq, dwk, dl = dev(sb), dev(wqb), dev(wkb), dev(lens)
    sc = out_buf(kern().hai_gqa_scratch_bytes(B, T, nq, D, cap))
    outs = []
    for fused in (False, True):
        kc, vc = dev(kcb), dev(vcb)
        out, g = out_buf(B * T * nq * D * 2), out_buf(B * T * nq * D * 2)
        if fused:
            hai.check(kern().hai_gqa_verify_fused_bf16(out.ptr, g.ptr, dsrc.ptr, ld, dwq.ptr, dwk.ptr, cd.ptr, sd.ptr,
                                                       cap, R, 1e-6, kc.ptr, vc.ptr, cap, sc.ptr, B, T, nq, nkv, D,
                                                       dl.ptr, T, cap, None), "fused")
        else:
            q = out_buf(B * T * nq * D * 2)
            hai.check(kern().hai_qkv_rmsnorm_rope_append_bf16(q.ptr, g.ptr, kc.ptr, vc.ptr, cap, dsrc.ptr, ld,
                                                               dwq.ptr, dwk.ptr, cd.ptr, sd.ptr, cap, B, T, nq, nkv,
                                                               D, R, dl.ptr, 0, 1e-6, None), "qkv")
            hai.check(kern().hai_gqa_verify_bf16(out.ptr, q.ptr, g.ptr, kc.ptr, vc.ptr, cap, sc.ptr, B, T, nq, nkv,
                                                 D, dl.ptr, T, cap, None), "attention")
        outs.append([buf.download(np.uint16) for buf in (out, g, kc, vc)])
    for name, a, b in zip(("output", "gate", "k cache", "v cache"), outs[0], outs[1]):
        assert np.array_equal(a, b), name


# ----------------------------------------------------------------- attention
@pytest.mark.parametrize("B,T,nq,nkv,D,lens", [
    (1, 2, 4, 2, 64, [30]), (1, 1, 4, 2, 64, [0]), (1, 4, 24, 4, 256, [60]), (1, 2, 24, 4, 256, [1278]),
    (2, 3, 4, 1, 128, [63, 200]), (1, 16, 4, 2, 64, [100]), (3, 1, 2, 2, 64, [0, 1, 64]),
    (1, 4, 24, 4, 256, [4092]),  # C2 micro-bench shape (cache 4096 incl. the 4 new rows)
    (1, 4, 24, 4, 256, [1590]),  # 100 chunk blocks: 8 of the 24 queries per block, 2 per wave
    (2, 4, 24, 4, 256, [6390, 100]),  # 800 chunk blocks: all 24 per block, 3 per wave on 8 waves
    (4, 4, 24, 4, 256, [8186, 3000, 64, 5000]),  # C4-like: all 24 per block
    (4, 2, 24, 4, 256, [8180, 10, 4000, 8100]),  # all 12 per block, 2 per wave on 8 waves
    (4, 4, 24, 4, 128, [8186, 300, 7000, 1]),  # head_dim 128, 6 per wave
    (8, 6, 8, 2, 64, [8100, 8000, 3, 64, 128, 4000, 8120, 500])])  # head_dim 64 (half the lanes in P.V)
def test_gqa_verify(B, T, nq, nkv, D, lens):
    rng = np.random.default_rng(B * 100 + T * 10 + D + sum(lens))
    lens = np.array(lens, np.int32)
    cap = int(lens.max()) + T + 5
    q, qb = rand_bf16(rng, (B * T, nq, D))
    g, gb = rand_bf16(rng, (B * T, nq, D))
    kcache, kb = rand_bf16(rng, (B, cap, nkv, D))
    vcache, vb = rand_bf16(rng, (B, cap, nkv, D))
    dq, dg, dk, dv, dl = dev(qb), dev(gb), dev(kb), dev(vb), dev(lens)
    max_len = cap
    scratch = out_buf(kern().hai_gqa_scratch_bytes(B, T, nq, D, max_len))
    dout = out_buf(B * T * nq * D * 2)
    hai.check(kern().hai_gqa_verify_bf16(dout.ptr, dq.ptr, dg.ptr, dk.ptr, dv.ptr, cap, scratch.ptr, B, T, nq,
                                         nkv, D, dl.ptr, T, max_len, None), "gqa")
    got = dout.download(np.uint16).reshape(B, T * nq * D)
    for b in range(B):
        L = int(lens[b]) + T
        want = orc.attention(q[b * T:(b + 1) * T], g[b * T:(b + 1) * T], kcache[b], vcache[b], T, L, nq, nkv, D)
        assert_bits_equal(got[b], want, f"gqa b={b}")


def _attention_f64(q, g, kc, vc, T, L, nq, nkv, D):
    """Gated causal GQA in float64 for one sequence: the output and, per
    element, sigmoid(gate) * sum_i p_i |v_i| / sum_i p_i (the scale of the
    P-rounding error)."""
    group = nq // nkv
    out = np.zeros((T, nq, D))
    mag = np.zeros((T, nq, D))
    pos = L - T + np.arange(T)
    for h in range(nq):
        k = kc[:L, h // group].astype(np.float64)
        v = vc[:L, h // group].astype(np.float64)
        s = q[:, h].astype(np.float64) @ k.T / np.sqrt(D)
        s[np.arange(L)[None, :] > pos[:, None]] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        l = p.sum(1, keepdims=True)
        sig = 1.0 / (1.0 + np.exp(-g[:, h].astype(np.float64)))
        out[:, h] = (p @ v) / l * sig
        mag[:, h] = (p @ np.abs(v)) / l * sig
    return out, mag


@pytest.mark.parametrize("B,T,nq,nkv,D,lens", [
    (1, 2, 4, 2, 64, [30]), (1, 1, 4, 2, 64, [0]), (3, 1, 2, 2, 64, [0, 1, 64]), (2, 3, 4, 1, 128, [63, 200]),
    (1, 16, 4, 2, 64, [100]),  # 32 queries: two query tiles
    (1, 16, 8, 2, 64, [300]),  # 64 queries: two blocks per KV head
    (1, 4, 24, 4, 256, [4092]),  # C2 micro-bench shape
    (4, 4, 24, 4, 256, [8186, 3000, 64, 5000]),  # C4 verify-like (24 queries per KV head)
    (8, 1, 24, 4, 256, [8190, 8000, 1, 63, 64, 127, 128, 4097]),  # C4 draft-like
    (6, 2, 24, 4, 256, [580, 10, 600, 511, 512, 513]),  # C5 verify-like
    (4, 4, 24, 4, 128, [8186, 300, 7000, 1]),
    (8, 6, 8, 2, 64, [8100, 8000, 3, 64, 128, 4000, 8120, 500]),
    (1, 32, 24, 4, 256, [64]),  # prompt chunk, 192 query rows per KV head: the flash form, two blocks
    (2, 24, 24, 4, 256, [500, 0]),  # flash form, ragged histories, a chunk with none
    (1, 64, 24, 4, 256, [1000])])  # three flash blocks over 1064 keys
def test_gqa_verify_mfma(B, T, nq, nkv, D, lens):
    """Tolerance-mode attention on the matrix cores against float64.  P is
    rounded to bf16 (unit roundoff 2^-8 per weight) before P.V, so an output
    element may move by 2^-8 * sum p |v| / sum p (times the gate); the
    output's own bf16 rounding adds 2^-8 |out|.  The bound is that sum with
    25 % slack for the fp32 accumulation and exp2 errors (~2^-22 relative)."""
    rng = np.random.default_rng(B * 100 + T * 10 + D + sum(lens) + 7)
    lens = np.array(lens, np.int32)
    cap = int(lens.max()) + T + 5
    q, qb = rand_bf16(rng, (B * T, nq, D))
    g, gb = rand_bf16(rng, (B * T, nq, D))
    kcache, kb = rand_bf16(rng, (B, cap, nkv, D))
    vcache, vb = rand_bf16(rng, (B, cap, nkv, D))
    dq, dg, dk, dv, dl = dev(qb), dev(gb), dev(kb), dev(vb), dev(lens)
    max_len = cap
    scratch = out_buf(kern().hai_gqa_mfma_scratch_bytes(B, T, nq, D, max_len))
    dout = out_buf(B * T * nq * D * 2)
    hai.check(kern().hai_gqa_verify_mfma_bf16(dout.ptr, dq.ptr, dg.ptr, dk.ptr, dv.ptr, cap, scratch.ptr, B, T, nq,
                                              nkv, D, dl.ptr, T, max_len, None), "gqa mfma")
    got = hai.bf16_to_f32(dout.download(np.uint16)).reshape(B, T, nq, D)
    for b in range(B):
        L = int(lens[b]) + T
        want, mag = _attention_f64(q[b * T:(b + 1) * T], g[b * T:(b + 1) * T], kcache[b], vcache[b], T, L, nq,
                                   nkv, D)
        err = np.abs(got[b] - want)
        bound = 1.25 * 2.0 ** -8 * (mag + np.abs(want)) + 1e-6
        assert np.isfinite(got[b]).all(), b
        assert (err <= bound).all(), (b, float((err / bound).max()))


# ----------------------------------------------------------------- deltanet
def _deltanet_case(rng, B, nk, nv, dk, dv, Kc=4):
    kw, vw = nk * dk, nv * dv
    C = 2 * kw + vw
    conv_w, cwb = rand_bf16(rng, (C, Kc), 0.3)
    a_log, alb = rand_bf16(rng, (nv,), 0.5)
    dt_bias, dtb = rand_bf16(rng, (nv,), 0.5)
    norm_w, nwb = rand_bf16(rng, (dv,), 0.5)
    return dict(C=C, conv_w=conv_w, cwb=cwb, a_log=a_log, alb=alb, dt_bias=dt_bias, dtb=dtb, norm_w=norm_w,
                nwb=nwb, Kc=Kc)


def _to_tiled(state, nv, dk, dv):
    """Reference [nv][dk][dv] state -> the kernel's column-tiled head layout:
    key i = g*(dk/4) + 4m + e, value j at ((m*dv + j)*4 + g)*4 + e."""
    t = state.reshape(nv, 4, dk // 16, 4, dv).transpose(0, 2, 4, 1, 3)
    return np.ascontiguousarray(t).reshape(nv, dv, dk)


@pytest.mark.parametrize("split", [False, True], ids=["one_block", "column_split"])
@pytest.mark.parametrize("nk,nv,dk,dv,steps", [(4, 4, 64, 64, [2, 1, 3]), (16, 48, 128, 128, [4, 2]),
                                               (2, 6, 64, 64, [16, 1])])
def test_deltanet_verify_rollback(nk, nv, dk, dv, steps, split):
    """Chained verify steps with partial acceptance: the kernel's committed
    state/conv ring after each accepted prefix must equal the oracle's
    sequential processing of the accepted tokens only.  column_split: the
    workspace entry point (each head's value columns over 4 blocks at these
    head counts)."""
    rng = np.random.default_rng(nk * 1000 + nv + dk)
    B = 1
    c = _deltanet_case(rng, B, nk, nv, dk, dv)
    C, Kc = c["C"], c["Kc"]
    vw = nv * dv
    width = C + vw + 2 * nv
    ring, nslots = 32, 17
    dring, dstate = out_buf(B * ring * C * 2), out_buf(nslots * B * nv * dk * dv * 4)
    dcw, dal, ddt, dnw = dev(c["cwb"]), dev(c["alb"]), dev(c["dtb"]), dev(c["nwb"])
    # oracle state in reference layout
    conv_state = np.zeros((C, Kc - 1), np.float32)
    state = np.zeros((nv, dk, dv), np.float32)
    L = 0
    lens = dev(np.array([0], np.int32))
    wsb = kern().hai_deltanet_workspace_bytes(B, nv, dv)
    dws = out_buf(wsb)
    for si, T in enumerate(steps):
        proj, pb = rand_bf16(rng, (T, width))
        dproj, dout = dev(pb), out_buf(T * vw * 2)
        lens.upload(np.array([L], np.int32))
        args = (dout.ptr, vw, dproj.ptr, width, 0, C, C + vw, C + vw + nv, dcw.ptr, dring.ptr, ring, dstate.ptr,
                nslots, 1, dal.ptr, ddt.ptr, dnw.ptr, lens.ptr, 0, B, T, nk, nv, dk, dv, Kc, 1e-6)
        if split:
            hai.check(kern().hai_deltanet_verify_ws_bf16(*args, dws.ptr, wsb, None), "deltanet split")
        else:
            hai.check(kern().hai_deltanet_verify_bf16(*args, None), "deltanet")
        got = dout.download(np.uint16).reshape(T, vw)
        # oracle over all T tokens from the committed state
        q, k, v, cs_all = orc.deltanet_conv(proj[:, :C], c["conv_w"], conv_state, T, nk, nv, dk, dv, Kc)
        out, st_all = orc.deltanet_recurrent(q, k, v, proj[:, C + vw:C + vw + nv], proj[:, C + vw + nv:],
                                             proj[:, C:C + vw], c["a_log"], c["dt_bias"], c["norm_w"], state, T,
                                             nk, nv, dk, dv)
        assert_bits_equal(got, out, f"deltanet step {si} out")
        # accept a prefix of length acc (1..T) and advance the oracle by exactly those tokens
        acc = 1 + (si % T)
        q2, k2, v2, conv_state = orc.deltanet_conv(proj[:acc, :C], c["conv_w"], conv_state, acc, nk, nv, dk, dv, Kc)
        _, state = orc.deltanet_recurrent(q2, k2, v2, proj[:acc, C + vw:C + vw + nv], proj[:acc, C + vw + nv:],
                                          proj[:acc, C:C + vw], c["a_log"], c["dt_bias"], c["norm_w"], state, acc,
                                          nk, nv, dk, dv)
        L += acc
        slot = L % nslots
        dev_state = dstate.download(np.float32).reshape(nslots, B, nv, dv, dk)[slot, 0]
        want_state = _to_tiled(state, nv, dk, dv)
        assert np.array_equal(dev_state.view(np.uint32), want_state.view(np.uint32)), f"state after step {si}"


@pytest.mark.parametrize("nk,nv,dk,B,ab,rounds", [
    (4, 4, 64, 2, False, [(2, [1, 2]), (3, [3, 1]), (4, [2, 4]), (1, [1, 1]), (4, [1, 3])]),
    (16, 48, 128, 2, True, [(2, [1, 2]), (2, [2, 2]), (4, [3, 1]), (2, [1, 1])]),
    (2, 6, 64, 3, True, [(3, [1, 2, 3]), (4, [4, 4, 1]), (1, [1, 1, 1])]),
])
def test_deltanet_records_replay_equals_per_token_slots(nk, nv, dk, B, ab, rounds):
    """Verify rounds of B sequences, each keeping its own prefix of the T
    tokens (a + 1 of them) followed by a one-token correction, run twice:
    with per-token state slots (write_all_slots: the correction reads the
    kept prefix's slot) and with rollback records (hai_deltanet_verify_rec_bf16:
    only the final state, replay = 1 for the correction from the verify's
    start).  Outputs of every call, the committed states and the conv rings
    bit for bit.  A round in which every sequence keeps all T tokens goes
    straight to the next verify; in the other rounds every sequence takes the
    correction, also one that kept all T (the engine's lockstep batches: its
    replay re-applies all T records).  With ab: the a|b projection formed in
    the kernel."""
    rng = np.random.default_rng(nk * 100 + nv * 10 + B)
    dv = dk
    kw, vw = nk * dk, nv * dv
    C = 2 * kw + vw
    H = 128
    Kc = 4
    width = C + vw + 2 * nv
    ring, nslots = 16, 5
    cw, cwb = rand_bf16(rng, (C, Kc), 0.3)
    al, alb = rand_bf16(rng, (nv,), 0.5)
    dt, dtb = rand_bf16(rng, (nv,), 0.5)
    nw, nwb = rand_bf16(rng, (dv,), 0.5)
    wab, wabb = rand_bf16(rng, (2 * nv, H), 0.05)
    st0 = (rng.standard_normal(nslots * B * nv * dk * dv) * 0.1).astype(np.float32)
    lens0 = np.array([2 + 3 * b for b in range(B)], np.int32)
    dcw, dal, ddt, dnw, dwab = dev(cwb), dev(alb), dev(dtb), dev(nwb), dev(wabb)
    rec_bytes = kern().hai_deltanet_records_bytes(nslots, B, nv, dk, dv)
    assert rec_bytes == nslots * B * nv * (dk + dv + 4) * 4
    inputs = []
    for T, keep in rounds:
        _, pb = rand_bf16(rng, (B * T, width))
        _, xnb = rand_bf16(rng, (B * T, H))
        _, cpb = rand_bf16(rng, (B, width))
        _, cxb = rand_bf16(rng, (B, H))
        inputs.append((T, keep, pb, xnb, cpb, cxb))

    def run(records):
        dstate, dring, lens = dev(st0), out_buf(B * ring * C * 2), dev(lens0)
        drec, dbase = (out_buf(rec_bytes), out_buf(B * 4)) if records else (None, None)
        L = lens0.astype(np.int64).copy()
        outs = []

        def call(T, pb, xnb, mode):
            dout, dproj, dxn = out_buf(B * T * vw * 2), dev(pb), dev(xnb)
            common = (dout.ptr, vw, dproj.ptr, width, 0, C)
            if records:
                hai.check(kern().hai_deltanet_verify_rec_bf16(
                    *common, C + vw, C + vw + nv, dxn.ptr if ab else None, H if ab else 0, dwab.ptr if ab else None,
                    H if ab else 0, dcw.ptr, dring.ptr, ring, dstate.ptr, nslots, drec.ptr, dbase.ptr,
                    1 if mode == "correction" else 0, dal.ptr, ddt.ptr, dnw.ptr, lens.ptr, 0, B, T, nk, nv, dk, dv,
                    Kc, 1e-6, None), "deltanet rec")
            else:
                tail = (dcw.ptr, dring.ptr, ring, dstate.ptr, nslots, 1 if mode == "verify" else 0, dal.ptr,
                        ddt.ptr, dnw.ptr, lens.ptr, 0, B, T, nk, nv, dk, dv, Kc, 1e-6)
                if ab:
                    hai.check(kern().hai_deltanet_verify_ab_bf16(*common, dxn.ptr, H, dwab.ptr, H, *tail, None), "ab")
                else:
                    hai.check(kern().hai_deltanet_verify_bf16(*common, C + vw, C + vw + nv, *tail, None), "dn")
            outs.append(dout.download(np.uint16))

        for T, keep, pb, xnb, cpb, cxb in inputs:
            lens.upload(L.astype(np.int32))
            call(T, pb, xnb, "verify")
            L = L + np.array(keep)
            if not all(k == T for k in keep):
                lens.upload(L.astype(np.int32))
                call(1, cpb, cxb, "correction")
                L = L + 1
        lens_np = L
        st = dstate.download(np.float32).reshape(nslots, B, nv * dk * dv)
        committed = np.stack([st[lens_np[b] % nslots, b] for b in range(B)])
        return outs, committed, dring.download(np.uint16)

    o_ref, st_ref, ring_ref = run(False)
    o_rec, st_rec, ring_rec = run(True)
    assert len(o_ref) == len(o_rec)
    for i, (a, b) in enumerate(zip(o_ref, o_rec)):
        assert np.array_equal(a, b), f"call {i}: outputs differ"
    assert np.array_equal(st_ref.view(np.uint32), st_rec.view(np.uint32)), "committed states differ"
    assert np.array_equal(ring_ref, ring_rec), "conv rings differ"


@pytest.mark.parametrize("nk,nv,dk,T,Kc", [(2, 6, 64, 37, 4), (16, 48, 128, 100, 4), (4, 4, 64, 16, 3),
                                         (16, 48, 128, 32, 4)])
def test_deltanet_prefill_against_oracle(nk, nv, dk, T, Kc):
    """hai_deltanet_prefill_bf16 (the chunkwise form of the gated delta rule:
    32-token chunks, a triangular solve per chunk and the state carried from
    chunk to chunk; tolerance mode) against the oracle's token-by-token conv
    + recurrence of the same T tokens for two sequences with different
    histories (conv inputs from the ring, initial state from slot L % nslots):
    outputs within the bf16 / fp32 reassociation bound, the state within 1e-4
    of its scale, and the conv ring's entries for the chunk's last positions
    bit for bit.  T = 37 and 100 end in a ragged chunk; T = 32 wraps the
    32-entry ring onto the entries the chunk reads first."""
    rng = np.random.default_rng(nv * 7 + T)
    B, dv = 2, dk
    kw, vw = nk * dk, nv * dv
    C = 2 * kw + vw
    hist = Kc - 1
    width = C + vw + 2 * nv
    ring, nslots = 32, 18
    cw, cwb = rand_bf16(rng, (C, Kc), 0.3)
    al, alb = rand_bf16(rng, (nv,), 0.5)
    dt, dtb = rand_bf16(rng, (nv,), 0.5)
    nw, nwb = rand_bf16(rng, (dv,), 0.5)
    proj, pb = rand_bf16(rng, (B * T, width))
    lens0 = np.array([5, 40], np.int32)
    ring0 = rng.standard_normal((B, ring, C)).astype(np.float32)
    ring0b = hai.bf16_bits(ring0)
    ring0 = hai.bf16_to_f32(ring0b)
    states = (rng.standard_normal((B, nv, dk, dv)) * 0.1).astype(np.float32)
    st_dev = np.zeros((nslots, B, nv, dv, dk), np.float32)
    for b in range(B):
        st_dev[lens0[b] % nslots, b] = _to_tiled(states[b], nv, dk, dv)
    dstate, dring, lens = dev(st_dev), dev(ring0b), dev(lens0)
    dout = out_buf(B * T * vw * 2)
    wsb = kern().hai_deltanet_prefill_workspace_bytes(B, T, nv, dv)
    dws = out_buf(wsb)
    # device copies held by name: a temporary's memory would be freed before the launch
    dp, dcw, dal, ddt, dnw = dev(pb), dev(cwb), dev(alb), dev(dtb), dev(nwb)
    hai.check(kern().hai_deltanet_prefill_bf16(dout.ptr, vw, dp.ptr, width, 0, C, C + vw, C + vw + nv, dcw.ptr,
                                               dring.ptr, ring, dstate.ptr, nslots, dal.ptr, ddt.ptr, dnw.ptr,
                                               lens.ptr, 0, B, T, nk, nv, dk, dv, Kc, 1e-6, dws.ptr, wsb, None),
              "deltanet_prefill")
    got = hai.bf16_to_f32(dout.download(np.uint16)).reshape(B, T, vw)
    st_got = dstate.download(np.float32).reshape(nslots, B, nv, dv, dk)
    ring_got = dring.download(np.uint16).reshape(B, ring, C)
    for b in range(B):
        L = int(lens0[b])
        pr = proj[b * T:(b + 1) * T]
        conv_state = np.stack([ring0[b, (L - hist + i) % ring] if L - hist + i >= 0 else np.zeros(C, np.float32)
                               for i in range(hist)], axis=1)
        q, k, v, _ = orc.deltanet_conv(pr[:, :C], cw, conv_state, T, nk, nv, dk, dv, Kc)
        want, st = orc.deltanet_recurrent(q, k, v, pr[:, C + vw:C + vw + nv], pr[:, C + vw + nv:], pr[:, C:C + vw],
                                          al, dt, nw, states[b], T, nk, nv, dk, dv)
        err = np.abs(got[b] - want)
        assert (err <= 2.0 ** -7 * np.abs(want) + 1e-3 * np.abs(want).max()).all(), (b, float(err.max()))
        st_want = _to_tiled(st, nv, dk, dv)
        st_err = np.abs(st_got[(L + T) % nslots, b] - st_want).max()
        assert st_err <= 1e-4 * np.abs(st_want).max(), (b, float(st_err))
        for i in range(hist):
            pos = L + T - hist + i
            assert np.array_equal(ring_got[b, pos % ring], pb.reshape(B, T, width)[b, T - hist + i, :C]), (b, i)


@pytest.mark.parametrize("B,nk,nv,dk,T,Kc,ab", [(3, 2, 6, 64, 40, 4, False), (2, 16, 48, 128, 33, 4, True),
                                                (1, 4, 4, 64, 100, 3, False)])
def test_deltanet_prompt_chunk_equals_16_token_launches(B, nk, nv, dk, T, Kc, ab):
    """One call over a prompt chunk of T > 16 tokens of B sequences (rows
    b*T + t) against the same tokens as launches of at most 16 with their
    rows gathered per launch: outputs, the final state slot and the conv
    ring bit for bit (with ab: the a|b projection formed in the kernel)."""
    rng = np.random.default_rng(B * 1000 + T + nv)
    dv = dk
    kw, vw = nk * dk, nv * dv
    C = 2 * kw + vw
    H = 256
    width = C + vw + 2 * nv
    ring, nslots = 32, 18
    cw, cwb = rand_bf16(rng, (C, Kc), 0.3)
    al, alb = rand_bf16(rng, (nv,), 0.5)
    dt, dtb = rand_bf16(rng, (nv,), 0.5)
    nw, nwb = rand_bf16(rng, (dv,), 0.5)
    xn, xnb = rand_bf16(rng, (B * T, H))
    wab, wabb = rand_bf16(rng, (2 * nv, H), 0.05)
    st0 = (rng.standard_normal(nslots * B * nv * dk * dv) * 0.1).astype(np.float32)
    lens0 = np.array([3 + 5 * b for b in range(B)], np.int32)
    proj, pb = rand_bf16(rng, (B * T, width))
    dcw, dal, ddt, dnw, dwab = dev(cwb), dev(alb), dev(dtb), dev(nwb), dev(wabb)

    def call(dout, dproj, dxn, rows, t0, n, dstate, dring, lens):
        common = (dout.ptr, vw, dproj.ptr, width, 0, C)
        tail = (dcw.ptr, dring.ptr, ring, dstate.ptr, nslots, 0, dal.ptr, ddt.ptr, dnw.ptr, lens.ptr, t0, B, n, nk,
                nv, dk, dv, Kc, 1e-6)
        if ab:
            hai.check(kern().hai_deltanet_verify_ab_bf16(*common, dxn.ptr, H, dwab.ptr, H, *tail, None), "ab")
        else:
            hai.check(kern().hai_deltanet_verify_bf16(*common, C + vw, C + vw + nv, *tail, None), "deltanet")

    got = {}
    for mode in ("one_call", "launches"):
        dstate, dring, lens = dev(st0), out_buf(B * ring * C * 2), dev(lens0)
        if mode == "one_call":
            dout = out_buf(B * T * vw * 2)
            call(dout, dev(pb), dev(xnb), B * T, 0, T, dstate, dring, lens)
            out = dout.download(np.uint16).reshape(B, T, vw)
        else:
            out = np.zeros((B, T, vw), np.uint16)
            for t0 in range(0, T, 16):
                n = min(16, T - t0)
                sub = np.ascontiguousarray(pb.reshape(B, T, width)[:, t0:t0 + n].reshape(B * n, width))
                subx = np.ascontiguousarray(xnb.reshape(B, T, H)[:, t0:t0 + n].reshape(B * n, H))
                dsout = out_buf(B * n * vw * 2)
                call(dsout, dev(sub), dev(subx), B * n, t0, n, dstate, dring, lens)
                out[:, t0:t0 + n] = dsout.download(np.uint16).reshape(B, n, vw)
        slots = dstate.download(np.uint32).reshape(nslots, B, -1)
        final = np.stack([slots[(int(lens0[b]) + T) % nslots, b] for b in range(B)])
        got[mode] = (out, final, dring.download(np.uint16))
    for i, what in enumerate(("outputs", "final state", "conv ring")):
        assert np.array_equal(got["one_call"][i], got["launches"][i]), what


@pytest.mark.parametrize("B,nk,nv,dk,T,Kc", [(1, 16, 48, 128, 2, 4), (3, 16, 48, 128, 4, 4), (2, 2, 6, 64, 16, 3),
                                             (1, 16, 48, 128, 17, 4)])
def test_deltanet_column_split_matches_one_block(B, nk, nv, dk, T, Kc):
    """The workspace entry point (value columns of a head over 4 blocks at
    48 heads, over 2 at 144) against the one-block kernel, bit for bit: the
    outputs, every state slot written, the conv ring, and the workspace
    counters back at zero.  Two launches in a row (the second from the state
    the first left), T = 17 as the two launches of a width-16 verify."""
    rng = np.random.default_rng(B * 100 + nv + T)
    dv = dk
    kw, vw = nk * dk, nv * dv
    C = 2 * kw + vw
    width = C + vw + 2 * nv
    ring, nslots = 40, 18
    cw, cwb = rand_bf16(rng, (C, Kc), 0.3)
    al, alb = rand_bf16(rng, (nv,), 0.5)
    dt, dtb = rand_bf16(rng, (nv,), 0.5)
    nw, nwb = rand_bf16(rng, (dv,), 0.5)
    st0 = (rng.standard_normal(nslots * B * nv * dk * dv) * 0.1).astype(np.float32)
    rg0 = hai.bf16_bits(rng.standard_normal(B * ring * C).astype(np.float32))
    lens0 = np.array([5 + 3 * b for b in range(B)], np.int32)
    proj, pb = rand_bf16(rng, (B * T, width))
    wsb = kern().hai_deltanet_workspace_bytes(B, nv, dv)
    results = []
    for split in (False, True):
        dstate, dring, dws = dev(st0), dev(rg0), out_buf(wsb)
        dcw, dal, ddt, dnw, dproj, lens = dev(cwb), dev(alb), dev(dtb), dev(nwb), dev(pb), dev(lens0)
        dout = out_buf(B * T * vw * 2)
        for t0 in range(0, T, 16):
            n = min(16, T - t0)
            # rows of launch t0: the projection rows t0.. of every sequence
            sub = np.ascontiguousarray(pb.reshape(B, T, width)[:, t0:t0 + n].reshape(B * n, width))
            dsub, dsout = dev(sub), out_buf(B * n * vw * 2)
            args = (dsout.ptr, vw, dsub.ptr, width, 0, C, C + vw, C + vw + nv, dcw.ptr, dring.ptr, ring, dstate.ptr,
                    nslots, 1, dal.ptr, ddt.ptr, dnw.ptr, lens.ptr, t0, B, n, nk, nv, dk, dv, Kc, 1e-6)
            if split:
                hai.check(kern().hai_deltanet_verify_ws_bf16(*args, dws.ptr, wsb, None), "deltanet split")
            else:
                hai.check(kern().hai_deltanet_verify_bf16(*args, None), "deltanet")
            results.append((split, t0, dsout.download(np.uint16)))
        results.append((split, "state", dstate.download(np.uint32)))
        results.append((split, "ring", dring.download(np.uint16)))
        if split:
            counters = dws.download(np.uint32)[: B * nv]
            assert not counters.any(), "workspace counters not reset"
    half = len(results) // 2
    for (s0, k0, a), (s1, k1, b) in zip(results[:half], results[half:]):
        assert k0 == k1 and not s0 and s1
        assert np.array_equal(a, b), f"column split differs from one block: {k0}"


# ----------------------------------------------------------------- argmax / accept
@pytest.mark.parametrize("V,ld", [(248320, 248320), (1003, 1008), (1003, 1003), (13, 13)],
                         ids=["vocab_27b", "ragged_row_aligned", "unaligned_rows", "tiny"])
def test_argmax_rows_ties_nan(V, ld):
    """First index on ties, NaN and -inf never win, -0 ties +0; 16-byte
    logit pieces where the rows allow them (ld % 8 == 0: the last piece of
    a ragged row read element by element), element loads otherwise."""
    rng = np.random.default_rng(3 + V)
    rows = 7
    x, _ = rand_bf16(rng, (rows, V))
    hi = V - 1
    x[1, min(100, hi)] = x[1, min(500, hi - 1)] = 50.0
    x[2, :] = np.nan
    x[3, :] = -np.inf
    x[4, 7] = np.nan
    x[4, 9] = 60.0
    x[5, :] = -1.0
    x[5, 10] = -0.0
    x[5, 11] = 0.0
    x[6, hi] = 70.0
    xp = np.zeros((rows, ld), np.float32)
    xp[:, :V] = x
    xpb = hai.bf16_bits(xp)
    d, o = dev(xpb), out_buf(rows * 8)
    scratch = out_buf(kern().hai_argmax_scratch_bytes(rows, V))
    hai.check(kern().hai_argmax_rows_bf16(o.ptr, d.ptr, ld, rows, V, scratch.ptr, None), "argmax")
    got = o.download(np.int64)
    want = orc.argmax_rows(hai.bf16_to_f32(xpb).reshape(rows, ld)[:, :V].copy())
    assert list(got) == list(want)
    assert got[2] == 0 and got[3] == 0 and got[4] == 9 and got[5] == 10 and got[6] == hi
    assert got[1] == min(min(100, hi), min(500, hi - 1))  # the first of the two maxima


def test_draft_chain_count_kernel():
    """hai_draft_chain_count over a width-3 round: a chain counts its drafts
    up to its cap, keeps an EOS candidate and stops after it
    (generator.cc:845-847); the last draft's candidate is never checked and a
    cap of 0 counts nothing."""
    EOS = [900, 901]
    T = 4  # next_target + 3 drafts
    vids = np.array([[5, 10, 11, 12],     # no EOS: 3
                     [5, 10, 11, 12],     # cap 0: 0
                     [5, 900, 11, 12],    # first draft EOS: 1
                     [5, 10, 901, 12],    # second draft EOS: 2
                     [5, 10, 11, 12],     # cap 2: 2
                     [5, 10, 11, 900]],   # last draft EOS: 3
                    np.int64)
    cap = np.array([3, 0, 3, 3, 2, 3], np.int32)
    B = len(cap)
    dv, dc, de = dev(vids), dev(cap), dev(np.array(EOS, np.int64))
    for eos_ptr, n_eos, want in ((de.ptr, 2, [3, 0, 1, 2, 2, 3]), (None, 0, [3, 0, 3, 3, 2, 3])):
        dn = dev(np.full(B, 7, np.int32))  # stale counts of an earlier round
        for i in range(3):
            hai.check(kern().hai_draft_chain_count(i, dv.ptr, T, dc.ptr, eos_ptr, n_eos, dn.ptr, B, None), "count")
        assert list(dn.download(np.int32)) == want
    with pytest.raises(hai.HaiError, match="draft_chain_count"):
        hai.check(kern().hai_draft_chain_count(3, dv.ptr, T, dc.ptr, de.ptr, 2, dn.ptr, B, None), "count")


def test_verify_accept_kernel():
    rng = np.random.default_rng(9)
    T, V, H = 4, 1000, 64
    x, xb = rand_bf16(rng, (T, V))
    preds = orc.argmax_rows(x)
    hid, hb = rand_bf16(rng, (T, H))
    for a_expect in range(T):
        ids = np.array([17] + [int(p) for p in preds[:T - 1]], np.int64)
        if a_expect < T - 1:
            ids[1 + a_expect] = (ids[1 + a_expect] + 1) % V
        dl, dh, di = dev(xb), dev(hb), dev(ids)
        dp, dres, dnext = out_buf(T * 8), out_buf(16), out_buf(8)
        tl, ml = dev(np.array([100], np.int32)), dev(np.array([50], np.int32))
        rec, hp = out_buf(H * 2), out_buf(H * 2)
        scratch = out_buf(kern().hai_argmax_scratch_bytes(T, V))
        hai.check(kern().hai_verify_argmax_accept_bf16(dl.ptr, V, dh.ptr, H, di.ptr, None, 1, T, dp.ptr, dres.ptr,
                                                       tl.ptr, ml.ptr, dnext.ptr, rec.ptr, hp.ptr, scratch.ptr,
                                                       None), "accept")
        res = dres.download(np.int32)
        a, full = int(res[0]), int(res[1])
        assert a == a_expect and full == int(a_expect == T - 1)
        assert list(dp.download(np.int64)) == list(preds)
        assert int(tl.download(np.int32)[0]) == 100 + a + 1
        assert int(ml.download(np.int32)[0]) == 50 - (0 if full else (T - 1 - a))
        assert int(dnext.download(np.int64)[0]) == int(preds[a])
        assert np.array_equal(rec.download(np.uint16), hb[a])
        if full:
            assert np.array_equal(hp.download(np.uint16), hb[T - 1])


# ----------------------------------------------------------------- synthetic weights
def test_fill_synthetic_matches_oracle():
    m = orc.Model(orc.TINY, seed=0)
    for tid, shape in [(orc.tensor_id(0, 0), (4096, 256)), (orc.tensor_id(2, 2), (768, 256)),
                       (orc.tensor_id(5, 11), (512, 256)), (orc.tensor_id(1, 0), (256, 512))]:
        want = m.tensor(tid).reshape(shape)
        rows, cols = shape
        ld = cols + 8
        d = out_buf(rows * ld * 2)
        hai.check(kern().hai_fill_synthetic_bf16(d.ptr, rows, cols, ld, 0, tid, 0.02, None), "fill")
        got = d.download(np.uint16).reshape(rows, ld)[:, :cols]
        assert_bits_equal(got, want, f"tensor {tid}")


# ----------------------------------------------------------------- Backend-contract launchers
@pytest.mark.parametrize("T,heads,D,R,pos0", [(3, 4, 64, 16, 0), (5, 6, 256, 64, 1000), (1, 2, 128, 128, 7)])
def test_partial_rope(T, heads, D, R, pos0):
    rng = np.random.default_rng(T * 100 + D + pos0)
    x, xb = rand_bf16(rng, (T * heads, D))
    npos = pos0 + T + 3
    cs, sn = orc.rope_table(0, npos, R, 1.0e7)
    dx, dy = dev(xb), out_buf(xb.nbytes)
    dc, ds = dev(cs.astype(np.float32)), dev(sn.astype(np.float32))
    hai.check(kern().hai_partial_rope_bf16(dy.ptr, dx.ptr, T, heads, D, R, dc.ptr, ds.ptr, npos, pos0, None),
              "partial_rope")
    want = orc.partial_rope(x, T, heads, D, R, pos0, 1.0e7, round_out=True)
    assert_bits_equal(dy.download(np.uint16), want, "partial_rope")
    # positions past the table are rejected before launch
    assert kern().hai_partial_rope_bf16(dy.ptr, dx.ptr, T, heads, D, R, dc.ptr, ds.ptr, npos, npos - T + 1,
                                        None) == hai.ERR_INVALID


@pytest.mark.parametrize("nk,nv,dk,Kc,T", [(4, 4, 64, 4, 5), (16, 48, 128, 4, 2), (2, 4, 64, 3, 1)])
def test_deltanet_conv_reference_layout(nk, nv, dk, Kc, T):
    rng = np.random.default_rng(nk + nv + T)
    dv = dk
    C = 2 * nk * dk + nv * dv
    qkv, qkvb = rand_bf16(rng, (T, C))
    w, wb = rand_bf16(rng, (C, Kc), 0.5)
    st, stb = rand_bf16(rng, (C, Kc - 1))
    dq, dk_, dvv = out_buf(T * nk * dk * 2), out_buf(T * nk * dk * 2), out_buf(T * nv * dv * 2)
    dst, dqkv, dw = dev(stb), dev(qkvb), dev(wb)
    hai.check(kern().hai_deltanet_conv_bf16(dq.ptr, dk_.ptr, dvv.ptr, dst.ptr, dqkv.ptr, dw.ptr, T, nk, nv, dk,
                                            dv, Kc, None), "deltanet_conv")
    q, k, v, st2 = orc.deltanet_conv(qkv, w, st, T, nk, nv, dk, dv, Kc)
    assert_bits_equal(dq.download(np.uint16), q, "conv q")
    assert_bits_equal(dk_.download(np.uint16), k, "conv k")
    assert_bits_equal(dvv.download(np.uint16), v, "conv v")
    assert_bits_equal(dst.download(np.uint16), st2, "conv state")


@pytest.mark.parametrize("nk,nv,dk,T", [(4, 4, 64, 3), (2, 6, 128, 21), (16, 48, 128, 4)])  # last: C2 shape
def test_deltanet_recurrent_reference_layout(nk, nv, dk, T):
    """State [nv][dk][dv] updated in place; T > 16 runs as chained launches."""
    rng = np.random.default_rng(nk * 10 + T)
    dv = dk
    q, qb = rand_bf16(rng, (T, nk * dk))
    k, kb = rand_bf16(rng, (T, nk * dk))
    v, vb = rand_bf16(rng, (T, nv * dv))
    a, ab = rand_bf16(rng, (T, nv))
    b, bb = rand_bf16(rng, (T, nv))
    z, zb = rand_bf16(rng, (T, nv * dv))
    al, alb = rand_bf16(rng, (nv,), 0.5)
    dt, dtb = rand_bf16(rng, (nv,), 0.5)
    nw, nwb = rand_bf16(rng, (dv,), 0.1)
    state = (rng.standard_normal((nv, dk, dv)) * 0.1).astype(np.float32)
    dbufs = [dev(t) for t in (qb, kb, vb, ab, bb, alb, dtb, nwb, zb)]
    dstate, dout = dev(state), out_buf(T * nv * dv * 2)
    hai.check(kern().hai_deltanet_recurrent_bf16(dout.ptr, dstate.ptr, *[d.ptr for d in dbufs], T, nk, nv, dk, dv,
                                                 1e-6, None), "deltanet_recurrent")
    out, st2 = orc.deltanet_recurrent(q, k, v, a, b, z, al, dt, nw, state, T, nk, nv, dk, dv)
    assert_bits_equal(dout.download(np.uint16), out, "recurrent out")
    got_state = dstate.download(np.float32).reshape(st2.shape)
    assert np.array_equal(got_state.view(np.uint32), st2.view(np.uint32)), "recurrent state"


# ----------------------------------------------------------------- FP8 weights
def _fp8_weights(rng, N, K, nan_codes=False):
    """Block-scaled E4M3 weights as the C5 config builds them: scales
    U(0.5, 2)/448 per 128x128 block, q = clamp(round(w / s), +-448)."""
    sb = ((N + 127) // 128, (K + 127) // 128)
    s = (rng.uniform(0.5, 2.0, sb) / 448.0).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    q = orc.fp8_encode(w / np.repeat(np.repeat(s, 128, 0), 128, 1)[:N, :K])
    if nan_codes:  # the reference decodes 0x7F / 0xFF as +-480
        q.reshape(-1)[rng.choice(q.size, 64, replace=False)] = rng.choice([0x7F, 0xFF], 64)
    return q, s


@pytest.mark.parametrize("M,N,K,nan_codes", [(1, 300, 256, False), (2, 1536, 5120, True), (3, 257, 1000, True),
                                             (16, 384, 768, False), (2, 5120, 17408, False),
                                             (2, 16390, 1000, True), (1, 8200, 2056, False)])
def test_gemm_fp8_store(M, N, K, nan_codes):
    rng = np.random.default_rng(M * 31 + N + K)
    x, xb = rand_bf16(rng, (M, K))
    q, s = _fp8_weights(rng, N, K, nan_codes)
    dx, dq, ds, dy = dev(xb), dev(q), dev(s), out_buf(M * N * 2)
    hai.check(kern().hai_gemm_fp8_bf16(dy.ptr, N, dx.ptr, K, dq.ptr, ds.ptr, None, M, N, K, hai.EPI_STORE, None, 0, None),
              "gemm_fp8")
    assert_bits_equal(dy.download(np.uint16), orc.gemm_fp8(x, q, s), f"gemm_fp8 {M}x{N}x{K}")


def test_gemm_fp8_residual_and_swiglu():
    rng = np.random.default_rng(77)
    M, F, K = 2, 640, 512
    x, xb = rand_bf16(rng, (M, K))
    # residual
    q, s = _fp8_weights(rng, 300, K)
    h, hb = rand_bf16(rng, (M, 300))
    dx, dq, ds, dh = dev(xb), dev(q), dev(s), dev(hb)
    hai.check(kern().hai_gemm_fp8_bf16(dh.ptr, 300, dx.ptr, K, dq.ptr, ds.ptr, None, M, 300, K, hai.EPI_RESIDUAL, dh.ptr,
                                       300, None), "gemm_fp8 residual")
    assert_bits_equal(dh.download(np.uint16), orc.add(h, orc.gemm_fp8(x, q, s)), "gemm_fp8 residual")
    # SwiGLU over interleaved (gate_f, up_f) rows with per-matrix scale planes
    qg, sg = _fp8_weights(rng, F, K, True)
    qu, su = _fp8_weights(rng, F, K)
    qi = np.empty((2 * F, K), np.uint8)
    qi[0::2], qi[1::2] = qg, qu
    dqi, dsi, dy = dev(qi), dev(np.stack([sg, su])), out_buf(M * F * 2)
    hai.check(kern().hai_gemm_fp8_bf16(dy.ptr, F, dx.ptr, K, dqi.ptr, dsi.ptr, None, M, 2 * F, K, hai.EPI_SILU_MUL, None,
                                       0, None), "gemm_fp8 silu")
    want = orc.silu_mul(orc.gemm_fp8(x, qg, sg), orc.gemm_fp8(x, qu, su))
    assert_bits_equal(dy.download(np.uint16), want, "gemm_fp8 silu_mul")


@pytest.mark.parametrize("special", [False, True])
def test_gemm_fp8_wide_swiglu_and_no_special_codes_flag(special):
    """M = 2 over 2F >= 16384 interleaved rows (the four-rows-per-wave launch);
    with HAI_FP8_NO_SPECIAL_CODES on weights that hold no 0x7F / 0xFF the
    result is unchanged."""
    rng = np.random.default_rng(5 + special)
    M, F, K = 2, 8200, 768
    x, xb = rand_bf16(rng, (M, K))
    qg, sg = _fp8_weights(rng, F, K, special)
    qu, su = _fp8_weights(rng, F, K)
    qi = np.empty((2 * F, K), np.uint8)
    qi[0::2], qi[1::2] = qg, qu
    dx, dqi, dsi, dy = dev(xb), dev(qi), dev(np.stack([sg, su])), out_buf(M * F * 2)
    flag = 0 if special else hai.FP8_NO_SPECIAL_CODES
    hai.check(kern().hai_gemm_fp8_bf16(dy.ptr, F, dx.ptr, K, dqi.ptr, dsi.ptr, None, M, 2 * F, K,
                                       hai.EPI_SILU_MUL | flag, None, 0, None), "gemm_fp8 wide silu")
    want = orc.silu_mul(orc.gemm_fp8(x, qg, sg), orc.gemm_fp8(x, qu, su))
    assert_bits_equal(dy.download(np.uint16), want, "gemm_fp8 wide silu_mul")


def test_gemm_fp8_scale_rows_map():
    """Rows of several checkpoint tensors stacked in one launch, each tensor
    with its own 128x128 grid (row counts not multiples of 128), through the
    per-row scale map; also a sub-range of the stack (map and codes offset)."""
    rng = np.random.default_rng(91)
    K = 1000
    parts = [(200, False), (64, True), (64, False), (130, True)]
    qs, ss, mp, g0 = [], [], [], 0
    for rows, nan in parts:
        q, s = _fp8_weights(rng, rows, K, nan)
        qs.append(q); ss.append(s)
        mp.extend(g0 + r // 128 for r in range(rows))
        g0 += s.shape[0]
    q = np.concatenate(qs); s = np.concatenate(ss); mp = np.array(mp, np.int32)
    N = q.shape[0]
    want_w = np.concatenate([orc.fp8_dequant_2d(qq, sq, 128, 128) for qq, sq in zip(qs, ss)])
    dq, ds, dm = dev(q), dev(s), dev(mp)
    for M in (1, 2, 5):
        x, xb = rand_bf16(rng, (M, K))
        dx, dy = dev(xb), out_buf(M * N * 2)
        hai.check(kern().hai_gemm_fp8_bf16(dy.ptr, N, dx.ptr, K, dq.ptr, ds.ptr, dm.ptr, M, N, K, hai.EPI_STORE,
                                           None, 0, None), "gemm_fp8 map")
        assert_bits_equal(dy.download(np.uint16), orc.gemm(x, want_w), f"gemm_fp8 map M={M}")
    # rows 264.. (the third and fourth tensors) alone
    r0 = 264
    x, xb = rand_bf16(rng, (2, K))
    dx, dy = dev(xb), out_buf(2 * (N - r0) * 2)
    hai.check(kern().hai_gemm_fp8_bf16(dy.ptr, N - r0, dx.ptr, K, dq.ptr + r0 * K, ds.ptr, dm.ptr + 4 * r0, 2,
                                       N - r0, K, hai.EPI_STORE, None, 0, None), "gemm_fp8 map rows")
    assert_bits_equal(dy.download(np.uint16), orc.gemm(x, want_w[r0:]), "gemm_fp8 map rows")


@pytest.mark.parametrize("rows,cols,ldq,ldw", [(300, 200, 200, 208), (128, 1024, 2048, 1024), (1, 8, 8, 8)])
def test_fp8_quantize_matches_oracle(rows, cols, ldq, ldw):
    rng = np.random.default_rng(rows + cols)
    sb = ((rows + 127) // 128, (cols + 127) // 128)
    s = (rng.uniform(0.5, 2.0, sb) / 448.0).astype(np.float32)
    w = rng.standard_normal((rows, cols)).astype(np.float32) * 0.02
    # saturating, subnormal-range, zero and negative-zero entries
    flat = w.reshape(-1)
    flat[: min(flat.size, 6)] = [5.0, -5.0, 1e-7, -1e-7, 0.0, -0.0][: min(flat.size, 6)]
    wb = orc.f32_to_bf16_bits(w)
    wf = hai.bf16_to_f32(wb)
    wpad = np.zeros((rows, ldw), np.uint16); wpad[:, :cols] = wb
    dw, ds, dq = dev(wpad), dev(s), out_buf(rows * ldq)
    hai.check(kern().hai_fp8_quantize_bf16(dq.ptr, ldq, dw.ptr, ldw, ds.ptr, rows, cols, None), "fp8_quantize")
    got = dq.download(np.uint8).reshape(rows, ldq)[:, :cols]
    want = orc.fp8_encode(wf / np.repeat(np.repeat(s, 128, 0), 128, 1)[:rows, :cols])
    assert np.array_equal(got, want)


def test_fp8_synthetic_scales_match_oracle():
    for seed, tid, n in ((0, 2 * 64 + 17, 1000), (7, 1024 * 64 + 11, 333)):
        d = out_buf(n * 4)
        hai.check(kern().hai_fill_synthetic_scales_f32(d.ptr, n, seed, tid, None), "fill_scales")
        assert np.array_equal(d.download(np.float32), orc.fp8_synthetic_scales(seed, tid, n))


@pytest.mark.parametrize("nospecial", [False, True])
@pytest.mark.parametrize("M,N,K_,epi,with_xn,mapped", [
    (1, 700, 5120, 0, False, False), (2, 2 * 8200, 1000, 2, True, False), (2, 640, 2048, 1, False, True),
    (3, 300, 5120, 0, True, False), (16, 256, 1024, 2, False, False), (2, 16400, 768, 0, True, True),
    (2, 2 * 8200, 5120, 2, False, False),  # four rows per wave, five whole chunk groups
    (2, 1000, 3384, 0, False, False),      # three whole groups, then a ragged chunk
    (1, 700, 1024, 1, False, False)])      # one whole group
def test_gemm_rmsnorm_fp8_fused(M, N, K_, epi, with_xn, mapped, nospecial):
    """hai_gemm_rmsnorm_fp8_bf16 == rmsnorm then the FP8 GEMM (LDS prologue
    below the fused limit, two kernels above it), with and without a
    per-row scale map (two stacked tensors, the second starting mid-block).
    The saturating quantiser writes no 0x7F / 0xFF, so the same weights also
    run with HAI_FP8_NO_SPECIAL_CODES (whose fused launches request the next
    chunk group's codes before computing the current one)."""
    rng = np.random.default_rng(131 + M * 7 + N + K_ + epi)
    x, xb = rand_bf16(rng, (M, K_))
    nw, nwb = rand_bf16(rng, (K_,), 0.02)
    xn_want = orc.rmsnorm(x, nw, 1e-6, True)
    if epi == hai.EPI_SILU_MUL:
        F = N // 2
        qg, sg = _fp8_weights(rng, F, K_)
        qu, su = _fp8_weights(rng, F, K_)
        q = np.empty((N, K_), np.uint8)
        q[0::2], q[1::2] = qg, qu
        s = np.stack([sg, su])
        y_lin = None
        want_lin = orc.silu_mul(orc.gemm_fp8(xn_want, qg, sg), orc.gemm_fp8(xn_want, qu, su))
        mp = None
    elif mapped:
        n0 = N // 2 + 64
        q0, s0 = _fp8_weights(rng, n0, K_)
        q1, s1 = _fp8_weights(rng, N - n0, K_)
        q, s = np.concatenate([q0, q1]), np.concatenate([s0, s1])
        mp = np.array([r // 128 for r in range(n0)] + [s0.shape[0] + r // 128 for r in range(N - n0)], np.int32)
        y_lin = np.concatenate([orc.gemm_fp8(xn_want, q0, s0), orc.gemm_fp8(xn_want, q1, s1)], axis=1)
    else:
        q, s = _fp8_weights(rng, N, K_)
        mp = None
        y_lin = orc.gemm_fp8(xn_want, q, s)
    ncols = N // 2 if epi == hai.EPI_SILU_MUL else N
    need_xn = with_xn or M * K_ > 16384
    dx, dnw, dq, ds = dev(xb), dev(nwb), dev(q), dev(s)
    dm = dev(mp) if mp is not None else None
    dxn = out_buf(M * K_ * 2) if need_xn else None
    h, hb = rand_bf16(rng, (M, ncols))
    dy = dev(hb) if epi == hai.EPI_RESIDUAL else out_buf(M * ncols * 2)
    hai.check(kern().hai_gemm_rmsnorm_fp8_bf16(dy.ptr, ncols, dx.ptr, K_, dnw.ptr, 1e-6, 1,
                                               dxn.ptr if dxn else None, K_, dq.ptr, ds.ptr,
                                               dm.ptr if dm else None, M, N, K_,
                                               epi | (hai.FP8_NO_SPECIAL_CODES if nospecial else 0),
                                               dy.ptr if epi == hai.EPI_RESIDUAL else None, ncols, None),
              "gemm_rmsnorm_fp8")
    if epi == hai.EPI_STORE:
        want = y_lin
    elif epi == hai.EPI_RESIDUAL:
        want = orc.add(h, y_lin)
    else:
        want = want_lin
    assert_bits_equal(dy.download(np.uint16), want, f"gemm_rmsnorm_fp8 {M}x{N}x{K_} epi {epi}")
    if dxn is not None:
        assert_bits_equal(dxn.download(np.uint16), xn_want, "normalised rows")


# ----------------------------------------------------------------- MFMA (tolerance mode)
@pytest.mark.parametrize("M,N,K,epi,with_ws", [(17, 300, 256, 0, True), (32, 1536, 5120, 1, True),
                                               (64, 1000, 1000, 2, True), (128, 640, 2048, 0, False),
                                               (40, 16480, 512, 0, True), (33, 2050, 2056, 2, True),
                                               (32, 1536, 5120, 1, False), (96, 5120, 6144, 1, True)])
def test_gemm_mfma_within_tolerance(M, N, K, epi, with_ws):
    """hai_gemm_bf16_mfma against the canonical GEMM: the bf16 outputs differ
    by at most a couple of bf16 ulps (fp32 accumulation in another order)."""
    rng = np.random.default_rng(M + N + K + epi)
    x, xb = rand_bf16(rng, (M, K))
    w, wb = rand_bf16(rng, (N, K), 0.05)
    ncols = N // 2 if epi == hai.EPI_SILU_MUL else N
    h, hb = rand_bf16(rng, (M, ncols))
    dx, dw = dev(xb), dev(wb)
    dy = dev(hb) if epi == hai.EPI_RESIDUAL else out_buf(M * ncols * 2)
    wsb = kern().hai_gemm_mfma_workspace_bytes(M, N)
    dws = out_buf(max(wsb, 16)) if with_ws else None
    hai.check(kern().hai_gemm_bf16_mfma(dy.ptr, ncols, dx.ptr, K, dw.ptr, M, N, K, epi,
                                        dy.ptr if epi == hai.EPI_RESIDUAL else None, ncols,
                                        dws.ptr if dws else None, wsb if dws else 0, None), "gemm_mfma")
    y = orc.gemm(x, w)
    if epi == hai.EPI_STORE:
        want = y
    elif epi == hai.EPI_RESIDUAL:
        want = orc.add(h, y)
    else:
        want = orc.silu_mul(y[:, 0::2], y[:, 1::2])
    got = hai.bf16_to_f32(dy.download(np.uint16).reshape(M, ncols))
    exact64 = x.astype(np.float64) @ w.astype(np.float64).T
    scale = np.abs(exact64).max()
    assert np.allclose(got, want, rtol=2 ** -6, atol=2e-3 * scale), float(np.abs(got - want).max())
    if epi == hai.EPI_STORE:
        assert np.abs(got - exact64).max() <= 2 ** -7 * np.abs(exact64).max() + 1e-6


@pytest.mark.parametrize("M,N,K,epi,mapped,special", [(32, 1536, 5120, 0, False, True), (64, 2 * 640, 1024, 2, False, False),
                                                      (17, 700, 1008, 1, True, False), (128, 5120, 2048, 1, False, False),
                                                      (48, 16400, 512, 0, True, True),
                                                      (40, 2000, 2048, 1, True, True), (24, 4096, 1536, 2, False, False),
                                                      (40, 9000, 1024, 0, True, True), (20, 12000, 768, 1, False, True),
                                                      (24, 8320, 256, 2, False, False)])
def test_gemm_fp8_mfma_within_tolerance(M, N, K, epi, mapped, special):
    """hai_gemm_fp8_mfma against the canonical FP8 GEMM (dequantised weights,
    fp32 dot): bf16 outputs within a couple of bf16 ulps; 0x7F / 0xFF codes
    decode to +-480 as in the reference."""
    rng = np.random.default_rng(7 * M + N + K + epi)
    x, xb = rand_bf16(rng, (M, K))
    if epi == hai.EPI_SILU_MUL:
        F = N // 2
        qg, sg = _fp8_weights(rng, F, K, special)
        qu, su = _fp8_weights(rng, F, K)
        q = np.empty((N, K), np.uint8)
        q[0::2], q[1::2] = qg, qu
        s, mp = np.stack([sg, su]), None
        y_lin = None
        want = orc.silu_mul(orc.gemm_fp8(x, qg, sg), orc.gemm_fp8(x, qu, su))
        ncols = F
    else:
        if mapped:
            n0 = N // 2 + 64
            q0, s0 = _fp8_weights(rng, n0, K, special)
            q1, s1 = _fp8_weights(rng, N - n0, K)
            q, s = np.concatenate([q0, q1]), np.concatenate([s0, s1])
            mp = np.array([r // 128 for r in range(n0)] + [s0.shape[0] + r // 128 for r in range(N - n0)], np.int32)
            y_lin = np.concatenate([orc.gemm_fp8(x, q0, s0), orc.gemm_fp8(x, q1, s1)], axis=1)
        else:
            q, s = _fp8_weights(rng, N, K, special)
            mp = None
            y_lin = orc.gemm_fp8(x, q, s)
        ncols = N
        h, hb = rand_bf16(rng, (M, N))
        want = y_lin if epi == hai.EPI_STORE else orc.add(h, y_lin)
    dx, dq, ds = dev(xb), dev(q), dev(s)
    dm = dev(mp) if mp is not None else None
    dy = dev(hb) if epi == hai.EPI_RESIDUAL else out_buf(M * ncols * 2)
    wsb = kern().hai_gemm_mfma_workspace_bytes(M, N)
    dws = out_buf(max(wsb, 16))
    flag = 0 if special else hai.FP8_NO_SPECIAL_CODES
    hai.check(kern().hai_gemm_fp8_mfma(dy.ptr, ncols, dx.ptr, K, dq.ptr, ds.ptr, dm.ptr if dm else None, M, N, K,
                                       epi | flag, dy.ptr if epi == hai.EPI_RESIDUAL else None, ncols, dws.ptr, wsb,
                                       None), "gemm_fp8_mfma")
    got = hai.bf16_to_f32(dy.download(np.uint16).reshape(M, ncols))
    scale = np.abs(want).max()
    assert np.allclose(got, want, rtol=2 ** -6, atol=2e-3 * scale), float(np.abs(got - want).max())


@pytest.mark.parametrize("M,N,K,epi", [(32, 34816, 5120, 2), (32, 5120, 17408, 1), (64, 16480, 5120, 0)])
def test_gemm_mfma_27b_shapes(M, N, K, epi):
    """The batched-verify GEMMs at their C4 (M = 8 sequences x 4 rows) and C5
    (M = 32 x 2) shapes: gate/up with SwiGLU, down with the residual add,
    DeltaNet in_proj; within tolerance of the canonical oracle GEMM."""
    rng = np.random.default_rng(N + K)
    x, xb = rand_bf16(rng, (M, K))
    w, wb = rand_bf16(rng, (N, K), 0.02)
    ncols = N // 2 if epi == hai.EPI_SILU_MUL else N
    h, hb = rand_bf16(rng, (M, ncols))
    dx, dw = dev(xb), dev(wb)
    dy = dev(hb) if epi == hai.EPI_RESIDUAL else out_buf(M * ncols * 2)
    wsb = kern().hai_gemm_mfma_workspace_bytes(M, N)
    dws = out_buf(max(wsb, 16))
    hai.check(kern().hai_gemm_bf16_mfma(dy.ptr, ncols, dx.ptr, K, dw.ptr, M, N, K, epi,
                                        dy.ptr if epi == hai.EPI_RESIDUAL else None, ncols, dws.ptr, wsb, None),
              "gemm_mfma 27b")
    y = orc.gemm(x, w)
    want = {hai.EPI_STORE: lambda: y, hai.EPI_RESIDUAL: lambda: orc.add(h, y),
            hai.EPI_SILU_MUL: lambda: orc.silu_mul(y[:, 0::2], y[:, 1::2])}[epi]()
    got = hai.bf16_to_f32(dy.download(np.uint16).reshape(M, ncols))
    scale = np.abs(want).max()
    assert np.allclose(got, want, rtol=2 ** -6, atol=2e-3 * scale), float(np.abs(got - want).max())


@pytest.mark.parametrize("M,N,K,epi", [(64, 34816, 5120, 2), (64, 5120, 17408, 1), (64, 16384, 5120, 0),
                                       (64, 14336, 5120, 0), (32, 14336, 5120, 0)])
def test_gemm_fp8_mfma_27b_shapes(M, N, K, epi):
    """The C5 batched-verify GEMMs (32 sequences x 2 rows, FP8 E4M3 weights
    with 128x128 scales): gate/up with SwiGLU over paired scale grids, down
    with the residual add, DeltaNet in_proj qkv|z; within tolerance of the
    oracle's FP8 GEMM (decode(q) * s, canonical fp32 dot)."""
    rng = np.random.default_rng(N + K + 64)
    x, xb = rand_bf16(rng, (M, K))
    if epi == hai.EPI_SILU_MUL:
        F = N // 2
        qg, sg = _fp8_weights(rng, F, K)
        qu, su = _fp8_weights(rng, F, K)
        q = np.empty((N, K), np.uint8)
        q[0::2], q[1::2] = qg, qu
        s = np.stack([sg, su])
        want = orc.silu_mul(orc.gemm_fp8(x, qg, sg), orc.gemm_fp8(x, qu, su))
        ncols = F
    else:
        q, s = _fp8_weights(rng, N, K)
        ncols = N
        h, hb = rand_bf16(rng, (M, N))
        y = orc.gemm_fp8(x, q, s)
        want = y if epi == hai.EPI_STORE else orc.add(h, y)
    dx, dq, ds = dev(xb), dev(q), dev(s)
    dy = dev(hb) if epi == hai.EPI_RESIDUAL else out_buf(M * ncols * 2)
    wsb = kern().hai_gemm_mfma_workspace_bytes(M, N)
    dws = out_buf(max(wsb, 16))
    hai.check(kern().hai_gemm_fp8_mfma(dy.ptr, ncols, dx.ptr, K, dq.ptr, ds.ptr, None, M, N, K,
                                       epi | hai.FP8_NO_SPECIAL_CODES, dy.ptr if epi == hai.EPI_RESIDUAL else None,
                                       ncols, dws.ptr, wsb, None), "gemm_fp8_mfma 27b")
    got = hai.bf16_to_f32(dy.download(np.uint16).reshape(M, ncols))
    scale = np.abs(want).max()
    assert np.allclose(got, want, rtol=2 ** -6, atol=2e-3 * scale), float(np.abs(got - want).max())


@pytest.mark.parametrize("M,N,K,fp8", [(32, 5120, 6144, False), (64, 5120, 17408, True), (17, 1536, 4096, False),
                                       (128, 5120, 2048, True)])
def test_mfma_keep_partials_then_residual_rmsnorm(M, N, K, fp8):
    """A residual MFMA GEMM that keeps its K-split partials, completed by
    hai_mfma_residual_rmsnorm_bf16, equals the unfused call bit for bit, and
    its normalised rows equal hai_rmsnorm_bf16 of them; without a norm weight
    only the residual rows are written."""
    rng = np.random.default_rng(M + N + K + fp8)
    x, xb = rand_bf16(rng, (M, K))
    h0, hb = rand_bf16(rng, (M, N))
    nw, nwb = rand_bf16(rng, (N,), 0.02)
    if fp8:
        q, s = _fp8_weights(rng, N, K)
        dq, ds = dev(q), dev(s)
    else:
        w, wb = rand_bf16(rng, (N, K), 0.02)
        dw = dev(wb)
    dx, dnw = dev(xb), dev(nwb)
    wsb = kern().hai_gemm_mfma_workspace_bytes(M, N)
    dws = out_buf(max(wsb, 16))
    splits = kern().hai_gemm_mfma_splits(M, N, K, dws.ptr, wsb)
    assert splits > 1

    def gemm(dh, flags):
        if fp8:
            return kern().hai_gemm_fp8_mfma(dh.ptr, N, dx.ptr, K, dq.ptr, ds.ptr, None, M, N, K,
                                            hai.EPI_RESIDUAL | hai.FP8_NO_SPECIAL_CODES | flags, dh.ptr, N,
                                            dws.ptr, wsb, None)
        return kern().hai_gemm_bf16_mfma(dh.ptr, N, dx.ptr, K, dw.ptr, M, N, K, hai.EPI_RESIDUAL | flags, dh.ptr, N,
                                         dws.ptr, wsb, None)

    ref_h, ref_xn = dev(hb), out_buf(M * N * 2)
    hai.check(gemm(ref_h, 0), "unfused gemm")
    hai.check(kern().hai_rmsnorm_bf16(ref_xn.ptr, N, ref_h.ptr, N, dnw.ptr, M, N, 1e-6, 1, None), "rmsnorm")
    dh, dxn = dev(hb), out_buf(M * N * 2)
    hai.check(gemm(dh, hai.MFMA_KEEP_PARTIALS), "gemm keeping partials")
    hai.check(kern().hai_mfma_residual_rmsnorm_bf16(dh.ptr, N, dws.ptr, wsb, M, N, splits, dnw.ptr, 1e-6, 1, dxn.ptr,
                                                    N, None), "residual rmsnorm")
    assert_bits_equal(dh.download(np.uint16), hai.bf16_to_f32(ref_h.download(np.uint16)), "residual rows")
    assert_bits_equal(dxn.download(np.uint16), hai.bf16_to_f32(ref_xn.download(np.uint16)), "normalised rows")
    dh2 = dev(hb)
    hai.check(gemm(dh2, hai.MFMA_KEEP_PARTIALS), "gemm keeping partials")
    hai.check(kern().hai_mfma_residual_rmsnorm_bf16(dh2.ptr, N, dws.ptr, wsb, M, N, splits, None, 0.0, 0, None, 0,
                                                    None), "residual only")
    assert_bits_equal(dh2.download(np.uint16), hai.bf16_to_f32(ref_h.download(np.uint16)), "residual rows, no norm")
    # keeping partials is for the residual epilogue only (operands sized for
    # the call, so even an accepted call would stay in bounds)
    if not fp8:
        for epi, ldy in ((hai.EPI_STORE, N), (hai.EPI_SILU_MUL, N // 2)):
            assert kern().hai_gemm_bf16_mfma(dh.ptr, ldy, dx.ptr, K, dw.ptr, M, N, K, epi | hai.MFMA_KEEP_PARTIALS,
                                             None, 0, dws.ptr, wsb, None) == hai.ERR_INVALID


@pytest.mark.parametrize("M,N,K,fp8", [(32, 5120, 6144, False), (32, 5120, 17408, False), (64, 5120, 17408, True),
                                       (17, 1536, 4096, False), (128, 5120, 2048, True)])
def test_mfma_fp32_accumulators_within_1e3(M, N, K, fp8):
    """The matrix-core GEMMs' fp32 accumulation, read directly: a residual
    GEMM that keeps its K-split partials leaves splits planes of fp32 sums in
    the workspace; their sum (in float64) is the GEMM's fp32-accumulated
    x . w before any bf16 rounding, and must be within 1e-3 of the float64
    product: |acc - exact| <= 1e-3 * max(|exact|, rms of the output row / 10).
    FP8 weights: w = decode(q) * s per 128 x 128 block (the scale applied per
    block in fp32 inside the kernel)."""
    rng = np.random.default_rng(3 * M + N + K + fp8)
    x, xb = rand_bf16(rng, (M, K))
    zeros = np.zeros((M, N), np.uint16)
    if fp8:
        q, s = _fp8_weights(rng, N, K)
        dq, ds = dev(q), dev(s)
        w64 = orc.fp8_dequant_2d(q, s, 128, 128).astype(np.float64)
    else:
        w, wb = rand_bf16(rng, (N, K), 0.02)
        dw = dev(wb)
        w64 = w.astype(np.float64)
    dx, dh = dev(xb), dev(zeros)
    wsb = kern().hai_gemm_mfma_workspace_bytes(M, N)
    dws = out_buf(max(wsb, 16))
    splits = kern().hai_gemm_mfma_splits(M, N, K, dws.ptr, wsb)
    assert splits > 1
    if fp8:
        rc = kern().hai_gemm_fp8_mfma(dh.ptr, N, dx.ptr, K, dq.ptr, ds.ptr, None, M, N, K,
                                      hai.EPI_RESIDUAL | hai.FP8_NO_SPECIAL_CODES | hai.MFMA_KEEP_PARTIALS, dh.ptr, N,
                                      dws.ptr, wsb, None)
    else:
        rc = kern().hai_gemm_bf16_mfma(dh.ptr, N, dx.ptr, K, dw.ptr, M, N, K, hai.EPI_RESIDUAL | hai.MFMA_KEEP_PARTIALS,
                                       dh.ptr, N, dws.ptr, wsb, None)
    hai.check(rc, "gemm keeping partials")
    planes = dws.download(np.float32)[: splits * M * N].reshape(splits, M, N).astype(np.float64)
    acc = planes.sum(0)
    exact = x.astype(np.float64) @ w64.T
    rms_row = np.sqrt(np.mean(exact ** 2, axis=1, keepdims=True))
    err = np.abs(acc - exact) / np.maximum(np.abs(exact), rms_row / 10)
    assert np.isfinite(acc).all()
    assert err.max() <= 1e-3, f"fp32 accumulators: max relative error {err.max():.2e}"
    # the planes are real partial sums, not one full sum and zeros
    assert np.abs(planes[1]).max() > 0


@pytest.mark.gpu
def test_operand_bounds_check():
    """The host-side check the launchers run under HAI_CHECK_BOUNDS (set for
    the whole test session): ranges inside an allocation pass, ranges that
    run past its end do not.  Nothing is launched."""
    import os
    assert os.environ.get("HAI_CHECK_BOUNDS") == "1"
    b = hai.DeviceBuffer(1 << 20)
    assert kern().hai_debug_check_extent(b.ptr, 1 << 20) == hai.OK
    assert kern().hai_debug_check_extent(b.ptr + 4096, (1 << 20) - 4096) == hai.OK
    assert kern().hai_debug_check_extent(b.ptr, 1 << 30) == hai.ERR_INVALID
    assert kern().hai_debug_check_extent(b.ptr + (1 << 19), 1 << 29) == hai.ERR_INVALID


@pytest.mark.gpu
def test_residual_rmsnorm_rejects_workspace_and_split_mistakes():
    """hai_mfma_residual_rmsnorm_bf16 refuses, before launching, a workspace
    smaller than splits * M * N floats and a split count of one (the GEMM
    then finished its rows itself and left no partials)."""
    M, N = 8, 1024
    h, ws = out_buf(M * N * 2), out_buf(4 * M * N * 4)
    k = kern()
    assert k.hai_mfma_residual_rmsnorm_bf16(h.ptr, N, ws.ptr, 3 * M * N * 4 - 4, M, N, 3, None, 0.0, 0, None, 0,
                                            None) == hai.ERR_INVALID
    assert k.hai_mfma_residual_rmsnorm_bf16(h.ptr, N, ws.ptr, 4 * M * N * 4, M, N, 1, None, 0.0, 0, None, 0,
                                            None) == hai.ERR_INVALID
    assert k.hai_mfma_residual_rmsnorm_bf16(h.ptr, N, ws.ptr, 4 * M * N * 4, M, N, 5, None, 0.0, 0, None, 0,
                                            None) == hai.ERR_INVALID


@pytest.mark.parametrize("H,nk,nv,dk,dv,B,T", [(256, 4, 4, 64, 64, 1, 2), (256, 2, 6, 64, 64, 3, 16),
                                               (5120, 16, 48, 128, 128, 1, 2), (5120, 16, 48, 128, 128, 4, 4),
                                               (1000, 4, 4, 64, 64, 2, 3)])
def test_deltanet_verify_ab_matches_projection_then_kernel(H, nk, nv, dk, dv, B, T):
    """hai_deltanet_verify_ab_bf16 forms the in_proj_a|b Linear of each head
    itself: outputs, every state slot and the conv ring must equal running
    that Linear with hai_gemm_bf16 into the proj columns (pinned to the
    oracle by the GEMM tests) and then hai_deltanet_verify_bf16."""
    rng = np.random.default_rng(H + nv + B * 10 + T)
    c = _deltanet_case(rng, B, nk, nv, dk, dv)
    C, Kc = c["C"], c["Kc"]
    vw = nv * dv
    width = C + vw + 2 * nv
    ring, nslots = 32, 17
    rows = B * T
    _, xnb = rand_bf16(rng, (rows, H))
    _, wab = rand_bf16(rng, (2 * nv, H), 0.05)
    _, pb = rand_bf16(rng, (rows, width))
    dcw, dal, ddt, dnw = dev(c["cwb"]), dev(c["alb"]), dev(c["dtb"]), dev(c["nwb"])
    dxn, dwab = dev(xnb), dev(wab)
    lens = dev(np.array([5 + 3 * b for b in range(B)], np.int32))
    res = []
    for mode in ("gemm", "ab"):
        dproj = dev(pb)
        dring = dev(rng.integers(0, 1 << 16, B * ring * C, dtype=np.uint16) * 0 + np.uint16(0x3f80))
        dstate = dev(np.full(nslots * B * nv * dk * dv, 0.25, np.float32))
        dout = out_buf(rows * vw * 2)
        if mode == "gemm":
            for m0 in range(0, rows, 16):  # the skinny GEMM takes 16 rows per call
                hai.check(kern().hai_gemm_bf16(dproj.ptr + ((C + vw) + m0 * width) * 2, width, dxn.ptr + m0 * H * 2,
                                               H, dwab.ptr, min(16, rows - m0), 2 * nv, H, hai.EPI_STORE, None, 0,
                                               None), "a|b gemm")
            hai.check(kern().hai_deltanet_verify_bf16(dout.ptr, vw, dproj.ptr, width, 0, C, C + vw, C + vw + nv,
                                                      dcw.ptr, dring.ptr, ring, dstate.ptr, nslots, 1, dal.ptr,
                                                      ddt.ptr, dnw.ptr, lens.ptr, 0, B, T, nk, nv, dk, dv, Kc, 1e-6,
                                                      None), "deltanet")
        else:
            hai.check(kern().hai_deltanet_verify_ab_bf16(dout.ptr, vw, dproj.ptr, width, 0, C, dxn.ptr, H, dwab.ptr,
                                                         H, dcw.ptr, dring.ptr, ring, dstate.ptr, nslots, 1, dal.ptr,
                                                         ddt.ptr, dnw.ptr, lens.ptr, 0, B, T, nk, nv, dk, dv, Kc,
                                                         1e-6, None), "deltanet_ab")
        res.append([dout.download(np.uint16), dstate.download(np.uint32), dring.download(np.uint16)])
    for name, g, w in zip(("out", "state", "ring"), res[1], res[0]):
        np.testing.assert_array_equal(g, w, err_msg=name)


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("M,N,K,epi", [(64, 34816, 5120, 2), (32, 34816, 5120, 0), (40, 33800, 5000, 1),
                                       (64, 33792, 2048, 0)])
def test_gemm_mfma_stream_k_matches_plain_grid(fp8, M, N, K, epi):
    """Shapes just past a whole number of tiles per CU take the stream-K
    split (two partial planes for the tiles two blocks share): the result is
    deterministic and equals the plain grid (no workspace) up to fp32
    regrouping of the K sum, whose error (~1e-7 of the partial sums) is many
    bf16 ulps only for outputs that cancel to near zero.  The FP8 kernels
    read codes in 16-byte groups: K % 16 != 0 is rejected on the host before
    any launch, and the output stays untouched."""
    rng = np.random.default_rng(N + K + M + epi)
    x, xb = rand_bf16(rng, (M, K))
    ncols = N // 2 if epi == hai.EPI_SILU_MUL else N
    _, hb = rand_bf16(rng, (M, ncols))
    dx = dev(xb)
    if fp8:
        if epi == hai.EPI_SILU_MUL:
            qg, sg = _fp8_weights(rng, N // 2, K)
            qu, su = _fp8_weights(rng, N // 2, K)
            q = np.empty((N, K), np.uint8)
            q[0::2], q[1::2] = qg, qu
            s = np.stack([sg, su])
        else:
            q, s = _fp8_weights(rng, N, K)
        dq, ds = dev(q), dev(s)
    else:
        _, wb = rand_bf16(rng, (N, K), 0.02)
        dw = dev(wb)
    wsb = kern().hai_gemm_mfma_workspace_bytes(M, N)
    dws = out_buf(max(wsb, 16))
    if fp8 and K % 16:
        dy = dev(hb)
        with pytest.raises(hai.HaiError, match=r"K % 16 != 0"):
            hai.check(kern().hai_gemm_fp8_mfma(dy.ptr, ncols, dx.ptr, K, dq.ptr, ds.ptr, None, M, N, K,
                                               epi | hai.FP8_NO_SPECIAL_CODES, dy.ptr, ncols, dws.ptr, wsb, None),
                      "fp8 mfma")
        np.testing.assert_array_equal(dy.download(np.uint16).reshape(M, ncols), hb)
        return
    outs = []
    for ws, n in ((dws.ptr, wsb), (dws.ptr, wsb), (None, 0)):
        dy = dev(hb) if epi == hai.EPI_RESIDUAL else out_buf(M * ncols * 2)
        res = dy.ptr if epi == hai.EPI_RESIDUAL else None
        if fp8:
            hai.check(kern().hai_gemm_fp8_mfma(dy.ptr, ncols, dx.ptr, K, dq.ptr, ds.ptr, None, M, N, K,
                                               epi | hai.FP8_NO_SPECIAL_CODES, res, ncols, ws, n, None), "fp8 mfma")
        else:
            hai.check(kern().hai_gemm_bf16_mfma(dy.ptr, ncols, dx.ptr, K, dw.ptr, M, N, K, epi, res, ncols, ws, n,
                                                None), "bf16 mfma")
        outs.append(dy.download(np.uint16).reshape(M, ncols))
    np.testing.assert_array_equal(outs[0], outs[1], err_msg="stream-K run to run")
    assert (outs[0] == outs[2]).mean() > 0.99
    sk, plain = hai.bf16_to_f32(outs[0]), hai.bf16_to_f32(outs[2])
    # SwiGLU rounds g and u to bf16 before silu(g) * u, and the residual
    # epilogue rounds acc before adding it: a regrouping flip compounds to a
    # few ulps of the operands, twice the one-sided oracle tolerance
    assert np.allclose(sk, plain, rtol=2 ** -6, atol=2 ** -8 * np.abs(plain).max()), float(np.abs(sk - plain).max())
