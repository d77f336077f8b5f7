"""Prompt-sized linear layers on the matrix cores (hai_gemm_bf16_tiled /
hai_gemm_fp8_tiled): every output within the tolerance of fp32 accumulation
and bf16 output rounding of the float64 product, at the 27B prefill shapes
(gate|up with SwiGLU, down / o / out with the residual add) and at ragged
ones (M, N not multiples of the tile, K with an odd number of 64-element
steps), bf16 and FP8 weights (128 x 128 scale grids, interleaved gate / up
grids, per-row scale maps, the reference's +-480 codes).

Tolerance (floating point, tolerance mode): a stored output differs from
the float64 product by at most 2^-8 of its magnitude (bf16 rounding, with a
factor 2 margin) plus 2^-14 of sum_k |x_k w_k| (fp32 accumulation);
residual and SwiGLU outputs as the other matrix-core GEMMs' tests
(rtol 2^-6, atol 2e-3 of the largest).  A vendor library GEMM (torch's bf16
matmul on the GPU, which runs hipBLASLt / rocBLAS on ROCm; the reference's
prompt GEMMs are rocblas_gemm_ex calls) is held to the same bound on the
same inputs, as a cross-check of the bound."""
import numpy as np
import pytest
import torch

from _hai import hai, orc, rand_bf16

pytestmark = pytest.mark.gpu
K_ = None


def kern():
    global K_
    if K_ is None:
        K_ = hai.kernels()
    return K_


def dev(a):
    return hai.DeviceBuffer.from_array(np.ascontiguousarray(a))


def out_buf(nbytes):
    b = hai.DeviceBuffer(nbytes)
    b.zero()
    return b


def fp8_weights(rng, N, K, special=False):
    """E4M3 codes and U(0.5, 2)/448 block scales, as the C5 weights."""
    sb = ((N + 127) // 128, (K + 127) // 128)
    s = (rng.uniform(0.5, 2.0, sb) / 448.0).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    q = orc.fp8_encode(w / np.repeat(np.repeat(s, 128, 0), 128, 1)[:N, :K])
    if special:
        q.reshape(-1)[rng.choice(q.size, 64, replace=False)] = rng.choice([0x7F, 0xFF], 64)
    return q, s


def dequant(q, s):
    """decode(q) * s per 128 x 128 block, float64 (fp8_dequant.cc:12-146)."""
    N, K = q.shape
    d = orc.fp8_decode(q).astype(np.float64)
    return d * np.repeat(np.repeat(s.astype(np.float64), 128, 0), 128, 1)[:N, :K]


def exact(x, w64):
    """float64 product x . w^T and sum |x| |w| on the GPU (fp64 GEMMs)."""
    xt = torch.from_numpy(x.astype(np.float64)).cuda()
    wt = torch.from_numpy(w64).cuda()
    return (xt @ wt.T).cpu().numpy(), (xt.abs() @ wt.abs().T).cpu().numpy()


def check(got, y64, absdot, epi, h=None):
    if epi == hai.EPI_STORE:
        bound = 2.0 ** -8 * np.abs(y64) + 2.0 ** -14 * absdot
        bad = np.abs(got - y64) > bound
        assert not bad.any(), f"{bad.sum()} outputs out of bound, worst {float(np.abs(got - y64).max())}"
        return
    if epi == hai.EPI_RESIDUAL:
        want = h.astype(np.float64) + y64
    else:
        g, u = y64[:, 0::2], y64[:, 1::2]
        want = g / (1.0 + np.exp(-g)) * u
    scale = np.abs(want).max()
    assert np.allclose(got, want, rtol=2 ** -6, atol=2e-3 * scale), float(np.abs(got - want).max())


def run(M, N, K, epi, fp8=False, special=False, mapped=False, seed=0, vendor=False):
    """vendor: torch's bf16 matmul on the GPU (bf16 weights, store epilogue)
    instead of the tiled kernel."""
    rng = np.random.default_rng(seed + M + 3 * N + 7 * K + epi)
    x, xb = rand_bf16(rng, (M, K))
    mp = None
    if not fp8:
        w, wb = rand_bf16(rng, (N, K), 0.02)
        w64 = w.astype(np.float64)
    elif epi == hai.EPI_SILU_MUL:
        F = N // 2
        qg, sg = fp8_weights(rng, F, K, special)
        qu, su = fp8_weights(rng, F, K)
        q = np.empty((N, K), np.uint8)
        q[0::2], q[1::2] = qg, qu
        s = np.stack([sg, su])
        w64 = np.empty((N, K), np.float64)
        w64[0::2], w64[1::2] = dequant(qg, sg), dequant(qu, su)
    elif mapped:
        n0 = N // 2 + 64
        q0, s0 = fp8_weights(rng, n0, K, special)
        q1, s1 = fp8_weights(rng, N - n0, K)
        q, s = np.concatenate([q0, q1]), np.concatenate([s0, s1])
        mp = np.array([r // 128 for r in range(n0)] + [s0.shape[0] + r // 128 for r in range(N - n0)], np.int32)
        w64 = np.concatenate([dequant(q0, s0), dequant(q1, s1)])
    else:
        q, s = fp8_weights(rng, N, K, special)
        w64 = dequant(q, s)
    ncols = N // 2 if epi == hai.EPI_SILU_MUL else N
    h, hb = rand_bf16(rng, (M, ncols))
    dx = dev(xb)
    dy = dev(hb) if epi == hai.EPI_RESIDUAL else out_buf(M * ncols * 2)
    res = dy.ptr if epi == hai.EPI_RESIDUAL else None
    if vendor:
        assert not fp8 and epi == hai.EPI_STORE
        xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
        wt = torch.from_numpy(w).cuda().to(torch.bfloat16).t().contiguous()
        got = (xt @ wt).float().cpu().numpy().astype(np.float64)
        y64, absdot = exact(x, w64)
        check(got, y64, absdot, epi, h)
        return
    if fp8:
        dq, ds = dev(q), dev(s)
        dm = dev(mp) if mp is not None else None
        flag = 0 if special else hai.FP8_NO_SPECIAL_CODES
        hai.check(kern().hai_gemm_fp8_tiled(dy.ptr, ncols, dx.ptr, K, dq.ptr, ds.ptr, dm.ptr if dm else None, M, N, K,
                                            epi | flag, res, ncols, None), "gemm_fp8_tiled")
    else:
        dw = dev(wb)
        hai.check(kern().hai_gemm_bf16_tiled(dy.ptr, ncols, dx.ptr, K, dw.ptr, M, N, K, epi, res, ncols, None),
                  "gemm_bf16_tiled")
    got = hai.bf16_to_f32(dy.download(np.uint16).reshape(M, ncols)).astype(np.float64)
    y64, absdot = exact(x, w64)
    check(got, y64, absdot, epi, h)


@pytest.mark.parametrize("M,N,K,epi", [
    (512, 34816, 5120, 2),    # 27B gate|up, SwiGLU
    (512, 5120, 17408, 1),    # 27B down, residual
    (1024, 5120, 6144, 1),    # 27B o_proj (128 x 64 tiles)
    (512, 16384, 5120, 0),    # 27B DeltaNet qkv|z
    (300, 1000, 576, 0),      # ragged rows and columns, 9 k-steps
    (130, 200, 64, 2),        # one k-step, ragged SwiGLU pairs
    (2048, 768, 256, 1),      # tiny-config down at a long prompt
])
def test_gemm_bf16_tiled(M, N, K, epi):
    run(M, N, K, epi)


@pytest.mark.parametrize("M,N,K", [(1024, 16480, 5120), (300, 1000, 576)])
def test_vendor_gemm_within_the_same_bound(M, N, K):
    """The bound the tiled kernels are held to also holds for a vendor
    library GEMM on the same inputs (fp32 accumulation, bf16 output)."""
    run(M, N, K, hai.EPI_STORE, vendor=True)


@pytest.mark.parametrize("M,N,K,epi,special,mapped", [
    (512, 34816, 5120, 2, False, False),   # gate|up, interleaved scale grids
    (512, 5120, 17408, 1, False, False),   # down
    (700, 2 * 640 + 130, 1088, 0, True, True),  # per-row scale map, +-480 codes, K/128 not whole
    (256, 6144, 5120, 1, True, False),     # o_proj with the special-code check
])
def test_gemm_fp8_tiled(M, N, K, epi, special, mapped):
    run(M, N, K, epi, fp8=True, special=special, mapped=mapped)


def test_gemm_tiled_refuses_bad_shapes():
    """K must be whole 64-element steps; operands past 4 GiB are refused."""
    d = out_buf(1 << 16)
    assert kern().hai_gemm_bf16_tiled(d.ptr, 64, d.ptr, 96, d.ptr, 4, 64, 96, 0, None, 0, None) == hai.ERR_INVALID
    assert kern().hai_gemm_bf16_tiled(d.ptr, 1 << 20, d.ptr, 8192, d.ptr, 1 << 20, 1 << 20, 8192, 0, None, 0,
                                      None) == hai.ERR_INVALID
