"""FP8 E4M3 weights in the CPU oracle (row A15): the reference's own FP8
known-answer tests (tests/ops_fp8_dequant_test.cc:15-71), the decode formula
of fp8_dequant.cc:12-26 over all 256 codes, the RNE encoder against a brute
force search, and the FP8 GEMM against the dequantized-weight GEMM."""
import numpy as np
import pytest

from _hai import orc


def test_reference_kat_decode_and_block_scale():
    # DecodesE4M3AndAppliesBlockScale: 0x38 -> 1.0, 0x40 -> 2.0, scale 2.0
    d = orc.fp8_decode(np.array([0x38, 0x40], np.uint8))
    assert d.tolist() == [1.0, 2.0]
    w = orc.fp8_dequant_2d(np.array([[0x38, 0x40]], np.uint8), np.array([[2.0]], np.float32), 1, 128)
    assert w.tolist() == [[2.0, 4.0]]


def test_reference_kat_two_dimensional_blocks():
    # DequantizesTwoDimensionalBlocks: [3,4] codes, 2x2 blocks, scales [[1,2],[3,4]]
    q = np.array([0x38, 0x38, 0x38, 0x38, 0x40, 0x40, 0x40, 0x40, 0x38, 0x38, 0x40, 0x40], np.uint8).reshape(3, 4)
    s = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    v = orc.fp8_dequant_2d(q, s, 2, 2).reshape(-1)
    for i, want in ((0, 1.0), (1, 1.0), (2, 2.0), (3, 2.0), (4, 2.0), (6, 4.0), (8, 3.0), (10, 8.0)):
        assert v[i] == want, i


def _decode_f64(c):
    s = -1.0 if c & 0x80 else 1.0
    e, m = (c >> 3) & 15, c & 7
    return s * (m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))


def test_decode_all_codes():
    got = orc.fp8_decode(np.arange(256, dtype=np.uint8))
    want = np.array([_decode_f64(c) for c in range(256)], np.float64)
    assert np.array_equal(got.astype(np.float64), want)
    assert got[0x7E] == 448.0 and got[0x7F] == 480.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6
    assert np.signbit(got[0x80]) and got[0x80] == 0.0


def test_encode_roundtrip_and_saturation():
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], np.uint8)
    assert np.array_equal(orc.fp8_encode(orc.fp8_decode(codes)), codes)
    assert orc.fp8_encode(np.array([480.0, 1e9, -1e9, np.inf], np.float32)).tolist() == [0x7E, 0x7E, 0xFE, 0x7E]


def test_encode_is_nearest_ties_to_even():
    grid_codes = np.arange(0, 0x7F, dtype=np.uint8)          # 0 .. 448, positive
    grid = orc.fp8_decode(grid_codes).astype(np.float64)
    rng = np.random.default_rng(0)
    mids = (grid[1:] + grid[:-1]) / 2                         # exact ties
    xs = np.concatenate([rng.uniform(0, 460, 20000), np.exp(rng.uniform(-14, 6, 20000)), mids]).astype(np.float32)
    got = orc.fp8_encode(xs)
    for x, g in zip(xs.astype(np.float64), got):
        if x >= 448:
            assert g == 0x7E
            continue
        d = np.abs(grid - x)
        best = np.flatnonzero(d == d.min())
        want = best[0] if len(best) == 1 else best[best % 2 == 0][0]  # tie: even mantissa
        assert g == grid_codes[want], (x, g, grid_codes[want])


@pytest.mark.parametrize("M,N,K", [(2, 300, 200), (1, 130, 520), (3, 256, 1024)])
def test_gemm_fp8_equals_dequantized_gemm(M, N, K):
    rng = np.random.default_rng(M + N + K)
    x = orc.round_bf16(rng.standard_normal((M, K)).astype(np.float32))
    sb = ((N + 127) // 128, (K + 127) // 128)
    s = (rng.uniform(0.5, 2.0, sb) / 448.0).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    srow = np.repeat(np.repeat(s, 128, 0), 128, 1)[:N, :K]
    q = orc.fp8_encode(w / srow)
    got = orc.gemm_fp8(x, q, s)
    assert np.array_equal(got, orc.gemm(x, orc.fp8_dequant_2d(q, s, 128, 128)))
    ref = x.astype(np.float64) @ (orc.fp8_decode(q).astype(np.float64) * srow).T
    assert np.allclose(got, ref, rtol=1e-2, atol=1e-3)


def test_synthetic_scales_are_uniform_half_to_two_over_448():
    s = orc.fp8_synthetic_scales(0, 2 * 64 + 17, 200000).astype(np.float64) * 448.0
    assert s.min() >= 0.5 and s.max() < 2.0
    # U(0.5, 2): mean 1.25, variance 1.5^2 / 12, deciles evenly spaced
    assert abs(s.mean() - 1.25) < 0.005 and abs(s.var() - 0.1875) < 0.003
    dec = np.quantile(s, np.linspace(0.1, 0.9, 9))
    assert np.allclose(dec, 0.5 + 1.5 * np.linspace(0.1, 0.9, 9), atol=0.01)
    # independent streams per tensor and seed, reproducible
    assert np.array_equal(orc.fp8_synthetic_scales(0, 145, 64), orc.fp8_synthetic_scales(0, 145, 64))
    assert not np.array_equal(orc.fp8_synthetic_scales(0, 145, 64), orc.fp8_synthetic_scales(1, 145, 64))
    assert not np.array_equal(orc.fp8_synthetic_scales(0, 145, 64), orc.fp8_synthetic_scales(0, 146, 64))


def test_fp8_model_quantizes_exactly_the_quantized_weight_linears():
    """orc_model_quantize_fp8 on the tiny config: the Linears the reference
    loads as QuantizedWeight become dequantize_2d(encode(w / s), s) on their
    own 128x128 grid; every other tensor keeps its bf16 value."""
    cfg = orc.TINY
    bf = orc.Model(cfg, seed=5)
    q8 = orc.Model(cfg, seed=5, fp8=True)
    H, F = cfg["hidden"], cfg["ffn"]
    qw, kvw = cfg["num_q_heads"] * cfg["head_dim"], cfg["num_kv_heads"] * cfg["head_dim"]
    vw = cfg["lin_v_heads"] * cfg["lin_v_dim"]
    C = 2 * cfg["lin_qk_heads"] * cfg["lin_k_dim"] + vw
    shapes = {2: (C, H), 3: (vw, H), 10: (H, vw), 11: (2 * qw, H), 12: (kvw, H), 13: (kvw, H), 14: (H, qw),
              17: (F, H), 18: (F, H), 19: (H, F)}
    n_quant = 0
    for slot in (0, 1, 2, 3, 4, 5, 1024):
        for kind in range(20):
            tid = slot * 64 + kind
            try:
                w = bf.tensor(tid)
            except KeyError:
                continue
            got = q8.tensor(tid)
            if slot >= 2 and kind in shapes:
                rows, cols = shapes[kind]
                sb = ((rows + 127) // 128, (cols + 127) // 128)
                s = orc.fp8_synthetic_scales(5, tid, sb[0] * sb[1]).reshape(sb)
                wq = orc.fp8_encode(w.reshape(rows, cols) / np.repeat(np.repeat(s, 128, 0), 128, 1)[:rows, :cols])
                assert np.array_equal(got.reshape(rows, cols), orc.fp8_dequant_2d(wq, s, 128, 128)), tid
                assert not np.array_equal(got, w)
                n_quant += 1
            else:
                assert np.array_equal(got, w), tid
    assert n_quant == 3 * 6 + 2 * 7   # 3 DeltaNet layers x 6, attention + MTP layer x 7
    bf.close(); q8.close()
