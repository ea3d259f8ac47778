"""Pins oracle/quant.py (the numpy restatement of quantize.py) against the
rules the reference states and its own checks:
- nibble packing order and two's-complement nibbles (quantize.py:36-99 docstrings);
- round-half-to-even of np.round (quantize.py:207, :252) on hand-made ties;
- fused == dequantize-then-matmul (tests/test_compress_v13.py:291-304, atol 1e-5);
- max|y_fp32 - y_q| / ||y_fp32||_F <= 0.05 for INT8 and INT4
  (tests/benchmark_quantize.py:121-135);
and the group-128 extension by exactness of q * fp16 scale and its error bound."""
import numpy as np
import pytest

from oracle import quant as Q


def test_pack_nibble_order_and_twos_complement():
    # -8 -> 8, -1 -> 15, 0 -> 0, 7 -> 7; low nibble holds the even index
    q = np.array([-8, -1, 0, 7], np.int8)
    assert Q.pack_int4(q).tolist() == [(15 << 4) | 8, (7 << 4) | 0]
    # odd length: padded with a zero high nibble
    assert Q.pack_int4(np.array([3, -2, 5], np.int8)).tolist() == [(14 << 4) | 3, 5]


@pytest.mark.parametrize("shape", [(7,), (8,), (3, 5), (4, 16)])
def test_pack_unpack_round_trip(shape):
    q = np.random.default_rng(0).integers(-8, 8, shape).astype(np.int8)
    assert np.array_equal(Q.unpack_int4(Q.pack_int4(q), shape), q)


def test_int4_round_half_even_and_clip():
    # max |w| = 7 -> scale exactly 1; ties go to even (np.round)
    w = np.array([[2.5, 3.5, -2.5, 0.5, 1.5, 7.0, -6.5, -0.5]], np.float32)
    packed, s = Q.quantize_int4(w)
    assert s.shape == (1, 1) and s[0, 0] == np.float32(1.0)
    assert Q.unpack_int4(packed, w.shape).tolist() == [[2, 4, -2, 0, 2, 7, -6, 0]]


def test_int8_rules():
    w = np.array([[127.0, 63.5, -0.5, 1.5, -127.0]], np.float32)
    q, s = Q.quantize_int8(w)
    assert s[0, 0] == np.float32(1.0)
    assert q.tolist() == [[127, 64, 0, 2, -127]]
    # zero rows: safe max 1 -> scale 1/127 (2-D); 1-D zero -> scale 1
    q0, s0 = Q.quantize_int8(np.zeros((2, 3), np.float32))
    assert np.all(q0 == 0) and np.all(s0 == np.float32(1.0) / np.float32(127.0))
    q1, s1 = Q.quantize_int8(np.zeros(4, np.float32))
    assert np.all(q1 == 0) and s1 == np.float32(1.0)


def test_one_d_and_two_d_scale_rules_agree():
    """1-D weights take max|w| / 127 in Python floats (fp64) then round to fp32;
    2-D weights divide in fp32 (quantize.py:205 vs :211).  For fp32 operands
    both give the correctly rounded quotient (fp64 has >= 2*24+2 bits, so the
    double rounding is innocuous), so the two paths must agree everywhere."""
    rng = np.random.default_rng(3)
    for m in rng.random(20000).astype(np.float32) * 10 + np.float32(1e-3):
        w1 = np.array([m, -m / 3], np.float32)
        _, s1 = Q.quantize_int8(w1)
        _, s2 = Q.quantize_int8(w1[None, :])
        assert s1 == np.float32(float(m) / 127.0) == s2[0, 0]


def test_fused_equals_dequantize_then_matmul():
    """tests/test_compress_v13.py:291-304: forward_fused == forward, atol 1e-5."""
    rng = np.random.default_rng(0)
    w = rng.normal(0, 0.25, (32, 16)).astype(np.float32)
    x = rng.normal(0, 1, (5, 16)).astype(np.float32)
    packed, s = Q.quantize_int4(w)
    fused = Q.matmul_int4(x, packed, s, w.shape)
    plain = x @ Q.dequantize_int4(packed, s, w.shape).T
    assert fused.shape == (5, 32)
    assert np.allclose(fused, plain, atol=1e-5)


@pytest.mark.parametrize("kind", ["int8", "int4", "int4_g128"])
def test_error_ratio_threshold(kind):
    """tests/benchmark_quantize.py:121-135: max|y - y_q| / ||y||_F <= 0.05."""
    rng = np.random.default_rng(7)
    K, N = 512, 512
    bound = 1.0 / np.sqrt(K)
    w = rng.uniform(-bound, bound, (N, K)).astype(np.float32)
    x = rng.normal(0, 1, (8, K)).astype(np.float32)
    if kind == "int8":
        q, s = Q.quantize_int8(w)
        wd = Q.dequantize_int8(q, s)
    elif kind == "int4":
        p, s = Q.quantize_int4(w)
        wd = Q.dequantize_int4(p, s, w.shape)
    else:
        p, s = Q.quantize_int4_g(w, 128)
        wd = Q.dequantize_int4_g(p, s, w.shape, 128)
    y, yq = x @ w.T, x @ wd.T
    assert np.max(np.abs(y - yq)) / np.linalg.norm(y) <= 0.05


def test_group128_dequant_is_exact_and_bounded():
    rng = np.random.default_rng(11)
    N, K = 64, 512
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    w[3, 128:256] = 0.0  # an all-zero group: scale fp16(1/7), q = 0
    p, s16 = Q.quantize_int4_g(w, 128)
    assert s16.dtype == np.float16 and s16.shape == (N, K // 128)
    assert s16[3, 1] == np.float16(np.float32(1.0) / np.float32(7.0))
    q = Q.unpack_int4(p, (N, K)).astype(np.float64).reshape(N, K // 128, 128)
    wd = Q.dequantize_int4_g(p, s16, (N, K), 128)
    exact = (q * s16.astype(np.float64)[..., None]).reshape(N, K)
    assert np.array_equal(wd.astype(np.float64), exact)  # q * fp16 scale is exact in fp32
    err = np.abs(w.astype(np.float64) - exact).reshape(N, K // 128, 128)
    half = s16.astype(np.float64)[..., None] / 2
    assert np.all(err <= half * (1 + 2e-3))  # rounding error of a symmetric grid
    assert q.min() >= -8 and q.max() <= 7
