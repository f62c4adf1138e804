"""Pins each oracle kernel against the reference's known-answer tests
(src/tensor/kernels.rs:1151-1593) and against closed forms / brute force that
a plausible slip (dropped weight, 1+w norm, 1/sqrt(d) scale, wrong GQA index,
one-sided window) would fail."""
import math

import numpy as np
import pytest

from oracle import oracle as O


def close(a, b, tol):
    np.testing.assert_allclose(np.asarray(a, np.float64), np.asarray(b, np.float64), atol=tol, rtol=0)


def test_linear_kat():  # kernels.rs:1401-1410
    out = O.linear([1, 2, 3, 4, 5, 6], [1, 0, -1, 0, 1, 1], 2, 3, 2)
    assert out.tolist() == [-2.0, 5.0, -2.0, 11.0]


def test_matmul_kats():  # kernels.rs:1198-1220
    assert O.matmul([1, 2, 3, 4, 5, 6], [7, 8, 9, 10, 11, 12], 2, 3, 2).tolist() == [58, 64, 139, 154]
    assert O.matmul([2, 3, 4, 5], [1, 0, 0, 1], 2, 2, 2).tolist() == [2, 3, 4, 5]
    assert O.matmul([1, 2, 3, 4], [5, 6, 7, 8], 2, 2, 2).tolist() == [19, 22, 43, 50]


def test_linear_matches_float64_brute_force():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((7, 33)).astype(np.float32)
    w = rng.standard_normal((5, 33)).astype(np.float32)
    out = O.linear(x, w, 7, 33, 5).reshape(7, 5)
    close(out, x.astype(np.float64) @ w.astype(np.float64).T, 1e-4)


def test_rms_norm_kats():  # kernels.rs:1267-1278, 1431-1443
    close(O.rms_norm_rows([3, 4], [1, 1], 1, 2, 0.0), [0.848528, 1.131371], 1e-5)
    close(O.rms_norm_rows([3, 4], [2, 2], 1, 2, 0.0), [1.697056, 2.262741], 1e-5)
    assert O.rms_norm_rows([0, 0], [1, 1], 1, 2, 1e-6).tolist() == [0.0, 0.0]
    close(O.rms_norm_rows([3, 4, 0, 2], [1, 1], 2, 2, 0.0), [0.848528, 1.131371, 0, math.sqrt(2)], 1e-5)
    close(O.rms_norm_rows_unscaled([3, 4], 1, 2, 0.0), [0.848528, 1.131371], 1e-5)


def test_rms_norm_weight_is_multiplied_not_one_plus():
    # A (1 + w) Gemma-3 style norm would give 2x here.
    close(O.rms_norm_rows([3, 4], [1, 1], 1, 2, 0.0), [0.848528, 1.131371], 1e-5)
    close(O.rms_norm_rows([1, 1], [0.5, 0.5], 1, 2, 0.0), [0.5, 0.5], 1e-6)


def test_rms_norm_rejections():  # kernels.rs:1446-1463
    with pytest.raises(O.OracleError):
        O.rms_norm_rows([1.0], [1.0], 1, 1, -1.0)
    with pytest.raises(O.OracleError):
        O.rms_norm_rows([float("nan")], [1.0], 1, 1, 0.0)


def test_gelu_geglu_kats():  # kernels.rs:1301-1316
    close([O.gelu_tanh_value(0.0)], [0.0], 1e-7)
    close([O.gelu_tanh_value(1.0)], [0.841192], 1e-5)
    close([O.gelu_tanh_value(-1.0)], [-0.158808], 1e-5)
    close([O.gelu_tanh_value(10.0)], [10.0], 1e-4)
    close(O.geglu([1.0, 0.0], [2.0, 3.0]), [1.682384, 0.0], 1e-5)


def test_softmax_kats():  # kernels.rs:1229-1264
    s = O.softmax([1.0, 2.0, 3.0])
    assert abs(s.sum() - 1) < 1e-6 and s[0] < s[1] < s[2]
    s = O.softmax([1000.0, 1001.0])
    assert np.isfinite(s).all() and abs(s.sum() - 1) < 1e-6
    assert O.softmax([float("inf"), 1.0]).tolist() == [1.0, 0.0]
    with pytest.raises(O.OracleError):
        O.softmax([float("-inf"), float("-inf")])
    with pytest.raises(O.OracleError):
        O.softmax([1.0, float("nan")])


def test_l2_pool_truncate_kats():  # kernels.rs:1319-1340, 1466-1491
    close(O.l2_normalize([3, 4]), [0.6, 0.8], 1e-7)
    with pytest.raises(O.OracleError):
        O.l2_normalize([0.0, 0.0])
    assert O.mean_pool([1, 2, 3, 4], 2, 2).tolist() == [2.0, 3.0]
    close(O.truncate_and_normalize([3, 4, 12], 2), [0.6, 0.8], 1e-7)
    with pytest.raises(O.OracleError):
        O.truncate_and_normalize([1.0], 2)
    with pytest.raises(O.OracleError):
        O.truncate_and_normalize([1.0], 0)


def test_rope_kats():  # kernels.rs:1343-1357, 1494-1509
    inv = O.rope_inv_freq(2, 10000.0)
    assert inv.tolist() == [1.0]
    close(O.rope_with_inv_freq([1.0, 0.0], 1, 1, 2, inv, offset=1), [0.540302, 0.841471], 1e-5)
    inv4 = O.rope_inv_freq(4, 10000.0)
    close(inv4, [1.0, 0.01], 1e-9)
    close(O.rope_with_inv_freq([1, 2, 3, 4], 1, 1, 4, inv4, 0), [1, 2, 3, 4], 1e-6)
    with pytest.raises(O.OracleError):
        O.rope_inv_freq(1, 10000.0)


def test_rope_rotate_half_pairs_j_with_j_plus_half():
    # head_dim 4: pair (0,2) rotates by pos*1, pair (1,3) by pos*0.01.
    inv = O.rope_inv_freq(4, 10000.0)
    out = O.rope_with_inv_freq([1, 0, 0, 0], 1, 1, 4, inv, offset=3)
    close(out, [math.cos(3), 0, math.sin(3), 0], 1e-6)


def test_attention_kats():  # kernels.rs:1529-1566
    close(O.bidirectional_attention([1, 1], [1, 0], [10, 20], 2, 1, 1, 1, None), [12.6894, 12.6894], 1e-4)
    q, k, v = [1, 1, 1], [1, 0, 0], [10, 20, 30]
    assert O.bidirectional_attention(q, k, v, 3, 1, 1, 1, 0).tolist() == [10.0, 20.0, 30.0]
    close(O.bidirectional_attention(q, k, v, 3, 1, 1, 1, 1), [12.6894, 16.3582, 25.0], 1e-4)
    close(O.bidirectional_attention([1, 1, 0, 0], [1, 0], [5, 7], 1, 4, 2, 1, None), [5, 5, 7, 7], 1e-6)


def test_attention_matches_float64_brute_force_with_window_and_gqa():
    rng = np.random.default_rng(1)
    seq, nh, nkv, hd, r = 9, 4, 2, 6, 2
    q = rng.standard_normal((seq, nh, hd)).astype(np.float32)
    k = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    out = O.bidirectional_attention(q, k, v, seq, nh, nkv, hd, r).reshape(seq, nh, hd)
    ref = np.zeros((seq, nh, hd))
    for i in range(seq):
        lo, hi = max(0, i - r), min(seq - 1, i + r)
        for h in range(nh):
            g = h // (nh // nkv)
            s = np.array([q[i, h].astype(np.float64) @ k[j, g] for j in range(lo, hi + 1)])
            p = np.exp(s - s.max())
            p /= p.sum()
            ref[i, h] = p @ v[lo:hi + 1, g].astype(np.float64)
    close(out, ref, 1e-5)
