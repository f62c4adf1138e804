"""GPU parity of each kernel of the seam (src/tensor/kernels.rs on device
pointers) against the reference's known answers and the CPU oracle.
Tolerances follow the reference's own SIMD-vs-scalar differential tests
(docs/adr/0012: 2e-4 relative for linear, 2e-5 for RMSNorm, 1e-6 for L2 and
pooling); attention is checked at 1e-4 absolute."""
import numpy as np
import pytest
import torch

import svl_amd as S
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV)


def host(t):
    return t.detach().cpu().numpy()


def empty(n):
    return torch.empty(n, dtype=torch.float32, device=DEV)


def test_linear_kat():  # kernels.rs:1401-1410
    out = empty(4)
    S.linear(dev([1, 2, 3, 4, 5, 6]), dev([1, 0, -1, 0, 1, 1]), 2, 3, 2, out)
    assert host(out).tolist() == [-2.0, 5.0, -2.0, 11.0]


# Shapes chosen to reach every tile path of the GEMM dispatcher: one-row
# grids with 256-, 128-, 64- and 32-wide K slices (32x32 tiles), grids too
# large for one round of those (64-wide slices, three stages), K not a
# multiple of 32 (64x64x16) or of 16 (the register-staged kernel's K tail) or
# of 4 (the scalar kernel), grids large enough for the cost model's 64x32,
# 64x64 and 128x128 choices (128x128 counts rounded to whole rounds), and
# narrow outputs (128x32 tiles, ragged N included).
@pytest.mark.parametrize("rows,inf,outf", [
    (1, 768, 768), (37, 768, 1280), (130, 1152, 768), (257, 256, 768), (5, 12, 20), (3, 10, 7),
    (64, 16, 8), (300, 1120, 96), (129, 784, 40), (2000, 100, 300), (9000, 256, 64),
    (2048, 768, 768), (4096, 768, 2304), (20000, 128, 32), (16500, 64, 20),
    (520, 768, 1280), (3000, 1024, 1024), (16384, 768, 1280)])
def test_linear_matches_oracle(rows, inf, outf):
    rng = np.random.default_rng(rows * 7 + inf)
    x = rng.standard_normal((rows, inf)).astype(np.float32)
    w = (rng.standard_normal((outf, inf)) / np.sqrt(inf)).astype(np.float32)
    out = empty(rows * outf)
    S.linear(dev(x), dev(w), rows, inf, outf, out)
    got = host(out).reshape(rows, outf)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(got, exact, atol=2e-4 * np.abs(exact).max(), rtol=0)
    if rows * inf * outf <= 2e9:   # the scalar oracle takes seconds per GFLOP
        ref = O.linear(x, w, rows, inf, outf).reshape(rows, outf)
        np.testing.assert_allclose(got, ref, atol=2e-4 * np.abs(exact).max(), rtol=0)


# A row's output bits do not depend on the launch around it: every tile shape
# and tile order runs the same MFMA sequence over k. The whole launches here
# take the grouped tile order (128 M blocks or more; a partial last group, the
# odd groups' N blocks in reverse) on 128x32, 64x64 and 64x32 tiles; 100-row
# slices take 32x32 tiles in the plain order.
@pytest.mark.parametrize("rows,inf,outf", [
    (16500, 64, 20), (9000, 768, 2304), (18688, 768, 256), (8229, 1152, 768)])
def test_linear_rows_do_not_depend_on_the_launch(rows, inf, outf):
    rng = np.random.default_rng(rows + outf)
    x = rng.standard_normal((rows, inf)).astype(np.float32)
    w = (rng.standard_normal((outf, inf)) / np.sqrt(inf)).astype(np.float32)
    xd, wd = dev(x), dev(w)
    out = empty(rows * outf)
    S.linear(xd, wd, rows, inf, outf, out)
    full = host(out).reshape(rows, outf)
    part = empty(100 * outf)
    for r0 in (0, rows // 2 + 3, rows - 100):
        S.linear(xd[r0:r0 + 100], wd, 100, inf, outf, part)
        np.testing.assert_array_equal(host(part).reshape(100, outf), full[r0:r0 + 100])


def test_linear_rejects_nonfinite_output():
    out = empty(1)
    with pytest.raises(S.SvlError) as e:
        S.linear(dev([float("inf")]), dev([1.0]), 1, 1, 1, out)
    assert e.value.kind == "Internal"


def test_rms_norm_kats():  # kernels.rs:1431-1443
    out = empty(4)
    S.rms_norm_rows(dev([3, 4, 0, 2]), dev([1, 1]), 2, 2, 0.0, out)
    np.testing.assert_allclose(host(out), [0.848528, 1.131371, 0, np.sqrt(2)], atol=1e-5)
    out2 = empty(2)
    S.rms_norm_rows(dev([3, 4]), None, 1, 2, 0.0, out2)
    np.testing.assert_allclose(host(out2), [0.848528, 1.131371], atol=1e-5)
    with pytest.raises(S.SvlError):
        S.rms_norm_rows(dev([float("nan")]), dev([1.0]), 1, 1, 0.0, empty(1))


@pytest.mark.parametrize("rows,width", [(1000, 768), (77, 256), (9, 16), (5, 7), (3, 2304)])
def test_rms_norm_matches_oracle(rows, width):
    rng = np.random.default_rng(width)
    x = rng.standard_normal((rows, width)).astype(np.float32) * 3
    w = rng.uniform(0.5, 1.5, width).astype(np.float32)
    out = empty(rows * width)
    S.rms_norm_rows(dev(x), dev(w), rows, width, 1e-6, out)
    np.testing.assert_allclose(host(out), O.rms_norm_rows(x, w, rows, width, 1e-6), atol=2e-5, rtol=2e-5)
    S.rms_norm_rows(dev(x), None, rows, width, 1e-6, out)
    np.testing.assert_allclose(host(out), O.rms_norm_rows_unscaled(x, rows, width, 1e-6), atol=2e-5, rtol=2e-5)


def test_rope_kat_and_oracle():  # kernels.rs:1494-1509
    v = dev([1.0, 0.0])
    S.rope_with_inv_freq(v, 1, 1, 2, S.rope_inv_freq(2, 10000.0), 1)
    np.testing.assert_allclose(host(v), [0.540302, 0.841471], atol=1e-5)
    rng = np.random.default_rng(3)
    seq, heads, hd = 300, 3, 256
    x = rng.standard_normal(seq * heads * hd).astype(np.float32)
    inv = O.rope_inv_freq(hd, 10000.0)
    np.testing.assert_array_equal(S.rope_inv_freq(hd, 10000.0), inv)
    t = dev(x)
    S.rope_with_inv_freq(t, seq, heads, hd, inv, 5)
    np.testing.assert_allclose(host(t), O.rope_with_inv_freq(x, seq, heads, hd, inv, 5), atol=1e-5)


def test_attention_kats():  # kernels.rs:1529-1566
    out = empty(2)
    S.bidirectional_attention(dev([1, 1]), dev([1, 0]), dev([10, 20]), 2, 1, 1, 1, None, 1.0, out)
    np.testing.assert_allclose(host(out), [12.6894, 12.6894], atol=1e-4)
    q, k, v = dev([1, 1, 1]), dev([1, 0, 0]), dev([10, 20, 30])
    out = empty(3)
    S.bidirectional_attention(q, k, v, 3, 1, 1, 1, 0, 1.0, out)
    assert host(out).tolist() == [10.0, 20.0, 30.0]
    S.bidirectional_attention(q, k, v, 3, 1, 1, 1, 1, 1.0, out)
    np.testing.assert_allclose(host(out), [12.6894, 16.3582, 25.0], atol=1e-4)
    out = empty(4)
    S.bidirectional_attention(dev([1, 1, 0, 0]), dev([1, 0]), dev([5, 7]), 1, 4, 2, 1, None, 1.0, out)
    np.testing.assert_allclose(host(out), [5, 5, 7, 7], atol=1e-6)


@pytest.mark.parametrize("seq,nh,nkv,hd,window", [
    (1, 3, 1, 256, None), (37, 3, 1, 256, None), (130, 3, 1, 256, 16), (700, 3, 1, 256, 512),
    (97, 4, 2, 256, 8), (64, 12, 12, 64, None), (50, 8, 8, 128, 7), (33, 4, 1, 512, None),
    (21, 2, 1, 8, 2), (9, 2, 1, 16, None), (300, 4, 4, 64, 40), (131, 6, 2, 128, None),
    (1000, 3, 1, 256, 100), (700, 4, 1, 512, None), (300, 8, 2, 512, 40), (1000, 4, 1, 512, 100),
    (5, 4, 1, 512, None), (129, 2, 2, 512, 3), (2000, 3, 1, 256, 512), (900, 4, 4, 128, 64),
    # head_dim 512 with 128 and with 64 work items: the 8-wave and the 4-wave variants
    (2048, 8, 2, 512, None), (1024, 8, 2, 512, 40),
    # 65 to 127 work items at head_dim 256 and 128: two 4-wave workgroups per item
    (3000, 3, 1, 256, 512), (2500, 4, 1, 128, None)])
def test_attention_matches_oracle(seq, nh, nkv, hd, window):
    rng = np.random.default_rng(seq + hd)
    # unit-RMS rows scaled like q/k after their norms (weights ~0.25)
    q = (rng.standard_normal((seq, nh, hd)) * 0.25).astype(np.float32)
    k = (rng.standard_normal((seq, nkv, hd)) * 0.25).astype(np.float32)
    v = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    out = empty(seq * nh * hd)
    S.bidirectional_attention(dev(q), dev(k), dev(v), seq, nh, nkv, hd, window, 1.0, out)
    ref = O.bidirectional_attention(q, k, v, seq, nh, nkv, hd, window, 1.0)
    np.testing.assert_allclose(host(out), ref, atol=1e-4, rtol=1e-4)


@pytest.fixture
def attention_path():
    """Sets the process-wide attention kernel choice for one test and puts
    it back to "auto" afterwards, also when the test fails."""
    yield S.set_attention_path
    S.set_attention_path("auto")


FALLBACK_SHAPES = [
    (1, 3, 1, 256, None), (37, 3, 1, 256, None), (130, 3, 1, 256, 16), (700, 3, 1, 256, 512),
    (97, 4, 2, 256, 8), (64, 12, 12, 64, None), (50, 8, 8, 128, 7), (33, 4, 1, 512, None),
    (300, 4, 4, 64, 40), (131, 6, 2, 128, None), (1000, 3, 1, 256, 100), (300, 8, 2, 512, 40),
    (129, 2, 2, 512, 3), (900, 4, 4, 128, 64), (200, 3, 1, 64, 33)]


@pytest.mark.parametrize("path", ["fallback", "generic"])
@pytest.mark.parametrize("seq,nh,nkv,hd,window", FALLBACK_SHAPES)
def test_fallback_attention_kernels_match_oracle(seq, nh, nkv, hd, window, path, attention_path):
    """The kernels that rows whose K/V operand window passes 2 GiB take (the
    register-staged 32x32x2 MFMA kernel at head_dim 64 / 128 / 256, the
    generic kernel at 512), and the generic kernel at every head dim, forced
    through the test hook on the shapes of the DMA kernel's parity test
    (kernels.rs:1037-1135)."""
    rng = np.random.default_rng(seq + hd)
    q = (rng.standard_normal((seq, nh, hd)) * 0.25).astype(np.float32)
    k = (rng.standard_normal((seq, nkv, hd)) * 0.25).astype(np.float32)
    v = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    out = empty(seq * nh * hd)
    attention_path(path)
    S.bidirectional_attention(dev(q), dev(k), dev(v), seq, nh, nkv, hd, window, 1.0, out)
    attention_path("auto")
    ref = O.bidirectional_attention(q, k, v, seq, nh, nkv, hd, window, 1.0)
    np.testing.assert_allclose(host(out), ref, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("seq,nh,nkv,hd,window", [
    (37, 3, 1, 256, None), (50, 8, 8, 128, 7), (131, 6, 2, 128, None), (300, 4, 4, 64, 40),
    (33, 4, 1, 512, None), (1000, 3, 1, 256, 100)])
def test_attention_ignores_memory_past_the_keys(seq, nh, nkv, hd, window):
    """The last key tile of a row reaches past the row end; those keys must
    read as zero. K and V here sit in allocations whose rows after the last
    key are NaN, so any read of them makes the output non-finite (and the
    call fails with Internal)."""
    rng = np.random.default_rng(7 * seq + hd)
    q = (rng.standard_normal((seq, nh, hd)) * 0.25).astype(np.float32)
    k = (rng.standard_normal((seq, nkv, hd)) * 0.25).astype(np.float32)
    v = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    pad = 64 * nkv * hd

    def poisoned(a):
        t = torch.full((a.size + pad,), float("nan"), dtype=torch.float32, device=DEV)
        t[:a.size] = dev(a.reshape(-1))
        return t

    out = empty(seq * nh * hd)
    S.bidirectional_attention(dev(q), poisoned(k), poisoned(v), seq, nh, nkv, hd, window, 1.0, out)
    got = host(out)
    assert np.isfinite(got).all()
    ref = O.bidirectional_attention(q, k, v, seq, nh, nkv, hd, window, 1.0)
    np.testing.assert_allclose(got, ref, atol=1e-4, rtol=1e-4)


def test_elementwise_kats():  # kernels.rs:1151-1160, 1301-1316
    out = empty(2)
    S.add(dev([1, 2]), dev([3, 4]), 2, out)
    assert host(out).tolist() == [4.0, 6.0]
    S.geglu(dev([1, 0]), dev([2, 3]), 2, out)
    np.testing.assert_allclose(host(out), [1.682384, 0.0], atol=1e-5)
    out4 = empty(4)
    S.gelu_tanh(dev([0, 1, -1, 10]), 4, out4)
    np.testing.assert_allclose(host(out4), [0, 0.841192, -0.158808, 10], atol=1e-4)
    x = np.linspace(-6, 6, 10001, dtype=np.float32)
    o = empty(x.size)
    S.gelu_tanh(dev(x), x.size, o)
    ref = np.array([O.gelu_tanh_value(float(t)) for t in x], np.float32)
    np.testing.assert_allclose(host(o), ref, atol=2e-6, rtol=2e-6)


def test_pool_and_l2_kats():  # kernels.rs:1319-1324, 1466-1477
    out = empty(2)
    S.mean_pool(dev([1, 2, 3, 4]), 2, 2, out)
    assert host(out).tolist() == [2.0, 3.0]
    S.l2_normalize(dev([3, 4]), 2, out)
    np.testing.assert_allclose(host(out), [0.6, 0.8], atol=1e-7)
    with pytest.raises(S.SvlError) as e:
        S.l2_normalize(dev([0, 0]), 2, out)
    assert e.value.kind == "Internal"
    rng = np.random.default_rng(5)
    x = rng.standard_normal((513, 768)).astype(np.float32)
    o = empty(768)
    S.mean_pool(dev(x), 513, 768, o)
    # same order of f32 operations as mean_pool_scalar: bit-identical
    np.testing.assert_array_equal(host(o), O.mean_pool(x, 513, 768))
