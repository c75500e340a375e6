"""The reference's kernel entry points, on the GPU, against the checker.

Same names and arguments as the reference's ctypes harnesses bind them
(python/verify/bconv_harness.py:36-47, maxpool_harness.py:46,
head_harness.py:37, realin_conv_harness.py:47, forward_driver.py:64-65);
integer results must be identical, float results bit-identical.
"""
import numpy as np
import pytest

from bnns_to_c_amd import blob as B
from bnns_to_c_amd import engine as E

pytestmark = pytest.mark.gpu

SELFTEST = [(8, 8, 8, 4, 3, 3, 1, 1), (16, 16, 16, 32, 3, 3, 1, 1), (32, 7, 5, 16, 3, 3, 1, 1),
            (3, 6, 6, 5, 3, 3, 0, 1)]
EDGE = [(1, 1, 1, 4), (3, 1, 5, 4), (5, 5, 1, 8), (7, 4, 4, 6), (16, 3, 3, 16), (17, 5, 7, 8),
        (130, 3, 10, 8), (192, 3, 12, 8), (63, 4, 6, 8), (64, 4, 6, 8), (65, 4, 6, 8), (130, 3, 3, 8),
        (48, 9, 9, 16)]
UNET = [(16, 16), (16, 32), (32, 32), (32, 64), (64, 64), (64, 128), (128, 128), (128, 256),
        (256, 256), (384, 128), (192, 64), (96, 32), (48, 16)]


def rand_pm1(rng, shape):
    return np.where(rng.random(shape) < 0.5, -1, 1).astype(np.int8)


@pytest.mark.parametrize("case", SELFTEST + [(c, h, w, o, 3, 3, 1, 1) for c, h, w, o in EDGE]
                         + [(9, 7, 6, 5, 3, 3, 1, 2), (12, 8, 8, 40, 1, 1, 0, 1), (33, 9, 9, 36, 3, 3, 1, 1)])
def test_bconv(orc, case):
    cin, H, W, cout, kh, kw, pad, stride = case
    rng = np.random.default_rng(abs(hash(case)) % 2**31)
    a = rand_pm1(rng, (cin, H, W))
    w = rand_pm1(rng, (cout, cin, kh, kw))
    bits = B.pack_kidx(w)
    want = orc.bconv(a, bits, cout, kh, kw, pad, stride)
    for fn in ("bconv_xnor", "bconv_xnor_packed", "bconv_dispatch"):
        got = E.bconv(a, bits, cout, kh, kw, pad, stride, fn=fn)
        assert np.array_equal(got, want), fn
    assert np.array_equal(E.bconv_naive_int(a, w, pad, stride), orc.bconv_naive(a, w, pad, stride))


@pytest.mark.parametrize("cin,cout", UNET)
def test_bconv_unet_shapes(orc, cin, cout):
    rng = np.random.default_rng(cin * 7 + cout)
    for H, W in ((2, 2), (4, 4), (9, 13)):
        a = rand_pm1(rng, (cin, H, W))
        w = rand_pm1(rng, (cout, cin, 3, 3))
        bits = B.pack_kidx(w)
        assert np.array_equal(E.bconv(a, bits, cout), orc.bconv(a, bits, cout)), (H, W)


def test_bconv_zero_activations(orc):
    rng = np.random.default_rng(3)
    a = rand_pm1(rng, (40, 6, 5))
    a[:, 2, :] = 0
    w = rand_pm1(rng, (8, 40, 3, 3))
    bits = B.pack_kidx(w)
    assert np.array_equal(E.bconv(a, bits, 8), orc.bconv(a, bits, 8))
    assert np.array_equal(E.bconv_naive_int(a, w), orc.bconv_naive(a, w))


def test_pack_weights():
    rng = np.random.default_rng(4)
    w = rand_pm1(rng, (9, 21, 3, 3))
    assert np.array_equal(E.pack_weights(w), B.pack_kidx(w))


@pytest.mark.parametrize("cin,H,W,cout,k,pad", [(120, 32, 32, 16, 3, 1), (120, 17, 23, 8, 3, 1),
                                                (5, 6, 6, 4, 3, 1), (3, 9, 7, 6, 3, 1), (2, 5, 5, 3, 3, 0),
                                                (64, 12, 10, 32, 3, 1), (20, 8, 8, 40, 3, 1),
                                                (120, 6, 6, 8, 1, 0), (7, 1, 9, 5, 3, 1)])
def test_conv_realin(orc, cin, H, W, cout, k, pad):
    rng = np.random.default_rng(cin + H * W + cout)
    x = (rng.standard_normal((cin, H, W)) * rng.choice([1e-3, 1.0, 1e3], (cin, 1, 1))).astype(np.float32)
    w = rand_pm1(rng, (cout, cin, k, k))
    alpha = rng.uniform(0.01, 0.1, cout).astype(np.float32)
    got = E.conv_realin(x, w, alpha, pad=pad)
    want = orc.conv_real(x, w, alpha, pad=pad)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_conv_realin_order():
    # in-order sum over ci: [1e8, 1, -1e8] sums to 0 in float32 only in that order
    x = np.array([1e8, 1.0, -1e8], np.float32).reshape(3, 1, 1)
    w = np.ones((1, 3, 3, 3), np.int8)
    assert E.conv_realin(x, w, np.ones(1, np.float32))[0, 0, 0] == 0.0


def test_maxpool(orc):
    rng = np.random.default_rng(5)
    for C, H, W in [(8, 8, 8), (16, 6, 10), (4, 4, 4), (3, 5, 7)]:
        P = rng.integers(-300, 300, (C, H, W)).astype(np.int32)
        assert np.array_equal(E.maxpool_P(P), orc.maxpool(P))


def test_fold_int(orc):
    P = np.arange(-40, 41, dtype=np.int32)
    rows = [(ty, t, lo, hi) for ty in range(7) for t in (-3, 0, 1, 40, -41)
            for lo, hi in ((-5, 5), (3, 3), (6, -6))]
    ty, t, lo, hi = (np.array(v, np.int32) for v in zip(*rows))
    PP = np.broadcast_to(P, (len(rows), 1, P.size)).copy()
    assert np.array_equal(E.apply_fold_int(PP, ty, t, lo, hi), orc.fold_int(PP, ty, t, lo, hi))


def test_fold_real(orc):
    rng = np.random.default_rng(6)
    x = rng.normal(0, 1, (16, 32, 32)).astype(np.float32)
    A = rng.uniform(0.5, 1.5, 16).astype(np.float32)
    Bv = rng.normal(0, 0.1, 16).astype(np.float32)
    s = rng.uniform(-0.5, 0.5, 16).astype(np.float32)
    r = rng.normal(0, 0.1, 16).astype(np.float32)
    assert np.array_equal(E.apply_fold_real(x, A, Bv, s, r), orc.fold_real(x, A, Bv, s, r))


def test_head(orc):
    rng = np.random.default_rng(7)
    for cin, H, W, cout in [(16, 8, 8, 3), (32, 5, 7, 4), (8, 16, 16, 2)]:
        a = rand_pm1(rng, (cin, H, W)).astype(np.float32)
        Wt = rng.normal(0, 0.5, (cout, cin)).astype(np.float32)
        b = rng.normal(0, 0.5, cout).astype(np.float32)
        assert np.array_equal(E.head_1x1(a, Wt, b).view(np.uint32), orc.head(a, Wt, b).view(np.uint32))
        a2 = rng.normal(0, 1, (cin, H, W)).astype(np.float32)
        assert np.array_equal(E.head_1x1(a2, Wt, b).view(np.uint32), orc.head(a2, Wt, b).view(np.uint32))
