"""Pinning the CPU checker (oracle/) before anything is compared against it.

Each kernel of the restatement is checked three ways where they apply:
against a brute-force or closed-form statement written independently here,
against the reference's own C built from its sources (oracle/_ref, skipped
when absent), and against invariants a plausible slip would break.
"""
import numpy as np
import pytest

from bnns_to_c_amd import blob as B
from bnns_to_c_amd import synth

# python/verify/bconv_harness.py:113-118 (Cin,H,W,Cout,kh,kw,pad,stride)
SELFTEST = [(8, 8, 8, 4, 3, 3, 1, 1), (16, 16, 16, 32, 3, 3, 1, 1), (32, 7, 5, 16, 3, 3, 1, 1),
            (3, 6, 6, 5, 3, 3, 0, 1)]
# csrc/bench_bconv.c:107-108 edge shapes {Cin,H,W,Cout}, k=3 pad=1 stride=1
EDGE = [(1, 1, 1, 4), (3, 1, 5, 4), (5, 5, 1, 8), (7, 4, 4, 6), (16, 3, 3, 16), (17, 5, 7, 8),
        (130, 3, 10, 8), (192, 3, 12, 8), (63, 4, 6, 8), (64, 4, 6, 8), (65, 4, 6, 8), (130, 3, 3, 8),
        (48, 9, 9, 16)]
# the 17 UNet binary convs (csrc/bench_bconv.c:57-67) at small spatial size
UNET = [(16, 16), (16, 32), (32, 32), (32, 64), (64, 64), (64, 128), (128, 128), (128, 256),
        (256, 256), (384, 128), (192, 64), (96, 32), (48, 16)]


def brute_P(a, w, pad, stride):
    """zero-padded +-1 correlation (python/verify/bconv_harness.py:93-108 restated)"""
    cin, H, W = a.shape
    cout, _, kh, kw = w.shape
    ap = np.zeros((cin, H + 2 * pad, W + 2 * pad), np.int64)
    ap[:, pad:pad + H, pad:pad + W] = a
    Ho, Wo = (H + 2 * pad - kh) // stride + 1, (W + 2 * pad - kw) // stride + 1
    P = np.zeros((cout, Ho, Wo), np.int64)
    wi = w.astype(np.int64)
    for oy in range(Ho):
        for ox in range(Wo):
            patch = ap[:, oy * stride:oy * stride + kh, ox * stride:ox * stride + kw]
            P[:, oy, ox] = np.tensordot(wi, patch, axes=([1, 2, 3], [0, 1, 2]))
    return P


def nvalid(H, W, kh, kw, pad, stride, cin):
    Ho, Wo = (H + 2 * pad - kh) // stride + 1, (W + 2 * pad - kw) // stride + 1
    ones = np.ones((1, H, W), np.int64)
    return brute_P(ones, np.ones((1, 1, kh, kw), np.int8), pad, stride)[0] * cin


def rand_pm1(rng, shape):
    return np.where(rng.random(shape) < 0.5, -1, 1).astype(np.int8)


@pytest.mark.parametrize("case", SELFTEST + [(c, h, w, o, 3, 3, 1, 1) for c, h, w, o in EDGE])
def test_bconv_vs_brute_force(orc, case):
    cin, H, W, cout, kh, kw, pad, stride = case
    rng = np.random.default_rng(hash(case) % 2**32)
    a = rand_pm1(rng, (cin, H, W))
    w = rand_pm1(rng, (cout, cin, kh, kw))
    want = brute_P(a, w, pad, stride)
    bits = orc.pack_kidx(w)
    assert np.array_equal(orc.bconv_naive(a, w, pad, stride), want)
    for kind in ("dense", "chan", "dispatch"):
        got = orc.bconv(a, bits, cout, kh, kw, pad, stride, kind=kind)
        assert np.array_equal(got, want), kind
    # invariants: P has the parity of N_valid and |P| <= N_valid
    nv = nvalid(H, W, kh, kw, pad, stride, cin)
    assert np.all((want - nv) % 2 == 0) and np.all(np.abs(want) <= nv)


@pytest.mark.parametrize("cin,cout", UNET)
def test_bconv_unet_shapes(orc, cin, cout):
    rng = np.random.default_rng(cin * 1000 + cout)
    a = rand_pm1(rng, (cin, 6, 7))
    w = rand_pm1(rng, (cout, cin, 3, 3))
    assert np.array_equal(orc.bconv(a, orc.pack_kidx(w), cout), brute_P(a, w, 1, 1))


def test_bconv_sign_symmetry(orc):
    # P(-a) = -P(a) and P(a, -w) = -P(a, w): a dropped sign or a swapped operand breaks these
    rng = np.random.default_rng(5)
    a = rand_pm1(rng, (40, 5, 6))
    w = rand_pm1(rng, (8, 40, 3, 3))
    P = orc.bconv(a, orc.pack_kidx(w), 8)
    assert np.array_equal(orc.bconv(-a, orc.pack_kidx(w), 8), -P)
    assert np.array_equal(orc.bconv(a, orc.pack_kidx(-w), 8), -P)


def test_bconv_zero_activation_semantics(orc):
    # the reference's XNOR kernels read a 0 activation as bit 0 (-1); only the
    # naive +-1 loop counts it as 0 (csrc/bnn_conv.c:66-68 vs 123, 162)
    rng = np.random.default_rng(6)
    a = rand_pm1(rng, (20, 4, 5))
    a[:, 1, 2] = 0
    w = rand_pm1(rng, (4, 20, 3, 3))
    a_m1 = np.where(a == 0, -1, a).astype(np.int8)
    assert np.array_equal(orc.bconv(a, orc.pack_kidx(w), 4, kind="dense"), brute_P(a_m1, w, 1, 1))
    assert np.array_equal(orc.bconv(a, orc.pack_kidx(w), 4, kind="chan"), brute_P(a_m1, w, 1, 1))
    assert np.array_equal(orc.bconv_naive(a, w), brute_P(a, w, 1, 1))


@pytest.mark.parametrize("C,H,W", [(8, 8, 8), (16, 6, 10), (4, 4, 4), (3, 5, 7)])
def test_maxpool(orc, C, H, W):
    # python/verify/maxpool_harness.py:77-89 cases, plus odd dims (floor mode)
    rng = np.random.default_rng(C * H * W)
    P = rng.integers(-300, 300, size=(C, H, W)).astype(np.int32)
    Ho, Wo = H // 2, W // 2
    want = P[:, :2 * Ho, :2 * Wo].reshape(C, Ho, 2, Wo, 2).max(axis=(2, 4))
    assert np.array_equal(orc.maxpool(P), want)


def test_fold_int_truth_table(orc):
    # every rule type on every P in a range, thresholds at and around parity edges
    P = np.arange(-40, 41, dtype=np.int32)
    rows = []
    for ty in range(7):
        for t in (-3, 0, 1, 2, 40, -41):
            for lo, hi in ((-5, 5), (0, 1), (3, 3), (6, -6)):
                rows.append((ty, t, lo, hi))
    ty, t, lo, hi = (np.array(v, np.int32) for v in zip(*rows))
    got = orc.fold_int(np.broadcast_to(P, (len(rows), 1, P.size)).copy(), ty, t, lo, hi)[:, 0, :]
    for i, (a, tt, l, h) in enumerate(rows):
        want = {0: np.full(P.size, tt > 0), 1: P >= tt, 2: P < tt, 3: (P >= l) & (P < h),
                4: (P < l) | (P >= h)}.get(a, np.zeros(P.size, bool))
        assert np.array_equal(got[i], np.where(want, 1, -1)), rows[i]


def _round_f32(q):
    """correctly rounded float32 of an exact rational (round-half-even)"""
    from fractions import Fraction
    f = np.float32(float(q))
    best = None
    for c in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        d = abs(Fraction(float(c)) - q)
        key = (d, int(np.frombuffer(np.float32(c).tobytes(), np.uint32)[0]) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return np.float32(best[1])


def test_fold_real_fused_step(orc):
    """z = A*x + B is one fused step (the reference build's vfmadd), then the
    slope multiply and the rsign add are separately rounded; r > 0 -> +1."""
    from fractions import Fraction as F
    rng = np.random.default_rng(9)
    n = 400
    A = rng.uniform(0.5, 1.5, n).astype(np.float32)
    B_ = rng.normal(0, 0.1, n).astype(np.float32)
    slope = rng.uniform(-0.5, 0.5, n).astype(np.float32)
    # rsign chosen so r lands within a few ulps of 0: the sign then depends on every rounding
    x = rng.normal(0, 1, n).astype(np.float32)
    z = [_round_f32(F(float(A[i])) * F(float(x[i])) + F(float(B_[i]))) for i in range(n)]
    z = [zz if zz >= 0 else _round_f32(F(float(slope[i])) * F(float(zz))) for i, zz in enumerate(z)]
    rsign = np.array([-zz + np.float32(k % 3 - 1) * np.spacing(zz) for k, zz in enumerate(z)], np.float32)
    want = np.array([1 if _round_f32(F(float(zz)) + F(float(rsign[i]))) > 0 else -1
                     for i, zz in enumerate(z)], np.int8)
    got = orc.fold_real(x.reshape(n, 1, 1), A, B_, slope, rsign)[:, 0, 0]
    assert np.array_equal(got, want)
    # the same rule with A*x rounded before + B gives other bits on these inputs,
    # so the test above does tell a fused step from an unfused one
    zu = [_round_f32(F(float(np.float32(A[i] * x[i]))) + F(float(B_[i]))) for i in range(n)]
    zu = [zz if zz >= 0 else _round_f32(F(float(slope[i])) * F(float(zz))) for i, zz in enumerate(zu)]
    want_u = np.array([1 if _round_f32(F(float(zz)) + F(float(rsign[i]))) > 0 else -1
                       for i, zz in enumerate(zu)], np.int8)
    assert (want_u != want).any()


def test_conv_real_order(orc):
    """The per-tap sum runs over ci in order from 0 (csrc/bnn_conv_realin.c:99-107):
    with 1 pixel, 1 tap and x = [1e8, 1, -1e8] the in-order float32 sum is 0;
    any other association returns 1."""
    x = np.array([1e8, 1.0, -1e8], np.float32).reshape(3, 1, 1)
    w = np.ones((1, 3, 3, 3), np.int8)
    out = orc.conv_real(x, w, np.ones(1, np.float32))
    assert out[0, 0, 0] == 0.0
    # taps add in row-major order into acc: 2x2 image, centre weight pattern
    x2 = np.zeros((1, 2, 2), np.float32)
    x2[0] = [[1e8, 1.0], [-1e8, 0.0]]
    w2 = np.ones((1, 1, 3, 3), np.int8)
    # output (0,0): taps (1,1)=1e8, (1,2)=1, (2,1)=-1e8, (2,2)=0 in that order -> 0
    assert orc.conv_real(x2, w2, np.ones(1, np.float32))[0, 0, 0] == 0.0


def test_conv_real_closed_form(orc):
    rng = np.random.default_rng(11)
    for cin, H, W, cout, pad in [(5, 6, 6, 4, 1), (3, 9, 7, 6, 1), (2, 5, 5, 3, 0), (120, 8, 8, 16, 1)]:
        # python/verify/realin_conv_harness.py:80 cases (+ the enc1 shape)
        x = rng.standard_normal((cin, H, W)).astype(np.float32)
        w = rand_pm1(rng, (cout, cin, 3, 3))
        alpha = rng.uniform(0.01, 0.1, cout).astype(np.float32)
        xp = np.zeros((cin, H + 2 * pad, W + 2 * pad))
        xp[:, pad:pad + H, pad:pad + W] = x
        Ho, Wo = H + 2 * pad - 2, W + 2 * pad - 2
        want = np.zeros((cout, Ho, Wo))
        for oy in range(Ho):
            for ox in range(Wo):
                want[:, oy, ox] = np.tensordot(w.astype(np.float64), xp[:, oy:oy + 3, ox:ox + 3], 3)
        want *= alpha[:, None, None]
        got = orc.conv_real(x, w, alpha, pad=pad)
        assert np.abs(got - want).max() < 1e-4


def test_conv_real_1x1_path(orc):
    rng = np.random.default_rng(12)
    x = rng.standard_normal((30, 5, 4)).astype(np.float32)
    w = rand_pm1(rng, (6, 30, 1, 1))
    alpha = rng.uniform(0.01, 0.1, 6).astype(np.float32)
    got = orc.conv_real(x, w, alpha, pad=0)
    want = np.einsum("oc,chw->ohw", w[:, :, 0, 0].astype(np.float64), x) * alpha[:, None, None]
    assert np.abs(got - want).max() < 1e-5


def test_head_closed_form(orc):
    # python/verify/head_harness.py:62 cases on +-1 input
    rng = np.random.default_rng(13)
    for cin, H, W, cout in [(16, 8, 8, 3), (32, 5, 7, 4), (8, 16, 16, 2)]:
        a = rand_pm1(rng, (cin, H, W)).astype(np.float32)
        Wt = rng.normal(0, 0.5, (cout, cin)).astype(np.float32)
        b = rng.normal(0, 0.5, cout).astype(np.float32)
        want = np.einsum("oc,chw->ohw", Wt.astype(np.float64), a) + b[:, None, None]
        assert np.abs(orc.head(a, Wt, b) - want).max() < 1e-5


def test_up_cat(orc):
    # python/verify/forward_driver.py:179-195 semantics, odd dims included
    rng = np.random.default_rng(14)
    for (sC, sH, sW), (xC, hH, hW) in [((4, 8, 8), (6, 4, 4)), ((3, 5, 7), (2, 2, 3)), ((2, 3, 3), (5, 1, 1))]:
        skip = rand_pm1(rng, (sC, sH, sW))
        x = rand_pm1(rng, (xC, hH, hW))
        up = np.repeat(np.repeat(x, 2, 1), 2, 2)
        dh, dw = sH - up.shape[1], sW - up.shape[2]
        up = np.pad(up, ((0, 0), (dh // 2, dh - dh // 2), (dw // 2, dw - dw // 2)))
        want = np.concatenate([skip, up], 0)
        assert np.array_equal(orc.up_cat(skip, x), want)


# --------------------------------------------------- against the reference C
@pytest.mark.parametrize("case", SELFTEST + [(c, h, w, o, 3, 3, 1, 1) for c, h, w, o in EDGE])
def test_bconv_vs_reference(orc, ref, case):
    cin, H, W, cout, kh, kw, pad, stride = case
    rng = np.random.default_rng(hash(case) % 2**31)
    a = rand_pm1(rng, (cin, H, W))
    w = rand_pm1(rng, (cout, cin, kh, kw))
    bits = ref.pack_weights(w)
    assert np.array_equal(orc.pack_kidx(w), bits)
    for kind in ("dense", "chan", "dispatch"):
        assert np.array_equal(orc.bconv(a, bits, cout, kh, kw, pad, stride, kind),
                              ref.bconv(a, bits, cout, kh, kw, pad, stride, kind)), kind
    assert np.array_equal(orc.bconv_naive(a, w, pad, stride), ref.bconv_naive(a, w, pad, stride))


def test_real_kernels_vs_reference(orc, ref):
    rng = np.random.default_rng(21)
    for cin, H, W, cout, k, pad in [(120, 12, 11, 16, 3, 1), (7, 5, 5, 3, 3, 0), (120, 6, 6, 8, 1, 0),
                                    (13, 1, 9, 5, 3, 1)]:
        x = (rng.standard_normal((cin, H, W)) * rng.choice([1e-3, 1, 1e3], (cin, 1, 1))).astype(np.float32)
        w = rand_pm1(rng, (cout, cin, k, k))
        alpha = rng.uniform(0.01, 0.1, cout).astype(np.float32)
        a = orc.conv_real(x, w, alpha, pad=pad)
        b = ref.conv_real(x, w, alpha, pad=pad)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    n = 200000
    xs = rng.normal(0, 1, (4, 1, n // 4)).astype(np.float32)
    A = rng.uniform(0.5, 1.5, 4).astype(np.float32)
    Bv = rng.normal(0, 0.1, 4).astype(np.float32)
    s = rng.uniform(-0.5, 0.5, 4).astype(np.float32)
    r = rng.normal(0, 0.1, 4).astype(np.float32)
    assert np.array_equal(orc.fold_real(xs, A, Bv, s, r), ref.fold_real(xs, A, Bv, s, r))
    a = rand_pm1(rng, (16, 9, 10)).astype(np.float32)
    Wt = rng.normal(0, 0.05, (3, 16)).astype(np.float32)
    bias = rng.normal(0, 0.05, 3).astype(np.float32)
    assert np.array_equal(orc.head(a, Wt, bias).view(np.uint32), ref.head(a, Wt, bias).view(np.uint32))
    # head on general float input: every step fused, as in the reference build
    a2 = rng.normal(0, 1, (16, 9, 10)).astype(np.float32)
    assert np.array_equal(orc.head(a2, Wt, bias).view(np.uint32), ref.head(a2, Wt, bias).view(np.uint32))
    P = rng.integers(-500, 500, (6, 9, 7)).astype(np.int32)
    assert np.array_equal(orc.maxpool(P), ref.maxpool(P))
    ty = rng.integers(0, 6, 6).astype(np.int32)
    t, lo, hi = (rng.integers(-50, 50, 6).astype(np.int32) for _ in range(3))
    assert np.array_equal(orc.fold_int(P, ty, t, lo, hi), ref.fold_int(P, ty, t, lo, hi))


@pytest.mark.parametrize("seed,base,cov,H,W", [(0, 16, False, 32, 32), (3, 16, True, 32, 32),
                                              (5, 8, False, 17, 23), (8, 16, False, 16, 16),
                                              (9, 32, False, 16, 16)])
def test_forward_vs_reference(orc, ref, blob_file, seed, base, cov, H, W):
    b = synth.make_blob(seed=seed, base=base, coverage=cov)
    path = blob_file(b)
    model = orc.parse(B.to_bytes(b))
    h, _, ncls = ref.load(path)
    x = synth.make_input(seed + 50, 2, 120, H, W)
    try:
        for n in range(2):
            got = model.forward(x[n])
            want = ref.forward(h, x[n], ncls)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finally:
        ref.free(h)


def test_forward_stages_vs_golden(orc, golden):
    """every stage of the restated forward against the reference kernel chain"""
    import hashlib
    meta, arrays = golden
    for name, c in meta["cases"].items():
        b = synth.make_blob(seed=c["blob_seed"], base=c["base"], coverage=c["coverage"])
        model = orc.parse(B.to_bytes(b))
        x = synth.make_input(c["input_seed"], c["N"], 120, c["H"], c["W"])
        for n in range(c["N"]):
            logits, st = model.forward(x[n], stages=True)
            assert set(st) == set(c["stages"][n]), name
            for k, v in st.items():
                assert hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest() == c["stages"][n][k], (name, k)
            assert np.array_equal(logits.view(np.uint32), arrays[f"{name}__logits"][n].view(np.uint32))


def test_batch_paths_agree(orc):
    b = synth.make_blob(seed=2)
    m = orc.parse(B.to_bytes(b))
    x = synth.make_input(3, 5)
    seq = m.forward_batch(x, parallel=False)
    par = m.forward_batch(x, parallel=True)
    assert np.array_equal(seq, par)
    assert np.array_equal(seq[4], m.forward(x[4]))


# ---------------------------------------------------------------- v2 stem --
@pytest.mark.parametrize("seed,base,stem,cov,H,W", [(1, 16, 16, False, 32, 32), (2, 8, 32, True, 17, 23),
                                                   (4, 32, 16, True, 16, 16), (6, 16, 24, False, 30, 34)])
def test_stem_forward_vs_reference(orc, ref, blob_file, seed, base, stem, cov, H, W):
    """the restated v2 forward against the reference's bnn_stem_forward
    (csrc/bnn_model_stem.c:168-255) built from its sources"""
    b = synth.make_blob_v2(seed=seed, base=base, stem=stem, coverage=cov)
    path = blob_file(b)
    model = orc.parse(B.to_bytes(b))
    h, _, ncls = ref.stem_load(path)
    x = synth.make_input(seed + 60, 2, 120, H, W)
    try:
        for n in range(2):
            got = model.forward(x[n])
            want = ref.stem_forward(h, x[n], ncls)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finally:
        ref.stem_free(h)


def test_stem_stages_vs_golden(orc, golden):
    """every v2 stage against the reference kernel chain (stem 1x1 conv,
    real fold, binary enc1 ...) recorded in tests/golden"""
    import hashlib
    meta, arrays = golden
    assert meta["stem_cases"]
    for name, c in meta["stem_cases"].items():
        b = synth.make_blob_v2(seed=c["blob_seed"], base=c["base"], stem=c["stem"], coverage=c["coverage"])
        assert hashlib.sha256(B.to_bytes(b)).hexdigest() == c["blob_sha256"], name
        model = orc.parse(B.to_bytes(b))
        x = synth.make_input(c["input_seed"], c["N"], 120, c["H"], c["W"])
        for n in range(c["N"]):
            logits, st = model.forward(x[n], stages=True)
            assert "stem.conv" in st and "enc1.conv1.P" in st and "enc1.conv1" not in st
            assert set(st) == set(c["stages"][n]), name
            for k, v in st.items():
                assert hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest() == c["stages"][n][k], (name, k)
            assert np.array_equal(logits.view(np.uint32), arrays[f"{name}__logits"][n].view(np.uint32))


def test_stem_blob_checks(orc):
    b = synth.make_blob_v2(seed=5)
    data = bytearray(B.to_bytes(b))
    m = orc.parse(bytes(data))
    assert m.forward(synth.make_input(1, 1)[0]).shape == (3, 32, 32)
    bad = bytearray(data)
    bad[28:32] = (2).to_bytes(4, "little")          # n_stem_layers = 2
    with pytest.raises(Exception, match="n_stem_layers"):
        orc.parse(bytes(bad))
