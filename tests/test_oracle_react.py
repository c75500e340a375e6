"""The v3 (ReActNet) CPU checker, oracle/bnn_oracle_react.c, pinned three
ways: known answers that only the reference's evaluation order gives,
closed forms against float64, and bit equality with the reference's own v3
kernels and engine built from its sources (oracle/_ref/libreactref.so,
skipped where that build is absent)."""
import os
import subprocess
from fractions import Fraction as F

import numpy as np
import pytest

from bnns_to_c_amd import blob as B
from bnns_to_c_amd import blob_react as R
from bnns_to_c_amd import synth

from test_oracle import _round_f32


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------ known answers --
def test_proj_order(rorc):
    """One chain over ci from +0 (csrc/bnn_realin_blk.h:59-70): x = [1e8, 1,
    -1e8] with unit weights sums to 0 in order; any other association gives 1."""
    x = np.array([1e8, 1.0, -1e8], np.float32).reshape(3, 1, 1)
    assert rorc.proj(x, np.ones((2, 3), np.float32))[:, 0, 0].tolist() == [0.0, 0.0]
    rng = np.random.default_rng(1)
    x = rng.standard_normal((24, 5, 7)).astype(np.float32)
    Wm = rng.normal(0, 0.3, (10, 24)).astype(np.float32)
    want = np.einsum("oc,chw->ohw", Wm.astype(np.float64), x.astype(np.float64))
    assert np.abs(rorc.proj(x, Wm) - want).max() < 1e-5


def test_conv3_order(rorc):
    """Input channels outermost, taps row-major inside, one chain
    (csrc/bnn_realin_blk.h:111-125).  At the centre of a 3x3 image,
    x[0] tap0 = 1e8, x[0] tap1 = 1, x[1] tap0 = -1e8 sums to 0 that way;
    taps outermost (or the v1 per-tap partial sums) give 1."""
    x = np.zeros((2, 3, 3), np.float32)
    x[0, 0, 0], x[0, 0, 1], x[1, 0, 0] = 1e8, 1.0, -1e8
    w = np.ones((8, 2, 3, 3), np.int8)
    out = rorc.conv3(x, w, np.ones(8, np.float32))
    assert out[0, 1, 1] == 0.0
    # alpha multiplies the finished sum once: 3 * (1/3) rounds differently
    # from summing alpha-scaled terms
    x = np.zeros((1, 1, 1), np.float32)
    x[0, 0, 0] = 3.0
    a = np.full(8, np.float32(1 / 3), np.float32)
    assert rorc.conv3(x, np.ones((8, 1, 3, 3), np.int8), a)[0, 0, 0] == np.float32(np.float32(1 / 3) * np.float32(3))


def test_conv3_closed_form(rorc):
    rng = np.random.default_rng(2)
    for cin, H, W, cout in [(5, 6, 6, 8), (3, 9, 7, 16), (120, 8, 8, 16), (4, 1, 5, 8)]:
        x = rng.standard_normal((cin, H, W)).astype(np.float32)
        w = np.where(rng.random((cout, cin, 3, 3)) < 0.5, -1, 1).astype(np.int8)
        alpha = rng.uniform(0.01, 0.1, cout).astype(np.float32)
        xp = np.zeros((cin, H + 2, W + 2))
        xp[:, 1:-1, 1:-1] = x
        want = np.zeros((cout, H, W))
        for oy in range(H):
            for ox in range(W):
                want[:, oy, ox] = np.tensordot(w.astype(np.float64), xp[:, oy:oy + 3, ox:ox + 3], 3)
        want *= alpha[:, None, None]
        assert np.abs(rorc.conv3(x, w, alpha) - want).max() < 1e-4


def _epi_exact(acc, res, A, Bv, m, w):
    """t = RN(RN(A*acc + RN(B + m)) + res) and the PReLU, from exact rationals"""
    out = []
    for i in range(len(acc)):
        Bm = _round_f32(F(float(Bv[i])) + F(float(m[i])))
        t = _round_f32(F(float(A[i])) * F(float(acc[i])) + F(float(Bm)))
        t = _round_f32(F(float(t)) + F(float(res[i])))
        out.append(t if t >= 0 else _round_f32(F(float(w[i])) * F(float(t))))
    return np.array(out, np.float32)


@pytest.mark.parametrize("kind", ["int", "real"])
def test_epilogue_fused_step(rorc, kind):
    """A*acc + (B + move1) is one fused step, the + res and the PReLU
    multiply round on their own (csrc/bnn_react_epi.c:38-53 as contracted
    by the reference build)."""
    rng = np.random.default_rng(3)
    n = 600
    acc = rng.integers(-300, 300, n).astype(np.int32) if kind == "int" else \
        rng.normal(0, 2, n).astype(np.float32)
    A = rng.uniform(0.01, 0.2, n).astype(np.float32)
    Bv = rng.normal(0, 1, n).astype(np.float32)
    m = rng.normal(0, 0.3, n).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, n).astype(np.float32)
    res = rng.normal(0, 1, n).astype(np.float32)
    want = _epi_exact(acc, res, A, Bv, m, w)
    got = rorc.epi(acc.reshape(n, 1, 1), res.reshape(n, 1, 1), A, Bv, m, w)[:, 0, 0]
    assert np.array_equal(bits(got), bits(want))
    # rounding A*acc first gives other values on these inputs
    Bm = (Bv + m).astype(np.float32)
    unf = (A * acc.astype(np.float32) + Bm).astype(np.float32) + res
    unf = np.where(unf >= 0, unf, w * unf).astype(np.float32)
    assert not np.array_equal(bits(unf), bits(want))


def test_epilogue_signed_zero(rorc):
    """t < 0 with prelu_w = 0 gives -0.0 (0 * negative), t = 0 stays +0."""
    P = np.array([-5, 0, 3], np.int32).reshape(3, 1, 1)
    one = np.ones(3, np.float32)
    z = np.zeros(3, np.float32)
    out = rorc.epi(P, np.zeros((3, 1, 1), np.float32), one, z, z, z)[:, 0, 0]
    assert bits(out).tolist() == [0x80000000, 0, bits(np.float32(3))[()]]


def test_tap(rorc):
    """bit = x + rsign > 0; an exact zero sum gives -1 (csrc/bnn_react_ops.c:72-84)"""
    x = np.array([1.0, -1.0, 0.5, 1e-30, 0.0, -0.0], np.float32).reshape(6, 1, 1)
    r = np.array([-1.0, 1.0, -0.25, 0.0, 0.0, 1e-30], np.float32)
    assert rorc.tap(x, r)[:, 0, 0].tolist() == [-1, -1, 1, 1, -1, 1]


def test_maxpool_real(rorc):
    """2x2 floor max reading (0,0), (0,1), (1,0), (1,1), first of equals kept
    (csrc/bnn_react_opt.c:61-66): -0 then +0 keeps -0, +0 then -0 keeps +0."""
    x = np.array([[[-0.0, 0.0], [0.0, 0.0]], [[0.0, -0.0], [-0.0, -0.0]]], np.float32)
    out = rorc.maxpool_real(x)
    assert bits(out).reshape(-1).tolist() == [0x80000000, 0]
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 9, 7)).astype(np.float32)
    want = x[:, :8, :6].reshape(3, 4, 2, 3, 2).max(axis=(2, 4))
    assert np.array_equal(rorc.maxpool_real(x), want)


def test_up_cat(rorc):
    rng = np.random.default_rng(5)
    for (sC, sH, sW), (xC, hH, hW) in [((4, 8, 8), (6, 4, 4)), ((3, 5, 7), (2, 2, 3)), ((2, 3, 3), (5, 1, 1))]:
        skip = rng.standard_normal((sC, sH, sW)).astype(np.float32)
        x = rng.standard_normal((xC, hH, hW)).astype(np.float32)
        up = np.repeat(np.repeat(x, 2, 1), 2, 2)
        dh, dw = sH - up.shape[1], sW - up.shape[2]
        up = np.pad(up, ((0, 0), (dh // 2, dh - dh // 2), (dw // 2, dw - dw // 2)))
        assert np.array_equal(rorc.up_cat(skip, x), np.concatenate([skip, up], 0))


def test_head_order(rorc):
    """bias first, then channels in order, one fused step each"""
    a = np.array([1.0, -1e8], np.float32).reshape(2, 1, 1)
    assert rorc.head(a, np.ones((1, 2), np.float32), np.array([1e8], np.float32))[0, 0, 0] == 0.0


def test_forward_stage_consistency(rorc):
    """The forward's stages are the kernels applied to each other's outputs
    in the reference's dataflow (csrc/bnn_model_react.c:6-14)."""
    b = synth.make_blob_react(seed=6, base=8)
    m = rorc.parse(R.to_bytes(b))
    x = synth.make_input(60, 1, 120, 16, 16)[0]
    logits, st = m.forward(x, stages=True)
    e1 = b.enc[0]
    assert np.array_equal(st["enc1.u1.proj"], rorc.proj(x, e1.proj1.W))
    assert np.array_equal(st["enc1.u1.conv"], rorc.conv3(x, e1.conv1.wsign, e1.conv1.alpha))
    d1 = b.dec[3]
    assert np.array_equal(st["dec1.u1.tap"], rorc.tap(st["dec1.cat"], d1.tap1.rsign))
    h2 = rorc.epi(st["dec1.u2.P"], st["dec1.h1"], d1.epi_a.A, d1.epi_a.B, d1.epi_a.move1, d1.epi_a.prelu_w)
    assert np.array_equal(bits(h2), bits(st["dec1.h2"]))
    assert np.array_equal(bits(logits), bits(rorc.head(h2, b.head.W, b.head.bias)))
    # the down path pools P and the highway separately, then one epilogue
    e2 = b.enc[1]
    dn = rorc.epi(st["enc2.pool.P"], rorc.maxpool_real(st["enc2.h1"]), e2.epi_b.A, e2.epi_b.B,
                  e2.epi_b.move1, e2.epi_b.prelu_w)
    assert np.array_equal(bits(dn), bits(st["enc2.down"]))


# ---------------------------------------------------------------- blob v3 --
def test_blob_roundtrip_and_reference_api(tmp_path):
    b = synth.make_blob_react(seed=7, base=8, coverage=True)
    data = R.to_bytes(b)
    assert R.to_bytes(R.from_bytes(data)) == data
    p = str(tmp_path / "m.blob")
    R.write(b, p)
    d = R.read_blob_react(p)
    assert d["version"] == 3 and set(d["blocks"]) == {n for n, _, _, _ in R.arch(8)}
    assert set(d["blocks"]["enc1"]) == {"conv1", "proj1", "epi1", "tap2", "conv2", "epi_skip", "epi_down"}
    assert set(d["blocks"]["dec2"]) == {"tap1", "conv1", "proj1", "epi1", "tap2", "conv2", "epi2"}
    # the reference's writer entry point from the folded-parameter dictionary
    fold = {"outc_W": b.head.W, "outc_b": b.head.bias}
    for (name, blk), (_, _, _, kind) in zip(b.blocks(), R.arch(8)):
        key = "bottleneck" if name == "bott" else name
        e = {"input_real": blk.input_real, "conv1_wsign": blk.conv1.signs(), "proj1_W": blk.proj1.W,
             "conv1_alpha": blk.conv1.alpha, "tap1_rsign": None if blk.tap1 is None else blk.tap1.rsign,
             "epi1": (blk.epi1.A, blk.epi1.B, blk.epi1.move1, blk.epi1.prelu_w),
             "conv2_wsign": blk.conv2.signs(), "tap2_rsign": blk.tap2.rsign}
        ea = (blk.epi_a.A, blk.epi_a.B, blk.epi_a.move1, blk.epi_a.prelu_w)
        if kind == "down":
            e["epi_skip"] = ea
            e["epi_down"] = (blk.epi_b.A, blk.epi_b.B, blk.epi_b.move1, blk.epi_b.prelu_w)
        else:
            e["epi2"] = ea
        fold[key] = e
    q = str(tmp_path / "f.blob")
    R.write_blob_react_from_fold(fold, q, base_channels=8)
    assert open(q, "rb").read() == data


def _mut(data: bytes, off: int, val: int) -> bytes:
    d = bytearray(data)
    d[off:off + 4] = np.int32(val).tobytes()
    return bytes(d)


def test_blob_checks(rorc):
    """Every corruption the C loader rejects (csrc/bnn_model_react.c:62-131)
    is rejected by the parser here and by the checker."""
    b = synth.make_blob_react(seed=8, base=8)
    data = R.to_bytes(b)
    # offsets: header ints at 4..24; enc1 conv1 (real) record starts at 24
    co, ci = b.enc[0].conv1.cout, b.enc[0].conv1.cin
    proj_at = 24 + 28 + co * ci * 9 + 4 * co
    epi_at = proj_at + 12 + 4 * co * ci
    tap2_at = epi_at + 12 + 16 * co
    bad = {
        "version": _mut(data, 4, 1),
        "upsampler": _mut(data, 20, 1),
        "conv tag": _mut(data, 24, 1),
        "proj tag": _mut(data, proj_at, 6),
        "proj dims": _mut(data, proj_at + 4, co + 1),
        "epi kind": _mut(data, epi_at + 4, 0),
        "tap tag": _mut(data, tap2_at, 5),
        "trailing": data + b"\0",
        "short": data[:-3],
    }
    for what, d in bad.items():
        with pytest.raises(B.BlobError):
            R.from_bytes(d)
        with pytest.raises(ValueError):
            rorc.parse(d)
    R.from_bytes(data)
    rorc.parse(data)


# ------------------------------------------------ against the reference v3 --
def test_kernels_vs_reference(rorc, rref):
    rng = np.random.default_rng(9)
    for cin, cout, H, W in [(120, 16, 32, 32), (48, 16, 17, 9), (384, 128, 2, 2), (20, 8, 3, 5)]:
        x = rng.standard_normal((cin, H, W)).astype(np.float32)
        Wm = rng.normal(0, 0.2, (cout, cin)).astype(np.float32)
        want = rorc.proj(x, Wm)
        assert np.array_equal(bits(rref.proj(x, Wm)), bits(want))
        assert np.array_equal(bits(rref.proj(x, Wm, blk=False)), bits(want))
    for cin, cout, H, W in [(120, 16, 32, 32), (7, 8, 9, 17), (3, 16, 1, 1), (5, 8, 2, 11)]:
        x = rng.standard_normal((cin, H, W)).astype(np.float32)
        w = np.where(rng.random((cout, cin, 3, 3)) < 0.5, -1, 1).astype(np.int8)
        al = rng.uniform(0.01, 0.1, cout).astype(np.float32)
        assert np.array_equal(bits(rref.conv3(x, w, al)), bits(rorc.conv3(x, w, al)))
    C, H, W = 12, 9, 11
    prm = [rng.uniform(0.01, 0.3, C).astype(np.float32), rng.normal(0, 1, C).astype(np.float32),
           rng.normal(0, 0.2, C).astype(np.float32), rng.uniform(-0.5, 0.5, C).astype(np.float32)]
    prm[3][:3] = 0.0
    res = rng.normal(0, 1, (C, H, W)).astype(np.float32)
    P = rng.integers(-400, 400, (C, H, W)).astype(np.int32)
    xr = rng.normal(0, 2, (C, H, W)).astype(np.float32)
    assert np.array_equal(bits(rref.epi(P, res, *prm)), bits(rorc.epi(P, res, *prm)))
    assert np.array_equal(bits(rref.epi(xr, res, *prm)), bits(rorc.epi(xr, res, *prm)))
    assert np.array_equal(bits(rref.epi_plain(P, res, *prm)), bits(rorc.epi_plain(P, res, *prm)))
    assert np.array_equal(bits(rref.epi_plain(xr, res, *prm)), bits(rorc.epi_plain(xr, res, *prm)))
    # the two forms round differently somewhere on these inputs
    assert not np.array_equal(bits(rorc.epi_plain(P, res, *prm)), bits(rorc.epi(P, res, *prm)))
    rs = rng.normal(0, 0.5, C).astype(np.float32)
    xr[0, 0, 0] = -rs[0]
    assert np.array_equal(rref.tap(xr, rs), rorc.tap(xr, rs))
    xz = np.where(rng.random((C, H, W)) < 0.5, np.float32(0.0), np.float32(-0.0)).astype(np.float32)
    for t in (xr, xz):
        assert np.array_equal(bits(rref.maxpool_real(t)), bits(rorc.maxpool_real(t)))
    want = P[:, :H // 2 * 2, :W // 2 * 2].reshape(C, H // 2, 2, W // 2, 2).max(axis=(2, 4))
    assert np.array_equal(rref.maxpool_P(P).astype(np.int32), want)
    Wh = rng.normal(0, 0.3, (3, C)).astype(np.float32)
    bh = rng.normal(0, 0.1, 3).astype(np.float32)
    assert np.array_equal(bits(rref.head(xr, Wh, bh)), bits(rorc.head(xr, Wh, bh)))


def test_bconv_i16_vs_oracle(orc, rref):
    """The v3 engine's int16 binary conv gives the v1 checker's integers"""
    rng = np.random.default_rng(10)
    for cin, cout, H, W in [(16, 16, 32, 32), (384, 128, 4, 4), (48, 16, 7, 5), (130, 8, 3, 10)]:
        a = np.where(rng.random((cin, H, W)) < 0.5, -1, 1).astype(np.int8)
        w = np.where(rng.random((cout, cin, 3, 3)) < 0.5, -1, 1).astype(np.int8)
        pk = B.pack_kidx(w)
        assert np.array_equal(rref.bconv(a, pk, cout).astype(np.int32), orc.bconv(a, pk, cout))


@pytest.mark.parametrize("seed,base,cov,H,W", [
    (0, 16, False, 32, 32), (1, 8, True, 17, 23), (2, 8, False, 80, 36), (3, 32, False, 16, 16),
    (4, 8, True, 33, 47), (5, 16, True, 32, 32),
    (6, 12, False, 32, 32), (7, 20, True, 17, 23)])  # enc1 Cout % 8 != 0: the general real conv
def test_forward_vs_reference(rorc, rref, tmp_path, seed, base, cov, H, W):
    """Whole forward bit-exact with the reference bnn_forward_react, odd
    sizes and (80 rows) its strip-wise enc1/dec1 included."""
    b = synth.make_blob_react(seed=seed, base=base, coverage=cov)
    data = R.to_bytes(b)
    p = tmp_path / "m.blob"
    p.write_bytes(data)
    h, _, nc = rref.load(str(p))
    try:
        x = synth.make_input(200 + seed, 1, 120, H, W)[0]
        want = rref.forward(h, x, nc)
    finally:
        rref.free(h)
    got = rorc.parse(data).forward(x)
    assert np.array_equal(bits(got), bits(want))


def test_patched_vs_reference(rorc, rref, tmp_path):
    b = synth.make_blob_react(seed=11, base=8)
    data = R.to_bytes(b)
    p = tmp_path / "m.blob"
    p.write_bytes(data)
    rng = np.random.default_rng(12)
    cube = rng.standard_normal((120, 40, 56)).astype(np.float32)
    m = rorc.parse(data)
    h, _, nc = rref.load(str(p))
    try:
        for P in (16, 32):
            want = rref.forward_patched(h, cube, nc, P)
            assert np.array_equal(bits(m.forward_patched(cube, P)), bits(want)), P
    finally:
        rref.free(h)


def test_cli_vs_reference(rorc, rref, tmp_path):
    """The reference CLI's output bytes, streaming and patch-wise file modes
    (csrc/main_react.c:60-99)."""
    from oracle.oracle import REACT_REF_CLI
    if not os.path.exists(REACT_REF_CLI):
        pytest.skip("reference CLI not built")
    b = synth.make_blob_react(seed=13, base=8)
    p = tmp_path / "m.blob"
    p.write_bytes(R.to_bytes(b))
    x = synth.make_input(14, 1, 120, 36, 52)[0]
    xin = tmp_path / "x.bin"
    x.tofile(xin)
    m = rorc.parse(R.to_bytes(b))
    for spec, want in ((str(xin), m.forward(x)), (f"patch16:{xin}", m.forward_patched(x, 16))):
        out = tmp_path / "o.bin"
        subprocess.run([REACT_REF_CLI, str(p), spec, str(out), "36", "52"], check=True, capture_output=True,
                       timeout=120)
        assert np.array_equal(np.fromfile(out, np.uint32), bits(want).reshape(-1)), spec


# -------------------------------------------------------- golden fixtures --
def _sha(a):
    import hashlib
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_stages_vs_golden(rorc, golden):
    """Every stage of the checker against the hashes of the reference's v3
    kernels chained as its engine chains them (tests/golden/make_golden.py)."""
    meta, arrays = golden
    for name, c in meta["react_cases"].items():
        b = synth.make_blob_react(seed=c["blob_seed"], base=c["base"], coverage=c["coverage"])
        data = R.to_bytes(b)
        import hashlib
        assert hashlib.sha256(data).hexdigest() == c["blob_sha256"], name
        x = synth.make_input(c["input_seed"], c["N"], 120, c["H"], c["W"])
        assert _sha(x) == c["input_sha256"], name
        m = rorc.parse(data)
        for n in range(c["N"]):
            logits, st = m.forward(x[n], stages=True)
            want = c["stages"][n]
            assert set(st) == set(want), name
            for k, v in st.items():
                assert _sha(v) == want[k], (name, n, k)
            assert np.array_equal(bits(logits), bits(arrays[f"{name}__logits"][n]))


def test_cli_golden(rorc, golden):
    meta, arrays = golden
    for name, c in meta["react_cli"].items():
        m = rorc.parse(R.to_bytes(synth.make_blob_react(seed=c["blob_seed"], base=c["base"])))
        x = synth.make_input(c["input_seed"], 1, 120, c["H"], c["W"])[0] if c["input_seed"] >= 0 else \
            synth.react_rand_cube(120, c["H"], c["W"])
        got = m.forward_patched(x, c["patch"]) if c["patch"] else m.forward(x)
        assert np.array_equal(bits(got), bits(arrays[f"{name}__cli"])), name
