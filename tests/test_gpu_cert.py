"""The certified first conv (launch_real_cert, csrc/bnn_real_cert.hip): the
enc1.act1 bits it writes equal the checker's (csrc/bnn_conv_realin.c:98-111
then csrc/bnn_fold.c:62-77), on inputs built so that the approximation's
bound cannot decide many outputs and the reference-order recompute must:

* every band +-1, so tap sums are integers, and each channel's fold placed
  exactly on one integer sum: about one output in a hundred sits on z = 0;
* bands scaled by 2^-20 .. 2^20, zero rows, and an infinity and a NaN;
* the scene path (edge patches partly outside the cube);
* rows wider than 32 (tiles of 32 columns whose edge outputs read the
  neighbouring columns from a one-column halo either side), with undecided
  and non-finite outputs at the tile edges.

The debug forward reports the act1 bits of the certified kernel (its float
conv output comes from the exact-order kernel); the plain forward's logits
must match too, and a model loaded with BNN_CERT=0 (exact-order kernel for
the bits) must give bit-identical logits on a larger batch.
"""
import os

import numpy as np
import pytest

from bnns_to_c_amd import blob as B
from bnns_to_c_amd import engine as E
from bnns_to_c_amd import scene
from bnns_to_c_amd import synth

pytestmark = pytest.mark.gpu


def _engine(tmp_path, b, name="m.blob", cert=True):
    p = tmp_path / name
    p.write_bytes(B.to_bytes(b))
    old = os.environ.get("BNN_CERT")
    if cert:
        os.environ.pop("BNN_CERT", None)
    else:
        os.environ["BNN_CERT"] = "0"
    try:
        return E.Engine(str(p))
    finally:
        if old is None:
            os.environ.pop("BNN_CERT", None)
        else:
            os.environ["BNN_CERT"] = old


def _bits_equal(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32) if a.dtype == np.float32 else a,
                          np.asarray(b).view(np.uint32) if b.dtype == np.float32 else b)


def _check(eng, model, x):
    logits, st = eng.forward_debug(x)
    plain = eng.forward_batch(x)
    for n in range(x.shape[0]):
        want, ref = model.forward(x[n], stages=True)
        assert np.array_equal(st["enc1.act1"][n], ref["enc1.act1"]), ("enc1.act1", n)
        assert _bits_equal(logits[n], want), ("logits", n)
        assert _bits_equal(plain[n], want), ("plain logits", n)


@pytest.mark.parametrize("H,W,base", [(32, 32, 16), (24, 76, 16), (24, 96, 16), (32, 32, 32), (24, 76, 32),
                                       (24, 40, 24)])
def test_cert_threshold_ties(tmp_path, orc, H, W, base):
    """Ties on the fold's threshold, so that many outputs are undecided and
    recomputed; bases 24 and 32 run both 16-channel groups in one block,
    whose recompute reads sign masks and halo columns from global memory."""
    b = synth.make_blob(seed=41, base=base)
    rng = np.random.default_rng(42)
    N = 2
    x = rng.choice(np.array([-1.0, 1.0], np.float32), size=(N, 120, H, W))
    model = orc.parse(B.to_bytes(b))
    _, ref = model.forward(x[0], stages=True)
    conv = ref["enc1.conv1"]  # alpha * tap sum, [16][H][W]
    act = b.enc_act1[0]
    A = act.A.astype(np.float32)
    Bv = act.B.copy()
    rs = act.rsign.copy()
    for c in range(conv.shape[0]):
        o0 = conv[c, 5 + c % 16, 3 + c % 16]  # one of the patch's own outputs
        Bv[c] = np.float32(-(A[c] * o0))
        rs[c] = np.float32(0.0) if c % 2 == 0 else np.float32(1e-30)
    act.B = Bv.astype(np.float32)
    act.rsign = rs.astype(np.float32)
    model = orc.parse(B.to_bytes(b))
    # how many outputs the fold puts on (or within a few ulps of) z = 0
    _, ref = model.forward(x[0], stages=True)
    z = A[:, None, None] * ref["enc1.conv1"] + Bv[:, None, None]
    assert (np.abs(z) <= 1e-5).sum() > 50
    eng = _engine(tmp_path, b)
    _check(eng, model, x)
    eng.close()


def test_cert_wide_range_and_nonfinite(tmp_path, orc):
    b = synth.make_blob(seed=43)
    rng = np.random.default_rng(44)
    N = 3
    x = rng.standard_normal((N, 120, 32, 32), dtype=np.float32)
    x *= (2.0 ** rng.integers(-20, 21, size=(1, 120, 1, 1))).astype(np.float32)
    x[0, :, 7, :] = 0.0          # a zero row
    x[1, :, :, 12] = 0.0         # a zero column
    x[1, 3, 20, 20] = np.inf     # non-finite inputs reach the recompute
    x[2, 77, 9, 30] = np.nan
    model = orc.parse(B.to_bytes(b))
    eng = _engine(tmp_path, b)
    _check(eng, model, x)
    eng.close()


@pytest.mark.parametrize("base", [16, 32])
def test_cert_wide_edges_nonfinite(tmp_path, orc, base):
    """Rows of 72 (tiles 0-31, 32-63, 64-71): an infinity, a NaN, a zero
    column and large values in the columns either side of each tile edge,
    which the edge outputs read through the halo."""
    b = synth.make_blob(seed=47, base=base)
    rng = np.random.default_rng(48)
    x = rng.standard_normal((3, 120, 20, 72), dtype=np.float32)
    x[0, 5, 4, 31] = np.inf
    x[0, 9, 11, 32] = -np.inf
    x[1, 77, 9, 63] = np.nan
    x[1, 3, 15, 64] = np.nan
    x[2, :, :, 32] = 0.0
    x[2, :, 6, 30:34] *= np.float32(1e6)
    model = orc.parse(B.to_bytes(b))
    eng = _engine(tmp_path, b)
    _check(eng, model, x)
    eng.close()


@pytest.mark.parametrize("base,H,W", [(16, 20, 32), (32, 20, 32), (16, 16, 72), (32, 16, 72)])
def test_cert_dense_infinities(tmp_path, orc, base, H, W):
    """Infinities of both signs on a grid (every third row and column in one
    band, one sample of each sign, one mixed), so that every output row has
    far more undecided outputs than one recompute batch of seven takes, in
    both 64-pixel halves of a wave and at the tile edges of wide rows; a
    window holding both signs sums to NaN."""
    b = synth.make_blob(seed=49, base=base)
    rng = np.random.default_rng(50)
    x = rng.standard_normal((3, 120, H, W), dtype=np.float32)
    x[0, 11, ::3, ::3] = np.inf
    x[1, 60, 1::3, ::3] = -np.inf
    x[2, 2, ::3, ::3] = np.inf
    x[2, 90, ::3, 1::3] = -np.inf
    model = orc.parse(B.to_bytes(b))
    eng = _engine(tmp_path, b)
    _check(eng, model, x)
    eng.close()


@pytest.mark.parametrize("N,H,W,base", [(100, 33, 32, 16), (200, 32, 32, 16), (250, 20, 32, 16), (60, 47, 44, 16),
                                         (40, 32, 64, 32), (3, 17, 36, 32)])
def test_cert_row_parts(tmp_path, orc, N, H, W, base):
    """A launch of fewer patches than a round of the GPU holds splits each
    patch's rows over two or four blocks, each starting one input row above
    its first output row: 100 patches of 33 rows in parts of 9, 9, 9 and 6;
    200 of 32 in halves; 250 of 20 in halves; tiled rows of 44 and 64 (both
    16-channel groups in one block at base 32), 17 rows in parts of 9 and 8.
    Logits of the whole batch bitwise against the order-exact kernel, act1
    bits and logits of three patches against the checker."""
    b = synth.make_blob(seed=70 + H, base=base)
    x = synth.make_input(71 + W, N, 120, H, W)
    x[N // 2, 40, H // 2, :] = np.inf  # an undecided row in a middle part
    fast = _engine(tmp_path, b, "a.blob", cert=True)
    exact = _engine(tmp_path, b, "b.blob", cert=False)
    assert _bits_equal(fast.forward_batch(x), exact.forward_batch(x))
    model = orc.parse(B.to_bytes(b))
    _check(fast, model, x[[0, N // 2, N - 1]])
    fast.close()
    exact.close()


@pytest.mark.parametrize("base,H,W", [(16, 32, 32), (32, 32, 32), (8, 16, 16), (16, 20, 28), (24, 32, 16),
                                       (16, 16, 72), (8, 20, 100), (32, 16, 256), (16, 36, 36)])
def test_cert_shapes(tmp_path, orc, base, H, W):
    b = synth.make_blob(seed=45 + base, base=base)
    x = synth.make_input(46 + H, 2, 120, H, W)
    model = orc.parse(B.to_bytes(b))
    eng = _engine(tmp_path, b)
    _check(eng, model, x)
    eng.close()


@pytest.mark.parametrize("nb,base,H,W", [(4, 8, 16, 16), (16, 16, 32, 32), (28, 16, 32, 32), (64, 16, 32, 40),
                                          (100, 8, 20, 32), (112, 16, 32, 32), (128, 16, 32, 32)])
def test_cert_band_counts(tmp_path, orc, nb, base, H, W):
    """Band counts from 4 to 128 (a wave's quarter of the channels from 1 to
    32, partly empty 8-channel loads, the guarded conversion below 112
    bands), each bit for bit against the checker."""
    b = synth.make_blob(seed=60 + nb, base=base, n_bands=nb)
    x = synth.make_input(61 + nb, 2, nb, H, W)
    model = orc.parse(B.to_bytes(b))
    eng = _engine(tmp_path, b)
    _check(eng, model, x)
    eng.close()


def test_cert_vs_exact_order_batch(tmp_path):
    b = synth.make_blob(seed=47)
    x = synth.make_input(48, 96, 120, 32, 32)
    x[5] *= np.float32(1e-3)
    x[6] += np.float32(3.0)
    fast = _engine(tmp_path, b, "a.blob", cert=True)
    exact = _engine(tmp_path, b, "b.blob", cert=False)
    assert _bits_equal(fast.forward_batch(x), exact.forward_batch(x))
    fast.close()
    exact.close()


def test_cert_wide_vs_exact_order(tmp_path):
    """Rows wider than 32 run as tiles of 32 columns with a halo: the large-tile
    configuration's shape (256 x 256, base 32: two 16-channel groups) against
    the order-exact kernel."""
    b = synth.make_blob(seed=51, base=32)
    x = synth.make_input(52, 2, 120, 256, 256)
    x[1, :, :, 100:140] *= np.float32(1e-4)  # a band of small values across tile edges
    fast = _engine(tmp_path, b, "a.blob", cert=True)
    exact = _engine(tmp_path, b, "b.blob", cert=False)
    assert _bits_equal(fast.forward_batch(x), exact.forward_batch(x))
    fast.close()
    exact.close()


def test_cert_scene(tmp_path, orc):
    b = synth.make_blob(seed=49)
    rng = np.random.default_rng(50)
    cube = rng.standard_normal((120, 70, 100), dtype=np.float32)
    cube += rng.uniform(-0.5, 0.5, (120, 1, 1)).astype(np.float32)
    model = orc.parse(B.to_bytes(b))
    eng = _engine(tmp_path, b)
    got = eng.forward_patched(cube, 32)
    want = scene.stitch(model.forward_batch(scene.cut(cube, 32)), 70, 100)
    assert _bits_equal(got, want)
    eng.close()


def test_cert_nan_windows_decided(tmp_path, orc):
    """An output whose 3x3 window holds a NaN has the reference's tap sum NaN
    and fold bit 0 for any parameters, so it is decided without a
    reference-order recompute: a patch of NaNs recomputes nothing, and a
    patch with NaN blocks only what its finite outputs need."""
    b = synth.make_blob(seed=53)
    x = synth.make_input(54, 3, 120, 32, 32)
    x[0] = np.nan                      # every window
    x[1, :, 4:12, 6:20] = np.nan       # a block in every band
    x[2, 17, :, 9] = np.nan            # a column of one band
    model = orc.parse(B.to_bytes(b))
    eng = _engine(tmp_path, b)
    eng.cert_stats()
    _check(eng, model, x)
    eng.cert_stats()
    eng.forward_batch(x[:1])
    und, outs = eng.cert_stats()
    assert (und, outs) == (0, 16 * 32 * 32)
    eng.close()


def test_cert_stats_counts(tmp_path):
    """bnn_cert_stats: outputs certified and recomputed since the last call,
    then both reset; the exact-order kernel reports none."""
    b = synth.make_blob(seed=55)
    x = synth.make_input(56, 64, 120, 32, 32)
    eng = _engine(tmp_path, b)
    eng.cert_stats()
    eng.forward_batch(x)
    und, outs = eng.cert_stats()
    assert outs == 64 * 16 * 32 * 32
    assert 0 < und < outs // 1000
    assert eng.cert_stats() == (0, 0)
    eng.close()
    ex = _engine(tmp_path, b, "e.blob", cert=False)
    ex.forward_batch(x)
    assert ex.cert_stats() == (0, 0)
    ex.close()


def test_cert_unaligned_input(tmp_path):
    """An input that is not 16-byte aligned runs (on the exact-order kernel,
    the certified one stages 16-byte groups) with the same logits as an
    aligned copy."""
    import torch

    b = synth.make_blob(seed=57)
    eng = _engine(tmp_path, b)
    N = 8
    x = synth.make_input(58, N, 120, 32, 32)
    buf = torch.empty(x.size + 1, dtype=torch.float32, device="cuda")
    buf[1:] = torch.from_numpy(x.ravel()).cuda()
    y = torch.empty((N, b.n_classes, 32, 32), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    eng.forward_device(buf.data_ptr() + 4, N, 32, 32, y.data_ptr(), None)
    torch.cuda.synchronize()
    want = eng.forward_batch(x)
    assert _bits_equal(y.cpu().numpy(), want)
    eng.close()
