"""Isolated binary conv layers at the benchmark shapes, on device buffers.

cfg1: 64->64, 64x64, batch 256, output the int32 accumulator P.
cfg2: 128->128, 32x32, batch 1024, rule on P (skip bits), 2x2 max of P and a
second rule (down bits at 16x16).  Patches are checked against the checker;
the full batches also through size-independent properties: P(-a) = -P(a),
the parity and range of P, and the fused fold+pool agreeing with the plain
P kernel followed by the rules (csrc/bnn_fold.c:37-60, bnn_maxpool.c:28-48).
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from bnns_to_c_amd import blob as B
from bnns_to_c_amd import engine as E
from bnns_to_c_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as T
    assert T.cuda.is_available(), "GPU tests need a visible device"
    return T


def _nvalid(H, W, cin):
    r = np.full(H, 3)
    r[0] -= 1
    r[-1] -= 1
    c = np.full(W, 3)
    c[0] -= 1
    c[-1] -= 1
    if H == 1:
        r[:] = 1
    if W == 1:
        c[:] = 1
    return np.outer(r, c) * cin


def _pack_on_device(T, a):
    N, Cc, H, W = a.shape
    da = T.from_numpy(a).cuda()
    dw = T.empty((N, H, W, (Cc + 31) // 32), dtype=T.int32, device="cuda")
    E.pack_act_device(da.data_ptr(), dw.data_ptr(), N, Cc, H, W, T.cuda.current_stream().cuda_stream)
    return dw


def test_pack_act_device(torch):
    a = synth.make_bits(1, 3, 5, 7, 70)
    dw = _pack_on_device(torch, a)
    torch.cuda.synchronize()
    assert np.array_equal(dw.cpu().numpy().view(np.uint32), E.pack_bits_nhwc(a))


@pytest.mark.parametrize("N,H,W,cin,cout", [(4, 64, 64, 64, 64), (3, 9, 11, 40, 24), (2, 2, 2, 256, 256)])
def test_layer_P_vs_checker(torch, orc, N, H, W, cin, cout):
    a = synth.make_bits(2, N, H, W, cin)
    w = synth.make_signs(3, cout, cin)
    bits = B.pack_kidx(w)
    L = E.ConvLayer(bits, cin, cout)
    act = _pack_on_device(torch, a)
    P = torch.empty((N, cout, H, W), dtype=torch.int32, device="cuda")
    L.P_device(act.data_ptr(), N, H, W, P.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = P.cpu().numpy()
    for n in range(N):
        assert np.array_equal(got[n], orc.bconv(a[n], bits, cout)), n


def test_cfg1_full_batch(torch, orc):
    N, H, W, C = 256, 64, 64, 64
    a = synth.make_bits(10, N, H, W, C)
    w = synth.make_signs(11, C, C)
    bits = B.pack_kidx(w)
    L = E.ConvLayer(bits, C, C)
    s = torch.cuda.current_stream().cuda_stream
    act = _pack_on_device(torch, a)
    actn = _pack_on_device(torch, (-a).astype(np.int8))
    P = torch.empty((N, C, H, W), dtype=torch.int32, device="cuda")
    Pn = torch.empty_like(P)
    L.P_device(act.data_ptr(), N, H, W, P.data_ptr(), s)
    L.P_device(actn.data_ptr(), N, H, W, Pn.data_ptr(), s)
    torch.cuda.synchronize()
    assert torch.equal(Pn, -P)
    nv = torch.from_numpy(_nvalid(H, W, C)).cuda()
    assert bool(((P - nv) % 2 == 0).all()) and bool((P.abs() <= nv).all())
    got = P.cpu().numpy()
    # every patch against the checker (its C calls release the GIL)
    with ThreadPoolExecutor(8) as ex:
        bad = [n for n, ok in enumerate(ex.map(lambda n: np.array_equal(got[n], orc.bconv(a[n], bits, C)), range(N)))
               if not ok]
    assert not bad, bad[:8]


def _host_fold(P, ty, t, lo, hi):
    Pb = P
    t = t[None, :, None, None]
    lo = lo[None, :, None, None]
    hi = hi[None, :, None, None]
    ty = ty[None, :, None, None]
    on = np.where(ty == 0, t > 0, np.where(ty == 1, Pb >= t, np.where(ty == 2, Pb < t, np.where(
        ty == 3, (Pb >= lo) & (Pb < hi), np.where(ty == 4, (Pb < lo) | (Pb >= hi), False)))))
    return np.where(on, 1, -1).astype(np.int8)


@pytest.mark.parametrize("N,H,W,C,cov", [(64, 32, 32, 128, False), (8, 13, 9, 40, True), (16, 2, 2, 256, False)])
def test_fold_pool_vs_checker(torch, orc, N, H, W, C, cov):
    a = synth.make_bits(20, N, H, W, C)
    w = synth.make_signs(21, C, C)
    bits = B.pack_kidx(w)
    if cov:
        f1 = synth.make_rules(24, C, C * 9, coverage=True)
        f2 = synth.make_rules(25, C, C * 9, coverage=True)
    else:
        f1 = synth.make_thresholds(22, C, C * 9 // 4)
        f2 = synth.make_thresholds(23, C, C * 9 // 4)
    L = E.ConvLayer(bits, C, C, f1, f2)
    act = _pack_on_device(torch, a)
    cw = (C + 31) // 32
    skip = torch.empty((N, H, W, cw), dtype=torch.int32, device="cuda")
    down = torch.empty((N, H // 2, W // 2, cw), dtype=torch.int32, device="cuda")
    down2 = torch.empty_like(down)
    s = torch.cuda.current_stream().cuda_stream
    L.fold_pool_device(act.data_ptr(), N, H, W, skip.data_ptr(), down.data_ptr(), s)
    L.fold_pool_device(act.data_ptr(), N, H, W, None, down2.data_ptr(), s)
    torch.cuda.synchronize()
    assert torch.equal(down, down2)
    sk = E.unpack_bits_nhwc(skip.cpu().numpy().view(np.uint32), C)
    dn = E.unpack_bits_nhwc(down.cpu().numpy().view(np.uint32), C)
    for n in range(N):
        P = orc.bconv(a[n], bits, C)
        assert np.array_equal(sk[n], orc.fold_int(P, *f1)), n
        assert np.array_equal(dn[n], orc.fold_int(orc.maxpool(P), *f2)), n


def test_cfg2_full_batch(torch, orc):
    N, H, W, C = 1024, 32, 32, 128
    a = synth.make_bits(30, N, H, W, C)
    w = synth.make_signs(31, C, C)
    bits = B.pack_kidx(w)
    f1 = synth.make_thresholds(32, C, 288)
    f2 = synth.make_thresholds(33, C, 288)
    L = E.ConvLayer(bits, C, C, f1, f2)
    s = torch.cuda.current_stream().cuda_stream
    act = _pack_on_device(torch, a)
    P = torch.empty((N, C, H, W), dtype=torch.int32, device="cuda")
    skip = torch.empty((N, H, W, 4), dtype=torch.int32, device="cuda")
    down = torch.empty((N, H // 2, W // 2, 4), dtype=torch.int32, device="cuda")
    L.P_device(act.data_ptr(), N, H, W, P.data_ptr(), s)
    L.fold_pool_device(act.data_ptr(), N, H, W, skip.data_ptr(), down.data_ptr(), s)
    torch.cuda.synchronize()
    Ph = P.cpu().numpy()
    pooled = Ph.reshape(N, C, H // 2, 2, W // 2, 2).max(axis=(3, 5))
    assert np.array_equal(E.unpack_bits_nhwc(skip.cpu().numpy().view(np.uint32), C), _host_fold(Ph, *f1))
    assert np.array_equal(E.unpack_bits_nhwc(down.cpu().numpy().view(np.uint32), C), _host_fold(pooled, *f2))
    sk = E.unpack_bits_nhwc(skip.cpu().numpy().view(np.uint32), C)
    dn = E.unpack_bits_nhwc(down.cpu().numpy().view(np.uint32), C)

    def patch_ok(n):
        Pn = orc.bconv(a[n], bits, C)
        return (np.array_equal(Ph[n], Pn) and np.array_equal(sk[n], orc.fold_int(Pn, *f1))
                and np.array_equal(dn[n], orc.fold_int(orc.maxpool(Pn), *f2)))

    # every patch's P, skip bits and pooled bits against the checker
    with ThreadPoolExecutor(8) as ex:
        bad = [n for n, ok in enumerate(ex.map(patch_ok, range(N))) if not ok]
    assert not bad, bad[:8]


@pytest.mark.parametrize("C,H,W", [(8, 6, 6), (24, 5, 8), (40, 4, 4), (16, 32, 32)])
def test_partial_words_fully_written(torch, orc, C, H, W):
    """Outputs whose channel count is not a multiple of 32 still get whole
    words: the bits above C come back 0 even over a buffer full of ones."""
    N = 4
    a = synth.make_bits(40, N, H, W, C)
    w = synth.make_signs(41, C, C)
    bits = B.pack_kidx(w)
    f1 = synth.make_rules(42, C, C * 9, coverage=True)
    f2 = synth.make_rules(43, C, C * 9, coverage=True)
    L = E.ConvLayer(bits, C, C, f1, f2)
    act = _pack_on_device(torch, a)
    cw = (C + 31) // 32
    skip = torch.full((N, H, W, cw), -1, dtype=torch.int32, device="cuda")
    down = torch.full((N, H // 2, W // 2, cw), -1, dtype=torch.int32, device="cuda")
    L.fold_pool_device(act.data_ptr(), N, H, W, skip.data_ptr(), down.data_ptr(),
                       torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for t in (skip, down):
        words = t.cpu().numpy().view(np.uint32)
        if C % 32:
            assert np.all(words[..., -1] >> np.uint32(C % 32) == 0)
    sk = E.unpack_bits_nhwc(skip.cpu().numpy().view(np.uint32), C)
    for n in range(N):
        assert np.array_equal(sk[n], orc.fold_int(orc.bconv(a[n], bits, C), *f1))
