"""The v3 (ReActNet, real-highway) model on the GPU (csrc/bnn_model_react.c):
the enc1 conv + projection + epilogue kernel on the matrix cores, the 1x1
projections on the matrix cores, and the binary convs with the RPReLU,
skip/down and head epilogues.

Every stage the GPU materialises (float highway stages, tap bits as +-1,
accumulators P, pooled P) is compared bit for bit with the checker
(oracle/bnn_oracle_react.c, itself pinned to the reference's v3 build), and
with the stage hashes, logits and CLI outputs of the reference's own v3
code (tests/golden).  Parameter sets cover base widths 8 to 32 (one and two
16-channel groups, a partial group), band counts that are not a multiple of
the 8-channel chunk, odd image sizes (the concat's pad pixel) and a tall
image the reference runs in row strips."""
import hashlib
import os
import subprocess

import numpy as np
import pytest

from bnns_to_c_amd import blob_react as R
from bnns_to_c_amd import engine as E
from bnns_to_c_amd import synth

pytestmark = pytest.mark.gpu


def _same(a, b):
    if a.dtype == np.float32:
        return np.array_equal(np.ascontiguousarray(a).view(np.uint32), np.ascontiguousarray(b).view(np.uint32))
    return np.array_equal(a, b)


def _engine(tmp_path, b, name="m.blob"):
    p = tmp_path / name
    p.write_bytes(R.to_bytes(b))
    return E.ReactEngine(str(p)), str(p)


# stages the checker names that the GPU never materialises: the decoders'
# concat and its tap (read in place from the skip and upsample), the pooled
# highway (pooled inside the down epilogue)
def _gpu_names(names):
    return {n for n in names if not (n.endswith(".cat") or n.endswith(".pool.h")
                                     or (n.startswith("dec") and n.endswith(".u1.tap")))}


def _check_stages(eng, model, x):
    logits, st = eng.forward_debug(x)
    for n in range(x.shape[0]):
        want, ref_st = model.forward(x[n], stages=True)
        assert set(st) == _gpu_names(ref_st), sorted(set(st) ^ _gpu_names(ref_st))
        for name, arr in st.items():
            if name == "logits":
                continue
            assert _same(arr[n], ref_st[name]), (name, n)
        assert _same(logits[n], want), n
    return logits


@pytest.mark.parametrize("seed,base,nb,cov,N,H,W", [
    (0, 16, 120, False, 3, 32, 32),
    (1, 8, 120, True, 2, 17, 23),     # odd sizes: concat pad pixels, floor pools
    (2, 32, 120, False, 2, 16, 16),   # two 16-channel groups in enc1, head of 32
    (3, 24, 13, True, 2, 30, 34),     # a partial channel group; 13 bands: a partial chunk
    (4, 16, 7, False, 2, 33, 47),
    (5, 8, 1, False, 1, 16, 16),      # one band
    (6, 16, 121, True, 1, 80, 36),    # taller than the reference's 64-row strips
    (7, 48, 120, False, 1, 32, 32),   # head over 48 channels: dec1 then the separate head kernel
    (8, 12, 120, False, 2, 32, 32),   # enc1 Cout % 8 != 0: the general-order conv, then the tail kernel
    (9, 20, 13, True, 2, 30, 34),     # the same with two channel groups, a partial chunk, odd sizes
])
def test_react_stages_vs_checker(tmp_path, rorc, seed, base, nb, cov, N, H, W):
    b = synth.make_blob_react(seed=seed, base=base, n_bands=nb, coverage=cov)
    eng, _ = _engine(tmp_path, b)
    assert (eng.version, eng.n_bands, eng.n_classes) == (3, nb, 3)
    model = rorc.parse(R.to_bytes(b))
    x = synth.make_input(seed + 300, N, nb, H, W)
    _check_stages(eng, model, x)
    eng.close()


def test_react_enc1_general_signs(tmp_path, rorc):
    """enc1.conv1 with Cout % 8 != 0 runs the reference's general real conv
    (csrc/bnn_model_react.c:152-158) for any int8 sign, here 0 and +-2 (the
    products stay exact): the engine's vector-ALU first conv, then the tail
    kernel; every stage matches the checker.  With Cout % 8 == 0 the
    register-blocked path needs +-1 signs, and such a blob is refused."""
    for base, ok in ((12, True), (16, False)):
        b = synth.make_blob_react(seed=30 + base, base=base)
        w = b.enc[0].conv1.wsign.copy()
        flat = w.reshape(-1)
        rng = np.random.default_rng(31)
        idx = rng.choice(flat.size, 64, replace=False)
        flat[idx[:32]] = 0
        flat[idx[32:48]] = 2
        flat[idx[48:]] = -2
        b.enc[0].conv1.wsign = w
        if not ok:
            p = tmp_path / "m16.blob"
            p.write_bytes(R.to_bytes(b))
            with pytest.raises(E.BnnError) as e:
                E.ReactEngine(str(p))
            assert e.value.code == E.BNN_EBLOB and "+-1" in str(e.value)
            continue
        eng, _ = _engine(tmp_path, b)
        x = synth.make_input(32, 2, 120, 32, 32)
        _check_stages(eng, rorc.parse(R.to_bytes(b)), x)
        eng.close()


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_react_vs_golden(tmp_path, golden):
    """Logits and every materialised stage against the reference's own v3
    kernels chained as its engine chains them (tests/golden)."""
    meta, arrays = golden
    for name, c in meta["react_cases"].items():
        b = synth.make_blob_react(seed=c["blob_seed"], base=c["base"], coverage=c["coverage"])
        eng, _ = _engine(tmp_path, b, name + ".blob")
        x = synth.make_input(c["input_seed"], c["N"], 120, c["H"], c["W"])
        logits, st = eng.forward_debug(x)
        assert _same(logits, arrays[f"{name}__logits"]), name
        assert _same(eng.forward_batch(x), arrays[f"{name}__logits"]), name
        for n in range(c["N"]):
            want = c["stages"][n]
            assert set(st) == _gpu_names(want), name
            for k, v in st.items():
                assert _sha(v[n]) == want[k], (name, n, k)
        eng.close()


def test_react_batch_1024(tmp_path, rorc):
    """The benchmark shape: batch 1024 of 32x32x120 at base 16, sampled
    patches against the checker, and the same patch at other batch
    positions gives the same bits."""
    b = synth.make_blob_react(seed=10, base=16)
    eng, _ = _engine(tmp_path, b)
    model = rorc.parse(R.to_bytes(b))
    N = 1024
    x = synth.make_input(11, N, 120, 32, 32)
    x[777] = x[3]
    got = eng.forward_batch(x)
    idx = [0, 1, 3, 63, 64, 255, 500, 511, 512, 777, 1022, 1023]  # both halves of the two-stream split
    want = model.forward_batch(np.ascontiguousarray(x[idx]))
    for i, n in enumerate(idx):
        assert _same(got[n], want[i]), n
    assert _same(got[777], got[3])
    eng.close()


def test_react_patched(tmp_path, rorc):
    """Patch-wise scene forward (csrc/bnn_model_react.c:454-476), host and
    device pointers, against the checker's patch-wise forward."""
    import torch
    b = synth.make_blob_react(seed=12, base=8)
    eng, _ = _engine(tmp_path, b)
    model = rorc.parse(R.to_bytes(b))
    rng = np.random.default_rng(13)
    cube = rng.standard_normal((120, 70, 101)).astype(np.float32)
    for P in (16, 32):
        want = model.forward_patched(cube, P)
        assert _same(eng.forward_patched(cube, P), want), P
        d_cube = torch.from_numpy(cube).cuda()
        d_map = torch.full((3, 70, 101), float("nan"), device="cuda")
        eng.forward_patched_device(d_cube.data_ptr(), 70, 101, d_map.data_ptr(), P)
        torch.cuda.synchronize()
        assert _same(d_map.cpu().numpy(), want), P
    eng.close()


def test_react_past_launch_limit(tmp_path):
    """Inputs past the 2 GiB one launch addresses: a batch of 4400 patches
    (2.16 GB) runs as two launches from host and from device pointers, and a
    2080 x 2160 x 120 cube (2.16 GB) runs patch-wise in strips of whole patch
    rows, each staged as a sub-cube.  The batch equals batches of 1024 bit
    for bit, the maps the batch forward of the host-cut patches, stitched."""
    import torch
    from bnns_to_c_amd import scene
    b = synth.make_blob_react(seed=40, base=8)
    eng, _ = _engine(tmp_path, b)
    N = 4400
    x = synth.make_input(41, N)
    assert x.nbytes >= 2 ** 31
    small = np.concatenate([eng.forward_batch(x[i:i + 1024]) for i in range(0, N, 1024)])
    assert _same(eng.forward_batch(x), small)
    d_x = torch.from_numpy(x).cuda()
    del x
    d_o = torch.full((N, 3, 32, 32), float("nan"), device="cuda")
    eng.forward_device(d_x.data_ptr(), N, 32, 32, d_o.data_ptr())
    torch.cuda.synchronize()
    assert _same(d_o.cpu().numpy(), small)
    del d_x, d_o, small
    H, W, P = 2080, 2160, 32
    cube = np.random.default_rng(42).standard_normal((120, H, W), dtype=np.float32)
    assert cube.nbytes >= 2 ** 31
    want = scene.stitch(eng.forward_batch(scene.cut(cube, P)), H, W)
    assert _same(eng.forward_patched(cube, P), want)
    d_cube = torch.from_numpy(cube).cuda()
    del cube
    d_map = torch.full((3, H, W), float("nan"), device="cuda")
    eng.forward_patched_device(d_cube.data_ptr(), H, W, d_map.data_ptr(), P)
    torch.cuda.synchronize()
    assert _same(d_map.cpu().numpy(), want)
    eng.close()


def test_react_device_batch(tmp_path, rorc):
    import torch
    b = synth.make_blob_react(seed=14, base=16)
    eng, _ = _engine(tmp_path, b)
    x = synth.make_input(15, 5, 120, 32, 32)
    want = eng.forward_batch(x)
    d_x = torch.from_numpy(x).cuda()
    d_o = torch.empty((5, 3, 32, 32), device="cuda")
    eng.forward_device(d_x.data_ptr(), 5, 32, 32, d_o.data_ptr())
    torch.cuda.synchronize()
    assert _same(d_o.cpu().numpy(), want)
    assert _same(eng.forward(x[2]), want[2])
    eng.close()


def test_react_cli_vs_golden(tmp_path, golden):
    """bnn_infer_react's output file against the reference CLI's, byte for
    byte: the whole image from a file, patch-wise, and the "rand" cube."""
    meta, arrays = golden
    for name, c in meta["react_cli"].items():
        b = synth.make_blob_react(seed=c["blob_seed"], base=c["base"])
        p = tmp_path / (name + ".blob")
        p.write_bytes(R.to_bytes(b))
        if c["input_seed"] >= 0:
            xin = tmp_path / (name + ".in")
            synth.make_input(c["input_seed"], 1, 120, c["H"], c["W"])[0].tofile(xin)
            spec = str(xin)
        else:
            spec = "rand"
        if c["patch"]:
            spec = f"patch{c['patch']}:{spec}"
        out = tmp_path / (name + ".out")
        r = subprocess.run([E.CLI_REACT_PATH, str(p), spec, str(out), str(c["H"]), str(c["W"]), "2"],
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        assert "# forward" in r.stdout
        got = np.fromfile(out, np.float32).reshape(-1, c["H"], c["W"])
        assert _same(got, arrays[f"{name}__cli"]), name
        assert _sha(got) == c["sha256"]


def test_react_errors(tmp_path):
    b = synth.make_blob_react(seed=16, base=8)
    data = bytearray(R.to_bytes(b))
    p = tmp_path / "bad.blob"
    p.write_bytes(bytes(data[:-5]))
    with pytest.raises(E.BnnError) as e:
        E.ReactEngine(str(p))
    assert e.value.code == E.BNN_EBLOB
    eng, _ = _engine(tmp_path, b)
    with pytest.raises(E.BnnError) as e:
        eng.forward_batch(np.zeros((1, 120, 8, 32), np.float32))
    assert e.value.code == E.BNN_EARG
    with pytest.raises(E.BnnError):
        eng.forward_patched(np.zeros((120, 32, 32), np.float32), 24)
    # a v1 blob is refused with the version named
    from bnns_to_c_amd import blob as B1
    q = tmp_path / "v1.blob"
    q.write_bytes(B1.to_bytes(synth.make_blob(seed=1, base=8)))
    with pytest.raises(E.BnnError) as e:
        E.ReactEngine(str(q))
    assert "version 1" in str(e.value)
    eng.close()


# ------------------------------------------------------- kernel entry points --
def _abi(fn, *args):
    return getattr(E.lib(), fn)(*args)


def test_react_kernel_abi(rorc, orc):
    """The reference's v3 kernel entry points (csrc/bnn_model_react.h:18-53)
    on the GPU, batch 1, against the checker."""
    import ctypes as C
    L = E.lib()
    f32 = C.POINTER(C.c_float)
    i8 = C.POINTER(C.c_int8)
    i16 = C.POINTER(C.c_int16)
    i32 = C.POINTER(C.c_int32)
    u64 = C.POINTER(C.c_uint64)
    ci = C.c_int
    rng = np.random.default_rng(17)

    def p(a, t):
        return a.ctypes.data_as(t)

    for nm in ("react_proj_blk", "react_proj_1x1"):
        getattr(L, nm).argtypes = [f32, f32, f32, ci, ci, ci, ci]
    for cin, cout, H, W in [(120, 16, 32, 32), (48, 16, 17, 9), (384, 128, 2, 2), (20, 8, 3, 5), (7, 3, 4, 4)]:
        x = rng.standard_normal((cin, H, W)).astype(np.float32)
        Wm = rng.normal(0, 0.2, (cout, cin)).astype(np.float32)
        want = rorc.proj(x, Wm)
        for nm in ("react_proj_blk", "react_proj_1x1"):
            if nm == "react_proj_blk" and cout % 8:
                continue
            out = np.zeros((cout, H, W), np.float32)
            getattr(L, nm)(p(x, f32), p(Wm, f32), p(out, f32), cin, H, W, cout)
            assert _same(out, want), (nm, cin, cout)
    L.react_conv3_blk.argtypes = [f32, i8, f32, f32, ci, ci, ci, ci]
    for cin, cout, H, W in [(120, 16, 32, 32), (7, 8, 9, 17), (3, 16, 1, 1)]:
        x = rng.standard_normal((cin, H, W)).astype(np.float32)
        w = np.where(rng.random((cout, cin, 3, 3)) < 0.5, -1, 1).astype(np.int8)
        al = rng.uniform(0.01, 0.1, cout).astype(np.float32)
        out = np.zeros((cout, H, W), np.float32)
        L.react_conv3_blk(p(x, f32), p(w, i8), p(al, f32), p(out, f32), cin, H, W, cout)
        assert _same(out, rorc.conv3(x, w, al))
    C_, H, W = 12, 9, 11
    prm = [rng.uniform(0.01, 0.3, C_).astype(np.float32), rng.normal(0, 1, C_).astype(np.float32),
           rng.normal(0, 0.2, C_).astype(np.float32), rng.uniform(-0.5, 0.5, C_).astype(np.float32)]
    prm[3][:3] = 0.0
    res = rng.normal(0, 1, (C_, H, W)).astype(np.float32)
    P = rng.integers(-400, 400, (C_, H, W)).astype(np.int32)
    xr = rng.normal(0, 2, (C_, H, W)).astype(np.float32)
    pp = [p(v, f32) for v in prm]
    for nm, acc, t, form in [("react_epilogue_int", P, i32, 0), ("react_epilogue_real", xr, f32, 0),
                             ("react_epilogue_int_v2", P, i32, 1), ("react_epilogue_real_v2", xr, f32, 1),
                             ("react_epilogue_int_i16", P.astype(np.int16), i16, 1)]:
        getattr(L, nm).argtypes = [t, f32, f32, ci, ci, ci, f32, f32, f32, f32]
        out = np.zeros((C_, H, W), np.float32)
        getattr(L, nm)(p(acc, t), p(res, f32), p(out, f32), C_, H, W, *pp)
        want = rorc.epi_plain(acc, res, *prm) if form == 0 else rorc.epi(acc.astype(acc.dtype), res, *prm)
        assert _same(out, want), nm
    L.react_tap.argtypes = [f32, i8, ci, ci, ci, f32]
    rs = rng.normal(0, 0.5, C_).astype(np.float32)
    xr[0, 0, 0] = -rs[0]
    out8 = np.zeros((C_, H, W), np.int8)
    L.react_tap(p(xr, f32), p(out8, i8), C_, H, W, p(rs, f32))
    assert np.array_equal(out8, rorc.tap(xr, rs))
    for nm in ("maxpool_real", "maxpool_real_v2"):
        getattr(L, nm).argtypes = [f32, f32, ci, ci, ci, ci, ci]
        xz = np.where(rng.random((C_, H, W)) < 0.5, np.float32(0.0), np.float32(-0.0)).astype(np.float32)
        for t in (xr, xz):
            out = np.zeros((C_, H // 2, W // 2), np.float32)
            getattr(L, nm)(p(t, f32), p(out, f32), C_, H, W, 2, 2)
            assert _same(out, rorc.maxpool_real(t)), nm
    want = P[:, :H // 2 * 2, :W // 2 * 2].reshape(C_, H // 2, 2, W // 2, 2).max(axis=(2, 4))
    L.maxpool_P_v2.argtypes = [i32, i32, ci, ci, ci, ci, ci]
    out = np.zeros((C_, H // 2, W // 2), np.int32)
    L.maxpool_P_v2(p(P, i32), p(out, i32), C_, H, W, 2, 2)
    assert np.array_equal(out, want)
    L.maxpool_P_i16.argtypes = [i16, i16, ci, ci, ci, ci, ci]
    P16 = P.astype(np.int16)
    o16 = np.zeros((C_, H // 2, W // 2), np.int16)
    L.maxpool_P_i16(p(P16, i16), p(o16, i16), C_, H, W, 2, 2)
    assert np.array_equal(o16.astype(np.int32), want)
    L.head_1x1_v2.argtypes = [f32, f32, f32, f32, ci, ci, ci, ci]
    Wh = rng.normal(0, 0.3, (3, C_)).astype(np.float32)
    bh = rng.normal(0, 0.1, 3).astype(np.float32)
    out = np.zeros((3, H, W), np.float32)
    L.head_1x1_v2(p(xr, f32), p(Wh, f32), p(bh, f32), p(out, f32), C_, H, W, 3)
    assert _same(out, rorc.head(xr, Wh, bh))
    from bnns_to_c_amd import blob as B1
    L.bconv_blk_b4p4.argtypes = [i8, u64, i32] + [ci] * 8
    L.bconv_blk_b4p4_i16.argtypes = [i8, u64, i16] + [ci] * 8
    for cin, cout, H, W in [(16, 16, 32, 32), (48, 16, 7, 5), (130, 8, 3, 10)]:
        a = np.where(rng.random((cin, H, W)) < 0.5, -1, 1).astype(np.int8)
        w = np.where(rng.random((cout, cin, 3, 3)) < 0.5, -1, 1).astype(np.int8)
        pk = B1.pack_kidx(w)
        want = orc.bconv(a, pk, cout)
        o32 = np.zeros((cout, H, W), np.int32)
        L.bconv_blk_b4p4(p(a, i8), p(pk, u64), p(o32, i32), cin, H, W, cout, 3, 3, 1, 1)
        assert np.array_equal(o32, want)
        o16 = np.zeros((cout, H, W), np.int16)
        L.bconv_blk_b4p4_i16(p(a, i8), p(pk, u64), p(o16, i16), cin, H, W, cout, 3, 3, 1, 1)
        assert np.array_equal(o16.astype(np.int32), want)


def test_react_split_batch_and_scene(tmp_path, rorc):
    """Batches of 256+ patches and scenes of 256+ patches run as two parts on
    two streams (the scene at whole patch rows, the planes keeping the whole
    batch's stride): an odd batch equals its patches run in small batches,
    and a 289-patch scene equals the checker's patch-wise forward."""
    import torch
    b = synth.make_blob_react(seed=16, base=8)
    eng, _ = _engine(tmp_path, b)
    x = synth.make_input(17, 301, 120, 16, 16)
    small = np.concatenate([eng.forward_batch(x[i:i + 50]) for i in range(0, 301, 50)])
    assert _same(eng.forward_batch(x), small)
    model = rorc.parse(R.to_bytes(b))
    rng = np.random.default_rng(18)
    cube = rng.standard_normal((120, 272, 270)).astype(np.float32)
    want = model.forward_patched(cube, 16)
    d_cube = torch.from_numpy(cube).cuda()
    d_map = torch.full((3, 272, 270), float("nan"), device="cuda")
    s = torch.cuda.Stream()
    eng.forward_patched_device(d_cube.data_ptr(), 272, 270, d_map.data_ptr(), 16, s.cuda_stream)
    torch.cuda.synchronize()
    assert _same(d_map.cpu().numpy(), want)
    eng.close()


def test_react_default_stream_is_ordered(tmp_path):
    """stream = NULL is the HIP default stream, as for the v1 entry points:
    work the caller enqueues on the default stream after the call (here the
    copy to the host, which waits for that stream only) sees the finished
    logits, for a split batch and for a scene."""
    import torch
    b = synth.make_blob_react(seed=19, base=8)
    eng, _ = _engine(tmp_path, b)
    N = 512
    x = synth.make_input(20, N, 120, 16, 16)
    want = eng.forward_batch(x)
    with torch.cuda.stream(torch.cuda.default_stream()):
        dx = torch.from_numpy(x).cuda()
        dy = torch.full((N, 3, 16, 16), float("nan"), device="cuda")
        torch.cuda.synchronize()
        eng.forward_device(dx.data_ptr(), N, 16, 16, dy.data_ptr(), None)
        got = dy.cpu().numpy()
        assert _same(got, want)
        rng = np.random.default_rng(21)
        cube = rng.standard_normal((120, 272, 270)).astype(np.float32)
        want_map = eng.forward_patched(cube, 16)
        d_cube = torch.from_numpy(cube).cuda()
        d_map = torch.full((3, 272, 270), float("nan"), device="cuda")
        torch.cuda.synchronize()
        eng.forward_patched_device(d_cube.data_ptr(), 272, 270, d_map.data_ptr(), 16, None)
        assert _same(d_map.cpu().numpy(), want_map)
    eng.close()


@pytest.mark.parametrize("H,W,budget", [(640, 200, 48 << 20), (333, 277, 50 << 20), (400, 600, 70 << 20)])
def test_react_whole_image_tiles(tmp_path, rorc, monkeypatch, H, W, budget):
    """A v3 whole image in tiles (row strips, or square tiles; core edges on
    16 px, 128 px of halo), forced here by a small tile budget: the logits of
    the untiled run bit for bit, and the checker's."""
    b = synth.make_blob_react(seed=43, base=8)
    eng, _ = _engine(tmp_path, b)
    x = synth.make_input(44, 1, 120, H, W)
    monkeypatch.delenv("BNN_TILE_BYTES", raising=False)
    whole = eng.forward_batch(x)
    monkeypatch.setenv("BNN_TILE_BYTES", str(budget))
    tiled = eng.forward_batch(x)
    monkeypatch.delenv("BNN_TILE_BYTES", raising=False)
    assert _same(tiled, whole)
    assert _same(tiled[0], rorc.parse(R.to_bytes(b)).forward(x[0]))
    eng.close()


def test_react_whole_image_past_2gib(tmp_path, rorc, monkeypatch):
    """A single 120-band v3 image of 2304 x 2048 (2.26 GB, past the 2 GiB a
    launch addresses): bnn_forward_react (host), the device entry point and
    the reference's file reader path (bnn_infer_react on an input file,
    bnn_forward_react_file) all run it in tiles and equal the checker."""
    import torch

    monkeypatch.delenv("BNN_TILE_BYTES", raising=False)
    b = synth.make_blob_react(seed=45, base=8)
    eng, path = _engine(tmp_path, b)
    H, W = 2304, 2048
    x = np.random.default_rng(46).standard_normal((120, H, W), dtype=np.float32)
    assert x.nbytes > 2**31
    print("v3 whole image: host path", flush=True)
    got = eng.forward(x)
    print("device path", flush=True)
    dx = torch.from_numpy(x).cuda()
    dy = torch.empty((1, b.n_classes, H, W), dtype=torch.float32, device="cuda")
    eng.forward_device(dx.data_ptr(), 1, H, W, dy.data_ptr())
    torch.cuda.synchronize()
    assert _same(dy.cpu().numpy()[0], got)
    del dx, dy
    print("file path (CLI)", flush=True)
    xin, out = tmp_path / "big.in", tmp_path / "big.out"
    x.tofile(xin)
    r = subprocess.run([E.CLI_REACT_PATH, path, str(xin), str(out), str(H), str(W), "1"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    assert _same(np.fromfile(out, np.float32).reshape(-1, H, W), got)
    os.unlink(xin)
    print("checker", flush=True)
    assert _same(got, rorc.parse(R.to_bytes(b)).forward(x))
    eng.close()
