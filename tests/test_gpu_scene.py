"""Scene inference by independent P x P patches (bnn_forward_patched, the
tiling of csrc/bnn_model_react.c:454-476 on the v1 forward): the GPU reads
the patches straight out of the cube and writes the logit map; the expected
map is the checker's per-patch forward of the host-cut patches, stitched."""
import numpy as np
import pytest

from bnns_to_c_amd import blob as B
from bnns_to_c_amd import engine as E
from bnns_to_c_amd import scene, synth

pytestmark = pytest.mark.gpu


def _same(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _engine(tmp_path, b):
    p = tmp_path / "m.blob"
    p.write_bytes(B.to_bytes(b))
    return E.Engine(str(p))


def _cube(seed, H, W, nb=120):
    """x ~ N(0,1) plus a per-band offset ~ U(-0.5, 0.5) (benchmark config 3)"""
    rng = np.random.default_rng(seed)
    off = rng.uniform(-0.5, 0.5, (nb, 1, 1)).astype(np.float32)
    return (rng.standard_normal((nb, H, W), dtype=np.float32) + off).astype(np.float32)


@pytest.mark.parametrize("seed,base,H,W,P", [(0, 16, 70, 100, 32), (4, 8, 40, 33, 16), (8, 16, 64, 64, 32),
                                             (9, 48, 50, 40, 32)])  # a 48-channel head writes the map
def test_scene_vs_checker(tmp_path, orc, seed, base, H, W, P):
    b = synth.make_blob(seed=seed, base=base)
    eng = _engine(tmp_path, b)
    cube = _cube(seed + 50, H, W)
    got = eng.forward_patched(cube, P)
    model = orc.parse(B.to_bytes(b))
    want = scene.stitch(model.forward_batch(scene.cut(cube, P)), H, W)
    assert _same(got, want)
    eng.close()


def test_scene_paths_agree(tmp_path):
    """host pipeline (4 strips of one patch row), device call and the batch
    forward of host-cut patches give the same bits"""
    import torch
    b = synth.make_blob(seed=2)
    eng = _engine(tmp_path, b)
    H, W, P = 100, 1100, 32   # one patch row of input is ~17 MB: one row per strip
    cube = _cube(3, H, W)
    host = eng.forward_patched(cube, P)
    batch = scene.stitch(eng.forward_batch(scene.cut(cube, P)), H, W)
    assert _same(host, batch)
    d_cube = torch.from_numpy(cube).cuda()
    d_map = torch.full((3, H, W), float("nan"), device="cuda")
    eng.forward_patched_device(d_cube.data_ptr(), H, W, d_map.data_ptr(), P,
                               torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert _same(d_map.cpu().numpy(), batch)
    # a second scene of another size reuses the model's buffers
    cube2 = _cube(4, 47, 61)
    assert _same(eng.forward_patched(cube2, P), scene.stitch(eng.forward_batch(scene.cut(cube2, P)), 47, 61))
    eng.close()


def test_scene_errors(tmp_path):
    eng = _engine(tmp_path, synth.make_blob(seed=0, base=8))
    with pytest.raises(E.BnnError, match="multiple of 16"):
        eng.forward_patched(np.zeros((120, 40, 40), np.float32), 24)
    eng.close()


def test_scene_split_at_patch_rows(tmp_path, orc):
    """a scene of 306 patches (18 patch rows, edge patches ragged) runs as two
    parts of whole patch rows on two streams: the map equals the checker's"""
    import torch
    b = synth.make_blob(seed=5)
    eng = _engine(tmp_path, b)
    H, W, P = 549, 520, 32
    cube = _cube(6, H, W)
    want = scene.stitch(orc.parse(B.to_bytes(b)).forward_batch(scene.cut(cube, P)), H, W)
    d_cube = torch.from_numpy(cube).cuda()
    d_map = torch.full((3, H, W), float("nan"), device="cuda")
    s = torch.cuda.Stream()
    eng.forward_patched_device(d_cube.data_ptr(), H, W, d_map.data_ptr(), P, s.cuda_stream)
    torch.cuda.synchronize()
    assert _same(d_map.cpu().numpy(), want)
    assert _same(eng.forward_patched(cube, P), want)
    eng.close()


def test_scene_cfg3_geometry(tmp_path, orc):
    """Benchmark config 3 at its exact geometry: a 956 x 684 x 120 cube
    (N(0,1) plus a per-band offset) cut into 30 x 22 = 660 patches of 32 x 32,
    the last patch row and column zero past the scene, run as two parts of
    whole patch rows.  Device and host-pointer maps against the checker's
    per-patch forward, stitched."""
    import torch
    b = synth.make_blob(seed=0, base=16)
    eng = _engine(tmp_path, b)
    H, W, P = 956, 684, 32
    assert scene.grid(H, W, P) == (30, 22)
    cube = _cube(40, H, W)
    want = scene.stitch(orc.parse(B.to_bytes(b)).forward_batch(scene.cut(cube, P)), H, W)
    d_cube = torch.from_numpy(cube).cuda()
    d_map = torch.full((3, H, W), float("nan"), device="cuda")
    s = torch.cuda.Stream()
    eng.forward_patched_device(d_cube.data_ptr(), H, W, d_map.data_ptr(), P, s.cuda_stream)
    torch.cuda.synchronize()
    assert _same(d_map.cpu().numpy(), want)
    assert _same(eng.forward_patched(cube, P), want)
    eng.close()


def test_scene_past_launch_limit(tmp_path):
    """A 2080 x 2160 x 120 cube, 2.16 GB: past what one launch addresses, so
    both the host-pointer and the device-pointer scene calls run it in strips
    of whole patch rows, each staged as its own sub-cube.  Their maps equal
    the batch forward of the host-cut patches, stitched."""
    import torch
    b = synth.make_blob(seed=15)
    eng = _engine(tmp_path, b)
    H, W, P = 2080, 2160, 32
    cube = _cube(16, H, W)
    assert cube.nbytes >= 2 ** 31
    want = scene.stitch(eng.forward_batch(scene.cut(cube, P)), H, W)
    assert _same(eng.forward_patched(cube, P), want)
    d_cube = torch.from_numpy(cube).cuda()
    del cube
    d_map = torch.full((3, H, W), float("nan"), device="cuda")
    eng.forward_patched_device(d_cube.data_ptr(), H, W, d_map.data_ptr(), P,
                               torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert _same(d_map.cpu().numpy(), want)
    eng.close()
