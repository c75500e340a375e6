"""Patch tiling helpers (bnns_to_c_amd/scene.py), the convention of
csrc/bnn_model_react.c:454-476: closed forms on small cubes."""
import numpy as np

from bnns_to_c_amd import scene


def test_grid():
    assert scene.grid(956, 684, 32) == (30, 22)   # 660 patches, edge patches zero-filled
    assert scene.grid(64, 64, 32) == (2, 2)
    assert scene.grid(1, 1, 16) == (1, 1)


def test_cut_places_every_value_once():
    rng = np.random.default_rng(0)
    c = rng.standard_normal((3, 70, 100)).astype(np.float32)
    p = scene.cut(c, 32)
    assert p.shape == (12, 3, 32, 32)
    for n in range(12):
        r, q = divmod(n, 4)
        h, w = min(32, 70 - 32 * r), min(32, 100 - 32 * q)
        assert np.array_equal(p[n, :, :h, :w], c[:, 32 * r:32 * r + h, 32 * q:32 * q + w])
        assert not p[n, :, h:, :].any() and not p[n, :, :, w:].any()
    # every scene value appears exactly once; the rest is zero padding
    assert np.isclose(p.sum(dtype=np.float64), c.sum(dtype=np.float64))


def test_stitch_inverts_cut():
    rng = np.random.default_rng(1)
    c = rng.standard_normal((3, 45, 33)).astype(np.float32)
    for P in (16, 32, 48):
        assert np.array_equal(scene.stitch(scene.cut(c, P), 45, 33), c)
