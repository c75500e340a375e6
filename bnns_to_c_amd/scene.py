"""Patch tiling of a scene cube, the convention of the reference's
csrc/bnn_model_react.c:454-476 (bnn_forward_react_patched): P x P patches
start at multiples of P, row-major; an edge patch is zero past the scene;
each patch's logits inside the scene are written back to the map.

These helpers cut and stitch on the host with numpy.  The engine's
bnn_forward_patched does the same on the GPU without materialising the
patches; tests use these to build the expected map from per-patch forwards.
"""
from __future__ import annotations

import numpy as np


def grid(H: int, W: int, P: int) -> tuple[int, int]:
    """(patch rows, patch columns) covering an H x W scene."""
    return (H + P - 1) // P, (W + P - 1) // P


def cut(cube: np.ndarray, P: int) -> np.ndarray:
    """[nb, H, W] -> [rows*cols, nb, P, P], zero past the scene."""
    nb, H, W = cube.shape
    pr, pc = grid(H, W, P)
    pad = np.zeros((nb, pr * P, pc * P), np.float32)
    pad[:, :H, :W] = cube
    return np.ascontiguousarray(pad.reshape(nb, pr, P, pc, P).transpose(1, 3, 0, 2, 4).reshape(pr * pc, nb, P, P))


def stitch(logits: np.ndarray, H: int, W: int) -> np.ndarray:
    """[rows*cols, ncls, P, P] -> [ncls, H, W] (the parts inside the scene)."""
    n, ncls, P, _ = logits.shape
    pr, pc = grid(H, W, P)
    assert n == pr * pc
    full = logits.reshape(pr, pc, ncls, P, P).transpose(2, 0, 3, 1, 4).reshape(ncls, pr * P, pc * P)
    return np.ascontiguousarray(full[:, :H, :W])
