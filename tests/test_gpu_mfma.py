"""The binary 3x3 conv on the int8 matrix cores (bnn_bconv_mfma.hip).

The kernel computes the same P as csrc/bnn_conv.c:23-36 (P = 2*D - S with
D the int8 product of 0/1 activation bytes and +-1 weights, S the weight sum
over the in-image taps), with the rule and the 2x2 max-pool of
csrc/bnn_fold.c:37-60 and csrc/bnn_maxpool.c:28-48 fused.  BNN_BCONV_MFMA=2
routes every conv it fits (cout % 64 == 0, W a power of two in 8..64, rows
that tile) through it; every stage of the forward must then equal the
checker's bit for bit, as on the popcount path.  The default rule (at least
four 64-channel input chunks) is checked to pick exactly the layers it
names, and the isolated layer entry point must agree with the popcount
kernel on the benchmark's fused config and smaller shapes.
"""
import numpy as np
import pytest

from bnns_to_c_amd import blob as B
from bnns_to_c_amd import engine as E
from bnns_to_c_amd import synth

pytestmark = pytest.mark.gpu


def _same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    if a.dtype == np.float32:
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return np.array_equal(a, b)


def _ops(eng, x):
    """label -> profiler op name of one forward."""
    E.prof_reset()
    E.prof_enable(True)
    try:
        eng.forward_batch(x)
    finally:
        E.prof_enable(False)
    return {lab: op for lab, op, _ms, _w in E.prof_records()}


def _check_stages(eng, model, x):
    logits, st = eng.forward_debug(x)
    for n in range(x.shape[0]):
        want, ref_st = model.forward(x[n], stages=True)
        for name, arr in st.items():
            if name == "logits":
                continue
            assert _same(arr[n], ref_st[name]), (name, n)
        assert _same(logits[n], want), n


# (seed, base, N, H, W): patches of several tiles (64x64, 96x64 and its
# 48x32 level), whole-patch tiles with a partial last tile (8x8 levels, N
# odd), an odd number of input words (base 24: 96 -> 192 channels at 8x8),
# rows wider than 64 in tiles of 32 columns (base 64 at 64x256: levels 256
# and 128 wide, with pools and concats, and a 4x16 bottleneck in tiles of
# four whole patches)
@pytest.mark.parametrize("seed,base,N,H,W", [
    (21, 32, 2, 64, 64),
    (22, 32, 3, 32, 32),
    (23, 16, 3, 32, 32),
    (24, 24, 1, 64, 64),
    (25, 32, 1, 96, 64),
    (26, 64, 1, 64, 256),
])
def test_forced_mfma_stages_vs_checker(tmp_path, orc, monkeypatch, seed, base, N, H, W):
    monkeypatch.setenv("BNN_BCONV_MFMA", "2")
    monkeypatch.setenv("BNN_MID", "0")  # the fused middle would take base 16's matrix-core layers
    b = synth.make_blob(seed=seed, base=base)
    p = tmp_path / "m.blob"
    p.write_bytes(B.to_bytes(b))
    eng = E.Engine(str(p))
    x = synth.make_input(seed + 100, N, 120, H, W)
    ops = _ops(eng, x)
    assert any(op.endswith("_mfma") for op in ops.values()), ops
    _check_stages(eng, orc.parse(B.to_bytes(b)), x)
    eng.close()


def test_default_rule_picks_wide_layers(tmp_path, orc, monkeypatch):
    """Default: the matrix cores for fold and pool layers with cout % 64 == 0,
    rows at least 16 wide and at least 64 input channels."""
    monkeypatch.delenv("BNN_BCONV_MFMA", raising=False)
    b = synth.make_blob(seed=26, base=32)
    p = tmp_path / "m.blob"
    p.write_bytes(B.to_bytes(b))
    eng = E.Engine(str(p))
    x = synth.make_input(126, 1, 120, 128, 128)
    ops = _ops(eng, x)
    # base 32 at 128x128: levels 1, 2, 3 are 64, 32 and 16 wide with 64,
    # 128 and 256 channels; level 0 (128 wide, 32 channels), enc2.c1 (32
    # input channels) and the 8 x 8 bottleneck stay on the popcount kernel
    want = {f"{lv}.c{k}" for lv in ("enc2", "enc3", "enc4", "dec4", "dec3", "dec2") for k in (1, 2)} - {"enc2.c1"}
    got = {lab for lab, op in ops.items() if op.endswith("_mfma")}
    assert got == want, (got, ops)
    _check_stages(eng, orc.parse(B.to_bytes(b)), x)
    eng.close()


@pytest.mark.parametrize("N,H,W,c", [(1024, 32, 32, 128), (5, 8, 8, 64), (3, 16, 16, 256), (2, 64, 64, 64),
                                     (2, 32, 128, 64), (1, 16, 256, 128)])
def test_layer_fold_pool_matches_popcount(monkeypatch, N, H, W, c):
    import torch
    a = synth.make_bits(40 + c, N, H, W, c)
    w = synth.make_signs(41, c, c)
    t1 = synth.make_thresholds(42, c, c * 9 // 4)
    t2 = synth.make_thresholds(43, c, c * 9 // 4)
    da = torch.from_numpy(a).cuda()
    act = torch.empty((N, H, W, c // 32), dtype=torch.int32, device="cuda")
    E.pack_act_device(da.data_ptr(), act.data_ptr(), N, c, H, W, None)
    torch.cuda.synchronize()
    outs = {}
    for mode in ("0", "2"):
        monkeypatch.setenv("BNN_BCONV_MFMA", mode)
        L = E.ConvLayer(B.pack_kidx(w), c, c, t1, t2)
        skip = torch.full((N, H, W, c // 32), -1, dtype=torch.int32, device="cuda")
        down = torch.full((N, H // 2, W // 2, c // 32), -1, dtype=torch.int32, device="cuda")
        L.fold_pool_device(act.data_ptr(), N, H, W, skip.data_ptr(), down.data_ptr(), None)
        torch.cuda.synchronize()
        outs[mode] = (skip.cpu().numpy(), down.cpu().numpy())
        L.close()
    assert np.array_equal(outs["0"][0], outs["2"][0])
    assert np.array_equal(outs["0"][1], outs["2"][1])
