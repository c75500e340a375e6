"""The whole v1 forward on the GPU (csrc/bnn_model.c:150-253).

Every stage (22 binary activations, 17 accumulators P, 4 pooled P, the real
first-conv output) is compared bit for bit with the checker and with the
stage hashes the reference's own kernels produced (tests/golden); logits
must be bit-identical (the head keeps the reference's summation order), so
the 1e-5 / argmax bar is met with margin.
"""
import hashlib
import os
import subprocess

import numpy as np
import pytest

from bnns_to_c_amd import blob as B
from bnns_to_c_amd import engine as E
from bnns_to_c_amd import synth

pytestmark = pytest.mark.gpu


def _engine(tmp_path, b, name="m.blob"):
    p = tmp_path / name
    p.write_bytes(B.to_bytes(b))
    return E.Engine(str(p)), str(p)


def _same(a, b):
    if a.dtype == np.float32:
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return np.array_equal(a, b)


@pytest.mark.parametrize("seed,base,cov,N,H,W", [
    (0, 16, False, 3, 32, 32),
    (3, 16, True, 3, 32, 32),
    (5, 8, False, 2, 17, 23),
    (6, 16, False, 2, 30, 34),
    (7, 8, True, 2, 16, 16),
    (9, 32, False, 2, 32, 32),
    (12, 16, False, 1, 47, 33),
    (13, 48, False, 2, 32, 32),   # head over 48 channels: dec1.conv2 then the separate head kernel
    (14, 64, True, 1, 30, 34),    # head over 64 channels, odd sizes
    (15, 8, True, 2, 33, 35),     # fused middle at base 8 (enc3 of 32 channels), level 2 of 8 x 8
    (16, 8, True, 2, 32, 33),     # fused middle with the level-1 layers at base 8 (paired taps)
])
def test_stages_vs_checker(tmp_path, orc, seed, base, cov, N, H, W):
    b = synth.make_blob(seed=seed, base=base, coverage=cov)
    eng, _ = _engine(tmp_path, b)
    model = orc.parse(B.to_bytes(b))
    x = synth.make_input(seed + 100, N, 120, H, W)
    logits, st = eng.forward_debug(x)
    assert len(st) == 49 - 4  # every stage except the four materialised up+concat inputs
    for n in range(N):
        want, ref_st = model.forward(x[n], stages=True)
        for name, arr in st.items():
            if name == "logits":
                continue
            assert _same(arr[n], ref_st[name]), (name, n)
        assert _same(logits[n], want), n
    eng.close()


def test_first_conv_general_signs(tmp_path, orc):
    """A first-conv weight outside {-1, +1} (0, +-2: the products stay
    exact) sends the engine to its vector-ALU real conv; the +-1 blob of the
    same seed runs on the matrix cores.  Both match the checker bit for bit."""
    b = synth.make_blob(seed=21)
    x = synth.make_input(22, 3, 120, 32, 32)
    rng = np.random.default_rng(23)
    w = b.enc_conv1[0].wsign.copy()
    flat = w.reshape(-1)
    idx = rng.choice(flat.size, 64, replace=False)
    flat[idx[:32]] = 0
    flat[idx[32:48]] = 2
    flat[idx[48:]] = -2
    for ws in (b.enc_conv1[0].wsign, w):
        b.enc_conv1[0].wsign = ws
        eng, _ = _engine(tmp_path, b)
        model = orc.parse(B.to_bytes(b))
        logits, st = eng.forward_debug(x)
        for n in range(3):
            want, ref_st = model.forward(x[n], stages=True)
            for name in ("enc1.conv1", "enc1.act1"):
                assert _same(st[name][n], ref_st[name]), (name, n)
            assert _same(logits[n], want), n
        eng.close()


@pytest.mark.parametrize("nb,H,W,N", [
    (13, 32, 32, 2),   # last chunk of 8 bands partly empty; 16-byte staging
    (37, 16, 36, 2),   # two tiles across, the second partly outside
    (120, 24, 64, 3),  # full chunks, two tiles across, a partial tile row
    (5, 20, 17, 2),    # width not a multiple of 4: the 4-byte staging kernel
    (120, 16, 16, 300),  # more tiles than the persistent grid, two batch parts
])
def test_first_conv_shapes(tmp_path, orc, nb, H, W, N):
    """The real first conv on both staging kernels (16-byte slots when the
    width is a multiple of 4, 4-byte rows otherwise), band counts that leave
    the last 8-channel chunk partly empty, tiles cut by the image edge and a
    batch larger than the persistent grid: enc1.conv1, enc1.act1 and the
    logits bit for bit against the checker."""
    b = synth.make_blob(seed=40 + nb, base=8, n_bands=nb)
    eng, _ = _engine(tmp_path, b)
    model = orc.parse(B.to_bytes(b))
    x = synth.make_input(41 + nb, N, nb, H, W)
    logits, st = eng.forward_debug(x)
    for n in sorted({0, N // 2, N - 1}):
        want, ref_st = model.forward(x[n], stages=True)
        for name in ("enc1.conv1", "enc1.act1"):
            assert _same(st[name][n], ref_st[name]), (name, n)
        assert _same(logits[n], want), n
    # the production path (no stage dumps, batch parts on two streams)
    assert _same(eng.forward_batch(x), logits)
    eng.close()


def test_golden_from_reference(tmp_path, golden):
    """stage hashes and logits recorded from the reference's own C"""
    meta, arrays = golden
    for name, c in meta["cases"].items():
        b = synth.make_blob(seed=c["blob_seed"], base=c["base"], coverage=c["coverage"])
        eng, _ = _engine(tmp_path, b, name + ".blob")
        x = synth.make_input(c["input_seed"], c["N"], 120, c["H"], c["W"])
        assert hashlib.sha256(x.tobytes()).hexdigest() == c["input_sha256"]
        logits, st = eng.forward_debug(x)
        assert _same(logits, arrays[f"{name}__logits"]), name
        assert _same(eng.forward_batch(x), arrays[f"{name}__logits"]), name
        for n in range(c["N"]):
            for k, v in st.items():
                h = hashlib.sha256(np.ascontiguousarray(v[n]).tobytes()).hexdigest()
                assert h == c["stages"][n][k], (name, n, k)
        eng.close()


def test_batch_1024(tmp_path, orc):
    b = synth.make_blob(seed=0)
    eng, _ = _engine(tmp_path, b)
    x = synth.make_input(1, 1024)
    got = eng.forward_batch(x)
    model = orc.parse(B.to_bytes(b))
    idx = np.r_[0:32, 500:532, 992:1024]
    want = model.forward_batch(np.ascontiguousarray(x[idx]))
    assert _same(got[idx], want)
    assert np.abs(got[idx] - want).max() <= 1e-5
    assert np.array_equal(got[idx].argmax(1), want.argmax(1))
    # patches are independent: a patch gives the same logits in any batch position
    assert _same(eng.forward_batch(x[idx[::-1]].copy())[::-1], got[idx])
    eng.close()


def test_batch_1024_every_patch(tmp_path, orc):
    """The headline batch (1024 patches of 32x32x120, the bench blob and
    input): every patch's enc1.act1 bits (the certified first conv) and its
    logits bit for bit against the checker, from the debug forward and from
    the plain forward (the headline path: two parts on two streams)."""
    from concurrent.futures import ThreadPoolExecutor

    b = synth.make_blob(seed=0)
    eng, _ = _engine(tmp_path, b)
    x = synth.make_input(1, 1024)
    logits, st = eng.forward_debug(x)
    plain = eng.forward_batch(x)
    assert _same(plain, logits)
    act1 = st["enc1.act1"]
    model = orc.parse(B.to_bytes(b))

    def patch_ok(n):
        want, ref = model.forward(x[n], stages=True)
        return np.array_equal(act1[n], ref["enc1.act1"]) and _same(logits[n], want)

    with ThreadPoolExecutor(8) as ex:
        bad = [n for n, ok in enumerate(ex.map(patch_ok, range(1024))) if not ok]
    assert not bad, bad[:8]
    eng.close()


def test_device_api_and_dropin(tmp_path):
    import torch
    b = synth.make_blob(seed=2)
    eng, _ = _engine(tmp_path, b)
    x = synth.make_input(2, 64)
    ref = eng.forward_batch(x)
    dx = torch.from_numpy(x).cuda()
    dy = torch.empty((64, 3, 32, 32), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream()
    eng.forward_device(dx.data_ptr(), 64, 32, 32, dy.data_ptr(), s.cuda_stream)
    s.synchronize()
    assert _same(dy.cpu().numpy(), ref)
    # the model's own stream, then the default stream (None)
    for st in (eng.stream(), None):
        dy.zero_()
        torch.cuda.synchronize()
        eng.forward_device(dx.data_ptr(), 64, 32, 32, dy.data_ptr(), st)
        torch.cuda.synchronize()
        assert _same(dy.cpu().numpy(), ref)
    assert _same(dy.cpu().numpy(), ref)
    # batch-1 drop-in entry point
    assert _same(eng.forward(x[5]), ref[5])
    # repeated calls are deterministic
    assert _same(eng.forward_batch(x), ref)
    eng.close()


def test_shape_errors(tmp_path):
    eng, _ = _engine(tmp_path, synth.make_blob(seed=0, base=8))
    with pytest.raises(E.BnnError, match="H, W >= 16"):
        eng.forward_batch(np.zeros((1, 120, 8, 32), np.float32))
    assert eng.forward_batch(np.zeros((0, 120, 32, 32), np.float32)).shape == (0, 3, 32, 32)
    eng.close()


def test_cli_matches_reference_cli(tmp_path, golden):
    """bnn_infer with the reference's argument order and `rand` input
    (csrc/main.c:22-76) writes the same bytes as the reference CLI."""
    meta, arrays = golden
    for name, c in meta["cli"].items():
        b = synth.make_blob(seed=c["blob_seed"], base=c["base"], coverage=c["coverage"])
        p = tmp_path / (name + ".blob")
        p.write_bytes(B.to_bytes(b))
        out = tmp_path / (name + ".bin")
        r = subprocess.run([E.CLI_PATH, str(p), "rand", str(out), str(c["H"]), str(c["W"]), "3"],
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        assert "# forward   :" in r.stderr and f"# H={c['H']} W={c['W']} bands=120 classes=3 reps=3" in r.stderr
        o = np.fromfile(out, np.float32).reshape(-1, c["H"], c["W"])
        assert _same(o, arrays[f"{name}__cli"]), name
    # input file path + profile table
    b = synth.make_blob(seed=0)
    p = tmp_path / "m.blob"
    p.write_bytes(B.to_bytes(b))
    x = synth.make_input(4, 1)[0]
    (tmp_path / "in.bin").write_bytes(x.tobytes())
    env = dict(os.environ, BNN_PROFILE="1")
    r = subprocess.run([E.CLI_PATH, str(p), str(tmp_path / "in.bin"), str(tmp_path / "o.bin")],
                       capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stderr
    assert "enc1.conv1" in r.stderr and "roll-up by op type" in r.stderr
    eng = E.Engine(str(p))
    assert _same(np.fromfile(tmp_path / "o.bin", np.float32).reshape(3, 32, 32), eng.forward(x))
    eng.close()
    # errors exit(1) with the message, like the reference
    r = subprocess.run([E.CLI_PATH, str(tmp_path / "missing.blob"), "rand", str(tmp_path / "o.bin")],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "cannot open" in r.stderr


@pytest.mark.parametrize("N", [256, 300, 513, 768, 769, 1031])
def test_batch_size_independent(tmp_path, N):
    """Any batch size, including ones that fill the last block partially,
    gives the same bits for every patch as batches of 64: halves in row
    parts (256, 300), one full round of the first conv and the rest in row
    quarters or halves (513, 768), halves in whole rows (769, 1031)."""
    import torch
    b = synth.make_blob(seed=11)
    eng, _ = _engine(tmp_path, b)
    x = synth.make_input(12, N)
    small = np.concatenate([eng.forward_batch(x[i:i + 64]) for i in range(0, N, 64)])
    big = eng.forward_batch(x)
    assert _same(big, small)
    dx = torch.from_numpy(x).cuda()
    dy = torch.full((N, 3, 32, 32), float("nan"), device="cuda")
    eng.forward_device(dx.data_ptr(), N, 32, 32, dy.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert _same(dy.cpu().numpy(), small)
    eng.close()


def test_cfg4_large_tile_vs_checker(tmp_path, orc, monkeypatch):
    """Benchmark config 4's shape (256x256x120, base 32, the default choice
    of conv kernels, matrix cores on the wide layers): every stage of one
    patch bitwise against the checker, and a batch of 3 whose patches match
    their single-patch runs."""
    monkeypatch.delenv("BNN_BCONV_MFMA", raising=False)
    b = synth.make_blob(seed=4, base=32)
    eng, _ = _engine(tmp_path, b)
    model = orc.parse(B.to_bytes(b))
    x = synth.make_input(104, 3, 120, 256, 256)
    logits, st = eng.forward_debug(x[:1])
    want, ref_st = model.forward(x[0], stages=True)
    for name, arr in st.items():
        if name != "logits":
            assert _same(arr[0], ref_st[name]), name
    assert _same(logits[0], want)
    batch = eng.forward_batch(x)
    assert _same(batch[0], want)
    for n in (1, 2):
        assert _same(batch[n], eng.forward_batch(x[n:n + 1])[0]), n
    eng.close()


def test_cfg4_full_batch(tmp_path, orc, monkeypatch):
    """Benchmark config 4 at its real batch: 64 patches of 256x256x120, base
    32 (the certified first conv in tiles of 32 columns with both 16-channel
    groups, the matrix-core binary convs).  Every patch of the batch equals
    its own single-patch run, and two patches equal the checker."""
    from concurrent.futures import ThreadPoolExecutor

    monkeypatch.delenv("BNN_BCONV_MFMA", raising=False)
    b = synth.make_blob(seed=0, base=32)
    eng, _ = _engine(tmp_path, b)
    x = synth.make_input(105, 64, 120, 256, 256)
    batch = eng.forward_batch(x)
    for n in range(64):
        assert _same(batch[n], eng.forward_batch(x[n:n + 1])[0]), n
    model = orc.parse(B.to_bytes(b))
    idx = (0, 63)
    with ThreadPoolExecutor(2) as ex:
        want = list(ex.map(lambda n: model.forward(x[n]), idx))
    for n, w in zip(idx, want):
        assert _same(batch[n], w), n
    eng.close()


def test_default_stream_is_ordered(tmp_path):
    """stream = NULL is the HIP default stream: the host copy the caller
    enqueues there next (it waits for that stream only) sees the finished
    logits of a split batch."""
    import torch
    eng, _ = _engine(tmp_path, synth.make_blob(seed=9))
    N = 512
    x = synth.make_input(10, N)
    want = eng.forward_batch(x)
    with torch.cuda.stream(torch.cuda.default_stream()):
        dx = torch.from_numpy(x).cuda()
        dy = torch.full((N, 3, 32, 32), float("nan"), device="cuda")
        torch.cuda.synchronize()
        eng.forward_device(dx.data_ptr(), N, 32, 32, dy.data_ptr(), None)
        assert _same(dy.cpu().numpy(), want)
    eng.close()


def test_split_forward_graph_capture(tmp_path):
    """bnn_forward_device of a split batch (600 patches: a full round of the
    certified conv, then 88 patches in row quarters, the first part's binary
    layers on the model's side stream) captured in a HIP graph after one
    eager call, replayed on new inputs with eager work between the replays:
    every replay bit-identical to the eager forward of the same input."""
    import torch
    eng, _ = _engine(tmp_path, synth.make_blob(seed=12))
    N, H, W = 600, 32, 32
    gen = torch.Generator(device="cuda").manual_seed(13)
    x = torch.randn((N, 120, H, W), device="cuda", generator=gen)
    y = torch.empty((N, 3, H, W), dtype=torch.float32, device="cuda")
    want = torch.empty_like(y)
    s = torch.cuda.Stream()
    eng.forward_device(x.data_ptr(), N, H, W, y.data_ptr(), s.cuda_stream)
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        eng.forward_device(x.data_ptr(), N, H, W, y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    for r in range(3):
        print(f"graph replay {r}", flush=True)
        x.copy_(torch.randn((N, 120, H, W), device="cuda", generator=gen))
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eng.forward_device(x.data_ptr(), N, H, W, want.data_ptr(), s.cuda_stream)
        s.synchronize()
        assert torch.equal(y.view(torch.int32), want.view(torch.int32)), r
    del graph
    eng.close()


def test_batch_past_launch_limit(tmp_path):
    """4400 patches, 2.16 GB of input: more than the 2 GiB one launch
    addresses, so the batch runs as two launches (4369 + 31 patches), from
    host pointers (bnn_forward_batch, staged one launch at a time) and from
    device pointers (bnn_forward_device); both equal batches of 1024 bit
    for bit."""
    import torch
    b = synth.make_blob(seed=13)
    eng, _ = _engine(tmp_path, b)
    N = 4400
    x = synth.make_input(14, N)
    assert x.nbytes >= 2 ** 31
    small = np.concatenate([eng.forward_batch(x[i:i + 1024]) for i in range(0, N, 1024)])
    assert _same(eng.forward_batch(x), small)
    d_x = torch.from_numpy(x).cuda()
    del x
    d_o = torch.full((N, b.n_classes, 32, 32), float("nan"), device="cuda")
    eng.forward_device(d_x.data_ptr(), N, 32, 32, d_o.data_ptr())
    torch.cuda.synchronize()
    assert _same(d_o.cpu().numpy(), small)
    eng.close()


def _ops(eng, x):
    E.prof_reset()
    E.prof_enable(True)
    try:
        eng.forward_batch(x)
    finally:
        E.prof_enable(False)
    return {lab: op for lab, op, _ms, _w in E.prof_records()}


_MID_LABEL = {"ext": "enc2-dec2", "mid": "enc3-dec3"}


@pytest.mark.parametrize("base,H,W,N,mode", [(16, 32, 32, 256, "ext"), (8, 32, 32, 256, "ext"),
                                             (16, 32, 32, 37, "mid"), (8, 35, 32, 256, "mid"),
                                             (8, 32, 33, 256, "ext"), (16, 28, 32, 37, "none"),
                                             (32, 32, 32, 37, "none")])
def test_fused_middle_rule_and_logits(tmp_path, monkeypatch, base, H, W, N, mode):
    """enc3.c1 .. dec3.c2 run as one kernel when level 2 is 8 x 8 and the
    widths fit (base <= 16); with enc2.c1, enc2.c2, dec2.c1 and dec2.c2
    around them when level 1 is 16 x 16 and a part of the batch has at
    least 256 patches.  BNN_MIDX=0 keeps the level-1 layers as per-layer
    kernels and BNN_MID=0 every layer, with the same logits bit for bit."""
    b = synth.make_blob(seed=40 + base, base=base)
    x = synth.make_input(41, N, 120, H, W)
    monkeypatch.delenv("BNN_MID", raising=False)
    monkeypatch.delenv("BNN_MIDX", raising=False)
    eng, _ = _engine(tmp_path, b)
    ops = _ops(eng, x)
    for m, lab in _MID_LABEL.items():
        assert (lab in ops) == (m == mode), ops
    assert ("enc2.c1" in ops) == (mode != "ext"), ops
    assert ("bott.c1" in ops) == (mode == "none"), ops
    got = eng.forward_batch(x)
    eng.close()
    monkeypatch.setenv("BNN_MIDX", "0")
    eng, _ = _engine(tmp_path, b, "x0.blob")
    ops = _ops(eng, x)
    assert "enc2-dec2" not in ops, ops
    assert ("enc3-dec3" in ops) == (mode != "none"), ops
    want_x = eng.forward_batch(x)
    eng.close()
    monkeypatch.delenv("BNN_MIDX", raising=False)
    monkeypatch.setenv("BNN_MID", "0")
    eng, _ = _engine(tmp_path, b, "m0.blob")
    ops = _ops(eng, x)
    assert not any(lab in ops for lab in _MID_LABEL.values()), ops
    want = eng.forward_batch(x)
    eng.close()
    assert _same(got, want)
    assert _same(want_x, want)


def _tile_budget(monkeypatch, nbytes):
    if nbytes is None:
        monkeypatch.delenv("BNN_TILE_BYTES", raising=False)
    else:
        monkeypatch.setenv("BNN_TILE_BYTES", str(nbytes))


@pytest.mark.parametrize("H,W,budget", [(640, 200, 48 << 20), (400, 600, 70 << 20), (333, 277, 50 << 20)])
def test_whole_image_tiles(tmp_path, orc, monkeypatch, H, W, budget):
    """A whole image run in tiles (full-width strips, or square tiles when a
    strip of 272 rows passes the budget; core edges on multiples of 16 px,
    128 px of halo) gives the logits of the untiled run bit for bit, and the
    checker's; the budget is lowered here so that small images tile."""
    b = synth.make_blob(seed=6)
    eng, _ = _engine(tmp_path, b)
    x = synth.make_input(107, 1, 120, H, W)
    _tile_budget(monkeypatch, None)
    whole = eng.forward_batch(x)
    _tile_budget(monkeypatch, budget)
    tiled = eng.forward_batch(x)
    _tile_budget(monkeypatch, None)
    assert _same(tiled, whole)
    want = orc.parse(B.to_bytes(b)).forward(x[0])
    assert _same(tiled[0], want)
    eng.close()


def test_whole_image_past_2gib(tmp_path, orc, monkeypatch):
    """A single 120-band image of 2304 x 2048 (2.26 GB of input, past the
    2 GiB a launch addresses) through bnn_forward's host path and through
    the device path: tiled, and equal to the checker's whole-image forward."""
    import torch

    _tile_budget(monkeypatch, None)
    b = synth.make_blob(seed=8)
    eng, _ = _engine(tmp_path, b)
    H, W = 2304, 2048
    x = np.random.default_rng(109).standard_normal((1, 120, H, W), dtype=np.float32)
    assert x.nbytes > 2**31
    print("whole image 2304x2048x120: host path", flush=True)
    got = eng.forward(x[0])
    print("device path", flush=True)
    dx = torch.from_numpy(x).cuda()
    dy = torch.empty((1, b.n_classes, H, W), dtype=torch.float32, device="cuda")
    eng.forward_device(dx.data_ptr(), 1, H, W, dy.data_ptr(), None)
    torch.cuda.synchronize()
    assert _same(dy.cpu().numpy()[0], got)
    del dx, dy
    print("checker", flush=True)
    want = orc.parse(B.to_bytes(b)).forward(x[0])
    assert _same(got, want)
    eng.close()
