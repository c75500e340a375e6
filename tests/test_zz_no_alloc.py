"""The allocation-free forward, bnn_forward_device_noalloc (no counterpart in
the reference: for callers that cannot allocate device memory), against
bnn_forward_device on the same inputs, through the C ABI on the GPU.

Two calls in a row share the one scratch array: the second is smaller and
has another geometry, so it runs over what the first left behind.  Logits
must be bit-identical to the allocating entry point's (whose parity with the
reference is pinned by the forward tests).
"""
import numpy as np
import pytest

from bnns_to_c_amd import blob as B
from bnns_to_c_amd import engine as E
from bnns_to_c_amd import synth

pytestmark = pytest.mark.gpu


def test_noalloc_matches_device_forward(tmp_path):
    import torch

    b = synth.make_blob(seed=0, base=16)
    p = tmp_path / "m.blob"
    p.write_bytes(B.to_bytes(b))
    eng = E.Engine(str(p))
    s = torch.cuda.Stream()
    for N, H, W in ((96, 32, 32), (7, 30, 34)):
        print(f"noalloc case N={N} H={H} W={W}", flush=True)
        x = torch.from_numpy(synth.make_input(300 + N, N, 120, H, W)).cuda()
        want = torch.empty((N, b.n_classes, H, W), dtype=torch.float32, device="cuda")
        got = torch.full((N, b.n_classes, H, W), float("nan"), dtype=torch.float32, device="cuda")
        eng.forward_device(x.data_ptr(), N, H, W, want.data_ptr(), s.cuda_stream)
        eng.forward_device_noalloc(x.data_ptr(), N, H, W, got.data_ptr(), s.cuda_stream)
        s.synchronize()
        g, w = got.cpu().numpy(), want.cpu().numpy()
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), (N, H, W)
    # a call whose tensors exceed the scratch array is refused before any launch
    with pytest.raises(E.BnnError) as ei:
        eng.forward_device_noalloc(x.data_ptr(), 4000, 32, 32, got.data_ptr(), s.cuda_stream)
    assert ei.value.code == E.BNN_EARG and "scratch" in str(ei.value)
    eng.close()


def test_noalloc_past_launch_limit(tmp_path):
    """A call whose input passes the per-launch limit (2 GiB) runs as
    sub-batches over the same scratch, like bnn_forward_device: 425 bands at
    32x32 is 1.74 MB per patch, so 1,300 patches are two launches."""
    import torch

    b = synth.make_blob(seed=3, base=16, n_bands=425)
    p = tmp_path / "m.blob"
    p.write_bytes(B.to_bytes(b))
    eng = E.Engine(str(p))
    N, H, W = 1300, 32, 32
    print(f"noalloc case N={N} bands=425", flush=True)
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn((N, 425, H, W), device="cuda", generator=g)
    assert x.numel() * 4 > 2**31
    s = torch.cuda.Stream()
    want = torch.empty((N, b.n_classes, H, W), dtype=torch.float32, device="cuda")
    got = torch.full((N, b.n_classes, H, W), float("nan"), dtype=torch.float32, device="cuda")
    eng.forward_device(x.data_ptr(), N, H, W, want.data_ptr(), s.cuda_stream)
    eng.forward_device_noalloc(x.data_ptr(), N, H, W, got.data_ptr(), s.cuda_stream)
    s.synchronize()
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))
    del x
    eng.close()


def test_noalloc_graph_capture(tmp_path):
    """The allocation-free forward captured in a HIP graph (after one eager
    call, which does the per-device set-up) and replayed on new inputs, with
    eager work between the replays: every replay bit-identical to
    bnn_forward_device on the same input."""
    import torch

    b = synth.make_blob(seed=1, base=16)
    p = tmp_path / "m.blob"
    p.write_bytes(B.to_bytes(b))
    eng = E.Engine(str(p))
    N, H, W = 64, 32, 32
    gen = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn((N, 120, H, W), device="cuda", generator=gen)
    y = torch.empty((N, b.n_classes, H, W), dtype=torch.float32, device="cuda")
    want = torch.empty_like(y)
    s = torch.cuda.Stream()
    eng.forward_device_noalloc(x.data_ptr(), N, H, W, y.data_ptr(), s.cuda_stream)
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        eng.forward_device_noalloc(x.data_ptr(), N, H, W, y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    for r in range(4):
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
