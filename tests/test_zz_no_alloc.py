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
