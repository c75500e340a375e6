"""The engine on blobs written from trained parameters (bnns_to_c_amd.fold):
v1 and v2 models whose rules were derived from float chains run on the GPU
with every stage bit-exact against the checker."""
import numpy as np
import pytest

from bnns_to_c_amd import blob as B
from bnns_to_c_amd import engine as E
from bnns_to_c_amd import fold, synth

pytestmark = pytest.mark.gpu


def _same(a, b):
    if a.dtype == np.float32:
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return np.array_equal(a, b)


@pytest.mark.parametrize("stem,base", [(0, 8), (16, 8), (0, 16)])
def test_params_blob_on_gpu(tmp_path, orc, stem, base):
    b = fold.blob_from_params(synth.make_params(seed=11 + stem + base, base=base, stem=stem))
    p = tmp_path / "p.blob"
    p.write_bytes(B.to_bytes(b))
    eng = (E.StemEngine if stem else E.Engine)(str(p))
    model = orc.parse(p.read_bytes())
    x = synth.make_input(12, 2, 120, 32, 32)
    logits, st = eng.forward_debug(x)
    for n in range(2):
        want, ref = model.forward(x[n], stages=True)
        for name, arr in st.items():
            if name != "logits":
                assert _same(arr[n], ref[name]), (name, n)
        assert _same(logits[n], want), n
    eng.close()
