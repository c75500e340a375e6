"""The drop-in claim, run: the reference's own CLI mains (csrc/main.c,
csrc/main_stem.c, csrc/main_react.c), compiled unchanged against include/
and linked to libbnn_hip.so by `make -C oracle dropin`, write the same output
bytes as the reference CLIs did on the golden cases (tests/golden), with the
forward on the GPU.

The binaries are built where the reference sources are (the build step);
they travel with the tree, and the tests skip where they were never built."""
import os
import subprocess

import numpy as np
import pytest

from bnns_to_c_amd import blob as B
from bnns_to_c_amd import blob_react as R
from bnns_to_c_amd import synth

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DROPIN = os.path.join(ROOT, "oracle", "_ref", "dropin")


def _bin(name):
    p = os.path.join(DROPIN, name)
    if not os.path.exists(p):
        pytest.skip(f"{p} not built (make -C oracle dropin needs the reference sources)")
    return p


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _linked_to_engine(exe):
    out = subprocess.run(["ldd", exe], capture_output=True, text=True).stdout
    return "libbnn_hip.so" in out and os.path.join("bnns_to_c_amd", "lib") in out


def test_reference_main_on_engine(tmp_path, golden):
    exe = _bin("bnn_infer")
    assert _linked_to_engine(exe)
    meta, arrays = golden
    for name, c in meta["cli"].items():
        p = tmp_path / (name + ".blob")
        p.write_bytes(B.to_bytes(synth.make_blob(seed=c["blob_seed"], base=c["base"], coverage=c["coverage"])))
        out = tmp_path / (name + ".bin")
        r = subprocess.run([exe, str(p), "rand", str(out), str(c["H"]), str(c["W"]), "3"],
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        assert f"# H={c['H']} W={c['W']} bands=120 classes=3 reps=3" in r.stderr
        got = np.fromfile(out, np.float32).reshape(-1, c["H"], c["W"])
        assert np.array_equal(_bits(got), _bits(arrays[f"{name}__cli"])), name
    # a bad blob: the library's exit(1) with a message, as the reference's
    r = subprocess.run([exe, str(tmp_path / "missing.blob"), "rand", str(tmp_path / "o.bin")],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "cannot open" in r.stderr


def test_reference_stem_main_on_engine(tmp_path, golden):
    exe = _bin("bnn_infer_stem")
    meta, arrays = golden
    for name, c in meta["stem_cli"].items():
        b = synth.make_blob_v2(seed=c["blob_seed"], base=c["base"], stem=c["stem"], coverage=c["coverage"])
        p = tmp_path / (name + ".blob")
        p.write_bytes(B.to_bytes(b))
        out = tmp_path / (name + ".bin")
        r = subprocess.run([exe, str(p), "rand", str(out), str(c["H"]), str(c["W"]), "3"],
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        got = np.fromfile(out, np.float32).reshape(-1, c["H"], c["W"])
        assert np.array_equal(_bits(got), _bits(arrays[f"{name}__cli"])), name


@pytest.mark.parametrize("stream_rows", [None, "5"])
def test_reference_react_main_on_engine(tmp_path, golden, stream_rows):
    """main_react.c streams a file input through bnn_forward_react_file /
    bnn_forward_react_patched_file, so this also runs the engine's streamed
    file path, twice per case (reps = 2 re-read the file); BNN_STREAM_ROWS=5
    cuts every band into strips of 5 rows and a short last one."""
    exe = _bin("bnn_infer_react")
    env = dict(os.environ)
    if stream_rows:
        env["BNN_STREAM_ROWS"] = stream_rows
    meta, arrays = golden
    for name, c in meta["react_cli"].items():
        p = tmp_path / (name + ".blob")
        p.write_bytes(R.to_bytes(synth.make_blob_react(seed=c["blob_seed"], base=c["base"])))
        if c["input_seed"] >= 0:
            xin = tmp_path / (name + ".in")
            synth.make_input(c["input_seed"], 1, 120, c["H"], c["W"])[0].tofile(xin)
            specs = [str(xin), "mem:" + str(xin)]
        else:
            specs = ["rand"]
        for spec in specs:
            if c["patch"]:
                spec = f"patch{c['patch']}:{spec}"
            out = tmp_path / (name + ".out")
            r = subprocess.run([exe, str(p), spec, str(out), str(c["H"]), str(c["W"]), "2"],
                               capture_output=True, text=True, timeout=120, env=env)
            assert r.returncode == 0, r.stderr
            assert "# forward" in r.stdout
            got = np.fromfile(out, np.float32).reshape(-1, c["H"], c["W"])
            assert np.array_equal(_bits(got), _bits(arrays[f"{name}__cli"])), (name, spec)
