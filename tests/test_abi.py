"""libbnn_hip.so loads without a GPU and exports every entry point that
include/bnn_model.h, include/bnn_model_stem.h and include/bnn_prof.h
declare; host-only pieces of the engine are checked here against the
checker."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from bnns_to_c_amd import engine as E
from bnns_to_c_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_header_symbols():
    lib = E.lib()
    names = (set(E.header_symbols()) | set(E.header_symbols(E.HEADER_STEM))
             | set(E.header_symbols(E.HEADER_REACT))
             | set(E.header_symbols(os.path.join(ROOT, "include", "bnn_prof.h"))))
    assert {"bnn_load", "bnn_forward", "bnn_free", "bconv_dispatch", "head_1x1", "prof_report",
            "bnn_stem_load", "bnn_stem_forward", "bnn_stem_free", "bnn_load_react", "bnn_forward_react",
            "bnn_forward_react_patched", "bnn_free_react", "react_epilogue_int_i16", "react_proj_blk",
            "bconv_blk_b4p4_i16"} <= names
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", E.LIB_PATH], capture_output=True, text=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert names <= exported, sorted(names - exported)


def test_library_built_for_gfx950():
    # the offload bundle in .hip_fatbin names its code objects by target id
    data = open(E.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data
    assert b"amdgcn-amd-amdhsa--gfx942" not in data


def test_header_compiles_as_c(tmp_path):
    # both model headers together, as a caller of both engines includes them
    src = tmp_path / "t.c"
    src.write_text('#include "bnn_model.h"\n#include "bnn_model_stem.h"\n#include "bnn_model_react.h"\n'
                   '#include "bnn_prof.h"\n'
                   "int main(void){ Model *m = 0; StemModel *s = 0; ModelR *r = 0; (void)m; (void)s; (void)r;\n"
                   "  return sizeof(Conv) == sizeof(ConvS) && sizeof(Act) == sizeof(ActS) ? 0 : 1; }\n")
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    "-c", str(src), "-o", str(tmp_path / "t.o")], check=True)


REFERENCE_CSRC = "/root/reference/csrc"


@pytest.mark.parametrize("main", ["main.c", "main_stem.c", "main_react.c"])
def test_reference_mains_build_against_include(tmp_path, main):
    """The reference's CLI mains compile unchanged against include/ (fed on
    standard input, so their #include "bnn_model.h" finds include/ and not
    the reference's header beside them) and link against libbnn_hip.so:
    every symbol they call is exported with a matching declaration."""
    src = os.path.join(REFERENCE_CSRC, main)
    if not os.path.exists(src):
        pytest.skip("reference sources absent")
    exe = tmp_path / main.replace(".c", "")
    with open(src, "rb") as f:
        r = subprocess.run(["gcc", "-O2", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                            "-x", "c", "-", "-x", "none", "-o", str(exe), "-L", os.path.dirname(E.LIB_PATH),
                            "-lbnn_hip", "-lm"], stdin=f, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    # the headers it resolved are this repository's
    with open(src, "rb") as f:
        deps = subprocess.run(["gcc", "-M", "-I", os.path.join(ROOT, "include"), "-x", "c", "-"], stdin=f,
                              capture_output=True, text=True).stdout
    assert os.path.join(ROOT, "include", "bnn_prof.h") in deps and REFERENCE_CSRC not in deps


def test_cli_argument_errors():
    """The CLIs' argument checks run before any GPU call and keep the
    reference's exit codes and messages (csrc/main.c:23-26,
    csrc/main_react.c:44-50)."""
    r = subprocess.run([E.CLI_PATH, "a.blob", "rand"], capture_output=True, text=True)
    assert r.returncode == 1 and "input.bin|rand output.bin [H W [reps]]" in r.stderr
    assert "weights.blob" in r.stderr
    r = subprocess.run([E.CLI_STEM_PATH], capture_output=True, text=True)
    assert r.returncode == 1 and "weights_stem.blob" in r.stderr
    r = subprocess.run([E.CLI_REACT_PATH, "a.blob", "rand", "o.bin", "32"], capture_output=True, text=True)
    assert r.returncode == 2 and "blob input|rand output H W [reps]" in r.stderr
    for hw in (["0", "32"], ["32", "-4"], ["32", "32", "0"]):
        r = subprocess.run([E.CLI_REACT_PATH, "a.blob", "rand", "o.bin"] + hw, capture_output=True, text=True)
        assert r.returncode == 2 and "bad H/W/reps" in r.stderr, hw


def test_model_struct_prefix_matches_reference():
    # main.c reads m->n_bands / m->n_classes: the leading ints keep their order
    class Conv(ctypes.Structure):
        _fields_ = [("i", ctypes.c_int * 8), ("p", ctypes.c_void_p * 3)]

    assert ctypes.sizeof(Conv) == 56


def test_stem_model_layout_matches_reference(tmp_path):
    """StemModel keeps csrc/bnn_model_stem.h:44-59's field order (main_stem.c
    reads n_bands, n_classes and stem_conv.Cout), with the device pointer
    last; the offsets the Python binding reads are the C compiler's."""
    src = tmp_path / "o.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "bnn_model_stem.h"\n'
                   "int main(void){ printf(\"%zu %zu %zu %zu %zu\\n\", offsetof(StemModel, n_bands),"
                   " offsetof(StemModel, has_stem), offsetof(StemModel, stem_conv.Cout),"
                   " offsetof(StemModel, head_bias), offsetof(StemModel, dev)); return 0; }\n")
    exe = tmp_path / "o"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    off = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True).stdout.split()]
    assert off[:3] == [8, 20, 36]          # the Python binding reads ints 2, 5 and 9
    assert off[4] == off[3] + 8            # dev is the one field past the reference's


def test_fold_canon_matches_rules(orc):
    """bit = ((uint32)(P - lo) < wid) ^ inv reproduces every rule on every
    reachable P (|P| <= 9 * Cin), thresholds at the extremes included."""
    rng = np.random.default_rng(0)
    c = 400
    ty, t, lo, hi = synth.make_rules(1, c, 288, coverage=True)
    ty = ty.copy(); t = t.copy(); lo = lo.copy(); hi = hi.copy()
    ext = np.array([np.iinfo(np.int32).min, np.iinfo(np.int32).max, -(1 << 30) - 5, (1 << 30) + 5], np.int32)
    t[:40] = rng.choice(ext, 40)
    lo[40:80] = rng.choice(ext, 40)
    hi[60:100] = rng.choice(ext, 40)
    ty[100:110] = [-1, 6, 100, 0, 0, 1, 2, 3, 4, 5]
    P = np.arange(-3456, 3457, dtype=np.int64)
    clo, cwid, cinv = E.fold_canon(ty, t, lo, hi)
    bit = (((P[None, :] - clo[:, None].astype(np.int64)) & 0xFFFFFFFF) < cwid[:, None]) ^ (cinv[:, None] > 0)
    want = orc.fold_int(np.broadcast_to(P.astype(np.int32), (c, 1, P.size)).copy(), ty, t, lo, hi)[:, 0, :]
    assert np.array_equal(np.where(bit, 1, -1), want)


def test_bench_refuses_multi_gpu():
    r = subprocess.run(["python", os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0 and "one GPU" in (r.stderr + r.stdout)


def test_react_model_layout_matches_reference(tmp_path):
    """ModelR keeps csrc/bnn_model_react.h:82-88's field order (main_react.c
    reads n_bands and n_classes), with the device pointer last; the records
    keep the reference's sizes."""
    src = tmp_path / "r.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "bnn_model_react.h"\n'
                   "int main(void){ printf(\"%zu %zu %zu %zu %zu %zu\\n\", offsetof(ModelR, n_bands),"
                   " offsetof(ModelR, n_classes), sizeof(ConvR), sizeof(BlockR),"
                   " offsetof(ModelR, head_bias), offsetof(ModelR, dev)); return 0; }\n")
    exe = tmp_path / "r"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    off = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True).stdout.split()]
    assert off[:3] == [8, 12, 56]
    # is_down, input_real, 2 taps, 2 convs, proj, 3 epis (LP64)
    assert off[3] == 8 + 2 * 16 + 2 * 56 + 16 + 3 * 40
    assert off[5] == off[4] + 8


def test_react_blob_check_host_only(tmp_path):
    """the v3 blob check parses and validates without a GPU"""
    from bnns_to_c_amd import blob_react as R
    b = synth.make_blob_react(seed=1, base=8)
    p = tmp_path / "m.blob"
    R.write(b, str(p))
    E.react_blob_check(str(p))
    b.dec[3].conv2.pad = 0
    R.write(b, str(p))
    with pytest.raises(E.BnnError) as e:
        E.react_blob_check(str(p))
    assert "3x3" in str(e.value)
    p.write_bytes(R.to_bytes(synth.make_blob_react(seed=1, base=8))[:-4])
    with pytest.raises(E.BnnError) as e:
        E.react_blob_check(str(p))
    assert e.value.code == E.BNN_EBLOB
