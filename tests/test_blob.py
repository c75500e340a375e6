"""weights.blob v1 writer/reader and the engine's host-side blob checks.

Layout: python/bnn2c/blob.py:36-114,159-200; loader checks:
csrc/bnn_model.c:17-24, 43, 48, 70, 86, 93.  No GPU is touched here:
bnn_blob_check() parses and validates on the host only.
"""
import hashlib
import struct

import numpy as np
import pytest

from bnns_to_c_amd import blob as B
from bnns_to_c_amd import synth


def test_pack_kidx_matches_definition():
    # closed form: bit k of row co is set iff the C-order element k of wsign[co] > 0
    rng = np.random.default_rng(0)
    for cout, cin, k in [(4, 3, 3), (5, 7, 3), (2, 64, 3), (3, 65, 1), (1, 1, 1)]:
        w = np.where(rng.random((cout, cin, k, k)) < 0.5, -1, 1).astype(np.int8)
        p = B.pack_kidx(w)
        K = cin * k * k
        assert p.shape == (cout, (K + 63) // 64)
        for co in range(cout):
            flat = w[co].reshape(-1)
            for kk in range(K):
                assert ((int(p[co, kk >> 6]) >> (kk & 63)) & 1) == int(flat[kk] > 0)
            # bits past K stay zero
            if K % 64:
                assert int(p[co, -1]) >> (K % 64) == 0
        assert np.array_equal(B.unpack_kidx(p, cin, k, k), w)


def test_pack_kidx_matches_reference(ref):
    rng = np.random.default_rng(1)
    w = np.where(rng.random((7, 19, 3, 3)) < 0.5, -1, 1).astype(np.int8)
    assert np.array_equal(B.pack_kidx(w), ref.pack_weights(w))


def test_roundtrip_and_sizes():
    b = synth.make_blob(seed=0)
    data = B.to_bytes(b)
    assert data[:4] == b"BNNC"
    assert struct.unpack("<5i", data[4:24]) == (1, 16, 120, 3, 0)
    b2 = B.from_bytes(data)
    assert B.to_bytes(b2) == data
    convs = b2.enc_conv1 + b2.enc_conv2 + [b2.bott_conv1, b2.bott_conv2] + b2.dec_conv1 + b2.dec_conv2
    assert len(convs) == 18
    acts = (b2.enc_act1 + b2.enc_act2_skip + b2.enc_act2_down + [b2.bott_act1, b2.bott_act2]
            + b2.dec_act1 + b2.dec_act2)
    assert len(acts) == 22
    # widths of the dual-skip UNet at base 16 (csrc/bench_bconv.c:57-67)
    got = [(c.cin, c.cout) for c in
           [b2.enc_conv1[0], b2.enc_conv2[0], b2.enc_conv1[1], b2.enc_conv2[1], b2.enc_conv1[2],
            b2.enc_conv2[2], b2.enc_conv1[3], b2.enc_conv2[3], b2.bott_conv1, b2.bott_conv2,
            b2.dec_conv1[0], b2.dec_conv2[0], b2.dec_conv1[1], b2.dec_conv2[1],
            b2.dec_conv1[2], b2.dec_conv2[2], b2.dec_conv1[3], b2.dec_conv2[3]]]
    assert got == [(120, 16), (16, 16), (16, 32), (32, 32), (32, 64), (64, 64), (64, 128), (128, 128),
                   (128, 256), (256, 256), (384, 128), (128, 128), (192, 64), (64, 64), (96, 32),
                   (32, 32), (48, 16), (16, 16)]


def test_generator_is_pinned(golden):
    meta, _ = golden
    for name, c in meta["cases"].items():
        b = synth.make_blob(seed=c["blob_seed"], base=c["base"], coverage=c["coverage"])
        assert hashlib.sha256(B.to_bytes(b)).hexdigest() == c["blob_sha256"], name
        x = synth.make_input(c["input_seed"], c["N"], 120, c["H"], c["W"])
        assert hashlib.sha256(x.tobytes()).hexdigest() == c["input_sha256"], name


def test_coverage_blob_has_every_rule():
    b = synth.make_blob(seed=3, coverage=True)
    types = np.concatenate([a.type for a in b.enc_act1[1:] + b.enc_act2_skip + b.enc_act2_down
                            + [b.bott_act1, b.bott_act2] + b.dec_act1 + b.dec_act2])
    assert set(np.unique(types)) == {0, 1, 2, 3, 4, 5}


# ----------------------------------------------------------- malformed blobs
def _corruptions():
    data = B.to_bytes(synth.make_blob(seed=0, base=8))
    out = [("bad magic", b"XNNC" + data[4:]),
           ("trailing bytes", data + b"\0"),
           ("short read", data[:-1]),
           ("short read", data[:30]),
           ("short read", data[:2]),
           ("unsupported blob version", data[:4] + struct.pack("<i", 3) + data[8:]),
           ("unsupported upsampler", data[:20] + struct.pack("<i", 1) + data[24:]),
           ("bad conv tag", data[:24] + struct.pack("<i", 9) + data[28:])]
    # first act record follows the real conv: 28 + 16*120*9 + 16*4 bytes after the header
    a0 = 24 + 28 + 8 * 120 * 9 + 8 * 4
    out.append(("bad act tag", data[:a0] + struct.pack("<i", 7) + data[a0 + 4:]))
    head = len(data) - (12 + 3 * 8 * 4 + 3 * 4)
    out.append(("bad head tag", data[:head] + struct.pack("<i", 5) + data[head + 4:]))
    return out


@pytest.mark.parametrize("msg,data", _corruptions())
def test_python_reader_rejects(msg, data):
    with pytest.raises(B.BlobError, match=msg):
        B.from_bytes(data)


@pytest.mark.parametrize("msg,data", _corruptions())
def test_engine_blob_check_rejects(msg, data, tmp_path):
    from bnns_to_c_amd import engine
    p = tmp_path / "bad.blob"
    p.write_bytes(data)
    with pytest.raises(engine.BnnError, match=msg):
        engine.blob_check(str(p))


@pytest.mark.parametrize("msg,data", _corruptions())
def test_oracle_rejects(msg, data, orc):
    with pytest.raises(ValueError, match=msg):
        orc.parse(data)


def test_engine_rejects_broken_chain(tmp_path):
    from bnns_to_c_amd import engine
    b = synth.make_blob(seed=0, base=8)
    # an act whose channel count does not match its conv
    a = b.dec_act1[2]
    b.dec_act1[2] = B.Act(0, a.c - 1, type=a.type[:-1], t=a.t[:-1], lo=a.lo[:-1], hi=a.hi[:-1])
    p = tmp_path / "chain.blob"
    p.write_bytes(B.to_bytes(b))
    with pytest.raises(engine.BnnError, match="does not chain"):
        engine.blob_check(str(p))
    b = synth.make_blob(seed=0, base=8)
    b.bott_conv2.pad = 0
    p.write_bytes(B.to_bytes(b))
    with pytest.raises(engine.BnnError, match="does not chain"):
        engine.blob_check(str(p))


def test_engine_accepts_valid(tmp_path):
    from bnns_to_c_amd import engine
    for base in (8, 16, 32):
        p = tmp_path / f"ok{base}.blob"
        p.write_bytes(B.to_bytes(synth.make_blob(seed=base, base=base)))
        engine.blob_check(str(p))


def test_v2_roundtrip_and_header():
    """v2 blobs: <7i> header (version 2, ..., has_stem 1, n_stem_layers 1),
    stem records right after it (python/bnn2c/blob.py:226-233)"""
    import struct
    b = synth.make_blob_v2(seed=3, base=8, stem=24)
    data = B.to_bytes(b)
    assert struct.unpack("<7i", data[4:32]) == (2, 8, 120, 3, 0, 1, 1)
    assert struct.unpack("<7i", data[32:60]) == (B.TAG_CONV_REAL, 24, 120, 1, 1, 0, 1)
    b2 = B.from_bytes(data)
    assert b2.has_stem and B.to_bytes(b2) == data
    assert b2.enc_conv1[0].tag == B.TAG_CONV_BIN and b2.enc_act1[0].kind == 0
    bad = bytearray(data)
    bad[24:28] = (0).to_bytes(4, "little")          # has_stem = 0
    with pytest.raises(B.BlobError, match="has_stem"):
        B.from_bytes(bytes(bad))


def test_engines_keep_their_versions(tmp_path):
    """each loader takes its own version only, with the reference's message
    for a v1 blob given to the v2 loader (csrc/bnn_model_stem.c:85-86)"""
    from bnns_to_c_amd import engine
    v1 = tmp_path / "v1.blob"
    v1.write_bytes(B.to_bytes(synth.make_blob(seed=0, base=8)))
    v2 = tmp_path / "v2.blob"
    v2.write_bytes(B.to_bytes(synth.make_blob_v2(seed=1, base=8)))
    engine.blob_check(str(v1))
    engine.stem_blob_check(str(v2))
    with pytest.raises(engine.BnnError, match="unsupported blob version 2.*bnn_stem_load"):
        engine.blob_check(str(v2))
    with pytest.raises(engine.BnnError, match="expected v2 blob, got v1"):
        engine.stem_blob_check(str(v1))


def _stem_corruptions():
    data = B.to_bytes(synth.make_blob_v2(seed=2, base=8, stem=16))
    out = [("n_stem_layers=1 supported", data[:28] + struct.pack("<i", 2) + data[32:]),
           ("n_stem_layers=1 supported", data[:24] + struct.pack("<i", 0) + data[28:]),
           ("short read", data[:40]),
           ("trailing bytes", data + b"\0"),
           ("bad conv tag", data[:32] + struct.pack("<i", 7) + data[36:])]
    # stem conv record: <7i> + 16*120 signs + 16 alphas; its act record follows
    a0 = 32 + 28 + 16 * 120 + 16 * 4
    out.append(("bad act tag", data[:a0] + struct.pack("<i", 1) + data[a0 + 4:]))
    # stem geometry the forward does not run: a 3x3 stem, pad 1
    b = synth.make_blob_v2(seed=2, base=8, stem=16)
    b.stem_conv = synth._real_conv(np.random.default_rng(1), 120, 16, k=3)
    out.append(("stem does not chain", B.to_bytes(b)))
    pad = bytearray(data)
    pad[52:56] = struct.pack("<i", 1)
    out.append(("stem does not chain", bytes(pad)))
    return out


@pytest.mark.parametrize("msg,data", _stem_corruptions(), ids=lambda v: v if isinstance(v, str) else "")
def test_engine_stem_blob_check_rejects(msg, data, tmp_path):
    from bnns_to_c_amd import engine
    p = tmp_path / "bad.blob"
    p.write_bytes(data)
    with pytest.raises(engine.BnnError, match=msg):
        engine.stem_blob_check(str(p))


def test_engine_stem_rejects_broken_chain(tmp_path):
    from bnns_to_c_amd import engine
    b = synth.make_blob_v2(seed=3, base=8, stem=24)
    b.enc_conv1[0] = synth._real_conv(np.random.default_rng(0), 24, 8)   # enc1.conv1 must be binary
    p = tmp_path / "chain.blob"
    p.write_bytes(B.to_bytes(b))
    with pytest.raises(engine.BnnError, match="enc1.conv1 does not chain"):
        engine.stem_blob_check(str(p))
    b = synth.make_blob_v2(seed=3, base=8, stem=24)
    b.stem_act = synth._int_act(np.random.default_rng(0), 24, 120, False)   # the stem fold is real
    p.write_bytes(B.to_bytes(b))
    with pytest.raises(engine.BnnError, match="stem does not chain"):
        engine.stem_blob_check(str(p))
