"""weights.blob v3: the ReActNet (real-highway) blob, writer and reader.

The layout is the reference's contract and is kept byte-for-byte:
  python/bnn2c/blob_react.py:8-41    (header, record order, record layouts)
  python/bnn2c/blob_react.py:17-18   (TAG_PROJ 5, TAG_EPI 6, TAG_TAP 7)
  python/bnn2c/blob_react.py:52-58   (block widths)
  csrc/bnn_model_react.c:44-135      (the C reader: tags, structural checks,
                                      no trailing bytes, upsampler 0 only)

Record order per encoder (down) block: [TAP tap1, absent for enc1], CONV
conv1 (real for enc1, else binary), PROJ proj1, EPI epi1 (real for enc1,
else int), TAP tap2, CONV conv2, EPI epi_skip, EPI epi_down.  Per plain
block (bottleneck, dec4..dec1): TAP tap1, CONV conv1, PROJ proj1, EPI epi1,
TAP tap2, CONV conv2, EPI epi2.  Then the HEAD record.

Besides the dataclass API (`BlobV3`, `to_bytes`, `from_bytes`), the module
offers the reference's own entry points with the same names and arguments
(`arch`, `pack_weights_np`, `write_blob_react_from_fold`, `read_blob_react`),
so a caller of python/bnn2c/blob_react.py can switch modules.
"""
from __future__ import annotations

import io
import struct
from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import numpy as np

from .blob import (MAGIC, TAG_CONV_BIN, TAG_CONV_REAL, TAG_HEAD, BlobError, Conv, Head,
                   pack_kidx, _Rd, _r_conv, _w_conv)

VERSION_REACT = 3
TAG_PROJ = 5
TAG_EPI = 6
TAG_TAP = 7
EPI_INT, EPI_REAL = 0, 1
UPSAMPLER = {"nearest": 0, "pixshuf": 1, "nnrefine": 2}
C0_DEFAULT = 16


def arch(c: int):
    """[(name, cin, cout, kind)] of the nine blocks, blob order
    (python/bnn2c/blob_react.py:52-58); kind "down" or "plain"."""
    return [("enc1", 120, c, "down"), ("enc2", c, 2 * c, "down"),
            ("enc3", 2 * c, 4 * c, "down"), ("enc4", 4 * c, 8 * c, "down"),
            ("bottleneck", 8 * c, 16 * c, "plain"),
            ("dec4", 24 * c, 8 * c, "plain"), ("dec3", 12 * c, 4 * c, "plain"),
            ("dec2", 6 * c, 2 * c, "plain"), ("dec1", 3 * c, c, "plain")]


def pack_weights_np(wsign: np.ndarray) -> Tuple[np.ndarray, int]:
    """(packed uint64 [Cout, nwords], nwords): the kidx sign-bit packing
    shared with v1 (python/bnn2c/blob_react.py:61-71)."""
    p = pack_kidx(wsign)
    return p, p.shape[1]


@dataclass
class Proj:
    """Real 1x1 shortcut projection, no bias (TAG_PROJ)."""
    cout: int
    cin: int
    W: np.ndarray                  # float32 [Cout, Cin]


@dataclass
class Epi:
    """BN affine + real add + RPReLU epilogue (TAG_EPI):
    t = A*acc + (B + move1) + res; out = t if t >= 0 else prelu_w * t."""
    kind: int                      # EPI_INT (acc = integer P) or EPI_REAL
    c: int
    A: np.ndarray
    B: np.ndarray
    move1: np.ndarray
    prelu_w: np.ndarray


@dataclass
class Tap:
    """Binarising tap: bit = (x + rsign > 0) (TAG_TAP)."""
    c: int
    rsign: np.ndarray


@dataclass
class Block:
    is_down: bool
    input_real: bool
    tap1: Optional[Tap]            # None for enc1 (input_real)
    conv1: Conv
    proj1: Proj
    epi1: Epi
    tap2: Tap
    conv2: Conv
    epi_a: Epi                     # down: skip epilogue; plain: epi2
    epi_b: Optional[Epi] = None    # down: pooled-down epilogue


@dataclass
class BlobV3:
    base_channels: int
    n_bands: int
    n_classes: int
    upsampler: int = 0
    version: int = VERSION_REACT
    enc: List[Block] = field(default_factory=list)     # enc1..enc4
    bott: Optional[Block] = None
    dec: List[Block] = field(default_factory=list)     # dec4..dec1
    head: Optional[Head] = None

    def blocks(self):
        """(name, block) in blob order."""
        names = ["enc1", "enc2", "enc3", "enc4", "bott", "dec4", "dec3", "dec2", "dec1"]
        return list(zip(names, self.enc + [self.bott] + self.dec))


# ----------------------------------------------------------------- writer --
def _f32(a, n: int, what: str) -> np.ndarray:
    a = np.ascontiguousarray(a, "<f4")
    if a.shape != (n,):
        raise BlobError(f"{what}: shape {a.shape} != ({n},)")
    return a


def _w_proj(f, p: Proj) -> None:
    W = np.ascontiguousarray(p.W, "<f4")
    if W.shape != (p.cout, p.cin):
        raise BlobError(f"proj shape {W.shape} != ({p.cout},{p.cin})")
    f.write(struct.pack("<3i", TAG_PROJ, p.cout, p.cin))
    f.write(W.tobytes())


def _w_epi(f, e: Epi) -> None:
    f.write(struct.pack("<3i", TAG_EPI, e.kind, e.c))
    for nm in ("A", "B", "move1", "prelu_w"):
        f.write(_f32(getattr(e, nm), e.c, f"epi.{nm}").tobytes())


def _w_tap(f, t: Tap) -> None:
    f.write(struct.pack("<2i", TAG_TAP, t.c))
    f.write(_f32(t.rsign, t.c, "tap.rsign").tobytes())


def to_bytes(b: BlobV3) -> bytes:
    """Serialise in the order of python/bnn2c/blob_react.py:117-143."""
    f = io.BytesIO()
    f.write(MAGIC)
    f.write(struct.pack("<5i", b.version, b.base_channels, b.n_bands, b.n_classes, b.upsampler))
    for _, k in b.blocks():
        if not k.input_real:
            _w_tap(f, k.tap1)
        _w_conv(f, k.conv1)
        _w_proj(f, k.proj1)
        _w_epi(f, k.epi1)
        _w_tap(f, k.tap2)
        _w_conv(f, k.conv2)
        _w_epi(f, k.epi_a)
        if k.is_down:
            _w_epi(f, k.epi_b)
    h = b.head
    f.write(struct.pack("<3i", TAG_HEAD, h.cout, h.cin))
    f.write(np.ascontiguousarray(h.W, "<f4").tobytes())
    f.write(np.ascontiguousarray(h.bias, "<f4").tobytes())
    return f.getvalue()


def write(b: BlobV3, path: str) -> str:
    with open(path, "wb") as fh:
        fh.write(to_bytes(b))
    return path


# ----------------------------------------------------------------- reader --
def _r_proj(r: _Rd) -> Proj:
    tag, cout, cin = r.ints(3)
    if tag != TAG_PROJ:
        raise BlobError(f"bad proj tag {tag}")
    if cout < 0 or cin < 0:
        raise BlobError("bad proj dims")
    return Proj(cout, cin, r.arr("<f4", cout * cin).reshape(cout, cin))


def _r_epi(r: _Rd) -> Epi:
    tag, kind, c = r.ints(3)
    if tag != TAG_EPI:
        raise BlobError(f"bad epi tag {tag}")
    if c < 0:
        raise BlobError("bad epi channel count")
    A, B, m, w = (r.arr("<f4", c) for _ in range(4))
    return Epi(kind, c, A, B, m, w)


def _r_tap(r: _Rd) -> Tap:
    tag, c = r.ints(2)
    if tag != TAG_TAP:
        raise BlobError(f"bad tap tag {tag}")
    if c < 0:
        raise BlobError("bad tap channel count")
    return Tap(c, r.arr("<f4", c))


def _check(ok: bool, what: str) -> None:
    if not ok:
        raise BlobError(f"blob layout mismatch: {what}")


def _r_block(r: _Rd, is_down: bool, input_real: bool) -> Block:
    """One block with the C loader's structural checks
    (csrc/bnn_model_react.c:86-106)."""
    tap1 = None if input_real else _r_tap(r)
    conv1 = _r_conv(r)
    proj1 = _r_proj(r)
    epi1 = _r_epi(r)
    tap2 = _r_tap(r)
    conv2 = _r_conv(r)
    epi_a = _r_epi(r)
    epi_b = _r_epi(r) if is_down else None
    _check(conv1.tag == (TAG_CONV_REAL if input_real else TAG_CONV_BIN), "conv1 tag")
    _check(conv2.tag == TAG_CONV_BIN, "conv2 tag")
    _check(proj1.cin == conv1.cin and proj1.cout == conv1.cout, "proj1 dims")
    _check(input_real or tap1.c == conv1.cin, "tap1 channels")
    _check(tap2.c == conv2.cin, "tap2 channels")
    _check(epi1.c == conv1.cout and epi1.kind == (EPI_REAL if input_real else EPI_INT), "epi1")
    _check(epi_a.c == conv2.cout and epi_a.kind == EPI_INT, "epi_a")
    _check(not is_down or (epi_b.c == conv2.cout and epi_b.kind == EPI_INT), "epi_b")
    return Block(is_down, input_real, tap1, conv1, proj1, epi1, tap2, conv2, epi_a, epi_b)


def from_bytes(data: bytes) -> BlobV3:
    """Parse a v3 blob with the checks of csrc/bnn_model_react.c:108-135."""
    r = _Rd(data)
    if bytes(r.take(4)) != MAGIC:
        raise BlobError("bad magic")
    version, base, nb, nc, ups = r.ints(5)
    if version != VERSION_REACT:
        raise BlobError(f"blob version {version}, this engine reads v3 (ReActNet)")
    if ups != 0:
        raise BlobError("only nearest upsampler supported")
    b = BlobV3(base, nb, nc, ups, version)
    for i in range(4):
        b.enc.append(_r_block(r, True, i == 0))
    b.bott = _r_block(r, False, False)
    for _ in range(4):
        b.dec.append(_r_block(r, False, False))
    tag, hco, hci = r.ints(3)
    if tag != TAG_HEAD:
        raise BlobError(f"bad head tag {tag}")
    W = r.arr("<f4", hco * hci).reshape(hco, hci)
    b.head = Head(hco, hci, W, r.arr("<f4", hco))
    if r.o != len(r.d):
        raise BlobError("trailing bytes in blob")
    return b


def read(path: str) -> BlobV3:
    with open(path, "rb") as fh:
        return from_bytes(fh.read())


# ------------------------------------------- the reference's entry points --
def _epi_of(kind: int, t) -> Epi:
    A, B, m, w = (np.asarray(v, np.float32) for v in t)
    return Epi(kind, len(A), A, B, m, w)


def _bin(wsign) -> Conv:
    w = np.asarray(wsign)
    return Conv(TAG_CONV_BIN, w.shape[0], w.shape[1], w.shape[2], w.shape[3], 1, 1, packed=pack_kidx(w))


def blob_from_fold(fold: dict, base_channels: int = C0_DEFAULT, n_bands: int = 120,
                   n_classes: int = 3, upsampler: str = "nearest") -> BlobV3:
    """BlobV3 from the folded-parameter dictionary the reference's
    extract_react_params produces (python/bnn2c/blob_react.py:168-198):
    per block "conv1_wsign", "conv1_alpha", "proj1_W", "epi1", "tap1_rsign",
    "conv2_wsign", "tap2_rsign", and "epi_skip"/"epi_down" (down blocks) or
    "epi2" (plain), each epi a tuple (A, B, move1, prelu_w); "outc_W",
    "outc_b" for the head."""
    b = BlobV3(base_channels, n_bands, n_classes, UPSAMPLER[upsampler])
    for name, _, _, kind in arch(base_channels):
        d = fold[name]
        real = bool(d["input_real"])
        if real:
            w = np.asarray(d["conv1_wsign"], np.int8)
            conv1 = Conv(TAG_CONV_REAL, w.shape[0], w.shape[1], w.shape[2], w.shape[3], 1, 1,
                         wsign=w, alpha=np.asarray(d["conv1_alpha"], np.float32))
        else:
            conv1 = _bin(d["conv1_wsign"])
        P = np.asarray(d["proj1_W"], np.float32)
        down = kind == "down"
        blk = Block(down, real,
                    None if real else Tap(len(d["tap1_rsign"]), np.asarray(d["tap1_rsign"], np.float32)),
                    conv1, Proj(P.shape[0], P.shape[1], P),
                    _epi_of(EPI_REAL if real else EPI_INT, d["epi1"]),
                    Tap(len(d["tap2_rsign"]), np.asarray(d["tap2_rsign"], np.float32)),
                    _bin(d["conv2_wsign"]),
                    _epi_of(EPI_INT, d["epi_skip"] if down else d["epi2"]),
                    _epi_of(EPI_INT, d["epi_down"]) if down else None)
        if name.startswith("enc"):
            b.enc.append(blk)
        elif name == "bottleneck":
            b.bott = blk
        else:
            b.dec.append(blk)
    W = np.asarray(fold["outc_W"], np.float32)
    b.head = Head(W.shape[0], W.shape[1], W, np.asarray(fold["outc_b"], np.float32))
    return b


def write_blob_react_from_fold(fold, path, base_channels=C0_DEFAULT, n_bands=120, n_classes=3,
                               upsampler="nearest"):
    """Same name, arguments and bytes as python/bnn2c/blob_react.py:117."""
    write(blob_from_fold(fold, base_channels, n_bands, n_classes, upsampler), path)
    return path


def read_blob_react(path) -> dict:
    """The dictionary python/bnn2c/blob_react.py:202-265 returns, from the
    checked parse above."""
    b = read(path)
    out = {"version": b.version, "base_channels": b.base_channels, "n_bands": b.n_bands,
           "n_classes": b.n_classes, "upsampler": b.upsampler, "blocks": {}}

    def conv(c: Conv):
        d = {"Cout": c.cout, "Cin": c.cin, "kh": c.kh, "kw": c.kw, "pad": c.pad, "stride": c.stride}
        if c.tag == TAG_CONV_BIN:
            d.update(tag="bin", packed=c.packed)
        else:
            d.update(tag="real", wsign=c.wsign, alpha=c.alpha)
        return d

    def epi(e: Epi):
        return {"kind": e.kind, "C": e.c, "A": e.A, "B": e.B, "move1": e.move1, "prelu_w": e.prelu_w}

    names = [n for n, _, _, _ in arch(b.base_channels)]
    for name, (_, k) in zip(names, b.blocks()):
        blk = {}
        if k.tap1 is not None:
            blk["tap1"] = {"C": k.tap1.c, "rsign": k.tap1.rsign}
        blk["conv1"] = conv(k.conv1)
        blk["proj1"] = {"Cout": k.proj1.cout, "Cin": k.proj1.cin, "W": k.proj1.W}
        blk["epi1"] = epi(k.epi1)
        blk["tap2"] = {"C": k.tap2.c, "rsign": k.tap2.rsign}
        blk["conv2"] = conv(k.conv2)
        if k.is_down:
            blk["epi_skip"] = epi(k.epi_a)
            blk["epi_down"] = epi(k.epi_b)
        else:
            blk["epi2"] = epi(k.epi_a)
        out["blocks"][name] = blk
    out["head"] = {"Cout": b.head.cout, "Cin": b.head.cin, "W": b.head.W, "bias": b.head.bias}
    return out
