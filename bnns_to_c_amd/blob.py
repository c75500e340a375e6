"""weights.blob v1: the byte layout the engine loads, with a writer and reader.

The layout is the reference's contract and is kept byte-for-byte:
  python/bnn2c/blob.py:36-44    (magic, version, record tags)
  python/bnn2c/blob.py:47-58    (kidx sign-bit packing of binary weights)
  python/bnn2c/blob.py:67-114   (CONV bin / CONV real / ACT / HEAD records)
  python/bnn2c/blob.py:159-200  (v1 record order)
  csrc/bnn_model.c:27-96        (the C reader, including the no-trailing-bytes rule)

Everything is little-endian; int32 header fields.  The writer here builds the
blob from numpy arrays (the reference builds it from a torch model, which is
outside this engine's scope); the reader mirrors the C loader's checks and
additionally rejects version != 1 and upsampler != 0, which the v1 engine
cannot run.
"""
from __future__ import annotations

import io
import struct
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

MAGIC = b"BNNC"
VERSION = 1
VERSION_STEM = 2            # spectral-stem blobs (python/bnn2c/blob.py:229-230)
UPSAMPLER_NEAREST = 0

TAG_CONV_BIN = 1
TAG_CONV_REAL = 2
TAG_ACT = 3
TAG_HEAD = 4

# int fold rule codes (csrc/bnn_fold.c:10-15, python/verify/forward_driver.py:85)
RULE_CONST, RULE_GE, RULE_LT, RULE_BAND_IN, RULE_BAND_OUT = 0, 1, 2, 3, 4

ENC = ("enc1", "enc2", "enc3", "enc4")
DEC = ("dec4", "dec3", "dec2", "dec1")


class BlobError(ValueError):
    """Raised for any malformed blob (the C loader exits(1) on the same cases)."""


def pack_kidx(wsign: np.ndarray) -> np.ndarray:
    """Sign bits of wsign[Cout,Cin,kh,kw] packed LSB-first into uint64 words in
    kidx order, kidx = (ci*kh + ky)*kw + kx, bit = 1 iff w > 0
    (csrc/bnn_conv.c:80-95, python/bnn2c/blob.py:47-58).  Vectorised: the
    C-order flatten of wsign[co] is exactly kidx order."""
    w = np.asarray(wsign)
    cout = w.shape[0]
    k = int(np.prod(w.shape[1:]))
    nwords = (k + 63) // 64
    bits = (w.reshape(cout, k) > 0).astype(np.uint8)
    padded = np.zeros((cout, nwords * 64), np.uint8)
    padded[:, :k] = bits
    # little-endian bit order inside each byte, bytes little-endian in the word
    by = np.packbits(padded.reshape(cout, nwords * 8, 8), axis=-1, bitorder="little")
    return by.reshape(cout, nwords * 8).view("<u8").reshape(cout, nwords).copy()


def unpack_kidx(packed: np.ndarray, cin: int, kh: int, kw: int) -> np.ndarray:
    """Inverse of pack_kidx: int8 wsign[Cout,Cin,kh,kw] in {-1,+1}."""
    p = np.ascontiguousarray(packed, dtype="<u8")
    cout, nwords = p.shape
    k = cin * kh * kw
    bits = np.unpackbits(p.view(np.uint8).reshape(cout, nwords * 8), axis=-1,
                         bitorder="little")[:, :k]
    return np.where(bits > 0, 1, -1).astype(np.int8).reshape(cout, cin, kh, kw)


@dataclass
class Conv:
    tag: int                       # TAG_CONV_BIN or TAG_CONV_REAL
    cout: int
    cin: int
    kh: int = 3
    kw: int = 3
    pad: int = 1
    stride: int = 1
    packed: Optional[np.ndarray] = None   # bin: uint64 [Cout, nwords]
    wsign: Optional[np.ndarray] = None    # real: int8 [Cout, Cin, kh, kw]
    alpha: Optional[np.ndarray] = None    # real: float32 [Cout]

    @property
    def nwords(self) -> int:
        return (self.cin * self.kh * self.kw + 63) // 64

    def signs(self) -> np.ndarray:
        """int8 +-1 weights [Cout,Cin,kh,kw] regardless of the record kind."""
        if self.tag == TAG_CONV_BIN:
            return unpack_kidx(self.packed, self.cin, self.kh, self.kw)
        return np.asarray(self.wsign, np.int8)


@dataclass
class Act:
    kind: int                      # 0 = int fold on P, 1 = real fold
    c: int
    type: Optional[np.ndarray] = None
    t: Optional[np.ndarray] = None
    lo: Optional[np.ndarray] = None
    hi: Optional[np.ndarray] = None
    A: Optional[np.ndarray] = None
    B: Optional[np.ndarray] = None
    slope: Optional[np.ndarray] = None
    rsign: Optional[np.ndarray] = None


@dataclass
class Head:
    cout: int
    cin: int
    W: np.ndarray                  # float32 [Cout, Cin]
    bias: np.ndarray               # float32 [Cout]


@dataclass
class BlobV1:
    base_channels: int
    n_bands: int
    n_classes: int
    upsampler: int = UPSAMPLER_NEAREST
    version: int = VERSION
    # per encoder stage: conv1, act1, conv2, act2_skip, act2_down
    enc_conv1: List[Conv] = field(default_factory=list)
    enc_act1: List[Act] = field(default_factory=list)
    enc_conv2: List[Conv] = field(default_factory=list)
    enc_act2_skip: List[Act] = field(default_factory=list)
    enc_act2_down: List[Act] = field(default_factory=list)
    bott_conv1: Optional[Conv] = None
    bott_act1: Optional[Act] = None
    bott_conv2: Optional[Conv] = None
    bott_act2: Optional[Act] = None
    # decoder stages in blob order dec4, dec3, dec2, dec1
    dec_conv1: List[Conv] = field(default_factory=list)
    dec_act1: List[Act] = field(default_factory=list)
    dec_conv2: List[Conv] = field(default_factory=list)
    dec_act2: List[Act] = field(default_factory=list)
    head: Optional[Head] = None
    # v2 (spectral stem, python/bnn2c/blob.py:203-245): version 2, a <7i>
    # header with has_stem = n_stem_layers = 1, the stem records after it,
    # and a binary enc1.conv1 with an integer enc1.act1
    stem_conv: Optional[Conv] = None
    stem_act: Optional[Act] = None

    @property
    def has_stem(self) -> bool:
        return self.version == VERSION_STEM


# ----------------------------------------------------------------- writer --
def _w_conv(f, c: Conv) -> None:
    if c.tag == TAG_CONV_BIN:
        packed = np.ascontiguousarray(c.packed, dtype="<u8")
        if packed.shape != (c.cout, c.nwords):
            raise BlobError(f"packed shape {packed.shape} != ({c.cout},{c.nwords})")
        f.write(struct.pack("<8i", TAG_CONV_BIN, c.cout, c.cin, c.kh, c.kw,
                            c.pad, c.stride, c.nwords))
        f.write(packed.tobytes())
    elif c.tag == TAG_CONV_REAL:
        f.write(struct.pack("<7i", TAG_CONV_REAL, c.cout, c.cin, c.kh, c.kw,
                            c.pad, c.stride))
        f.write(np.ascontiguousarray(c.wsign, np.int8).tobytes())
        f.write(np.ascontiguousarray(c.alpha, "<f4").tobytes())
    else:
        raise BlobError(f"bad conv tag {c.tag}")


def _w_act(f, a: Act) -> None:
    f.write(struct.pack("<3i", TAG_ACT, a.kind, a.c))
    arrs = (a.type, a.t, a.lo, a.hi) if a.kind == 0 else (a.A, a.B, a.slope, a.rsign)
    dt = "<i4" if a.kind == 0 else "<f4"
    for arr in arrs:
        arr = np.ascontiguousarray(arr, dt)
        if arr.shape != (a.c,):
            raise BlobError(f"act array shape {arr.shape} != ({a.c},)")
        f.write(arr.tobytes())


def to_bytes(b: BlobV1) -> bytes:
    """Serialise in the record order of python/bnn2c/blob.py:181-199 (v1) or
    :226-245 (v2: the stem records right after the header)."""
    f = io.BytesIO()
    f.write(MAGIC)
    if b.has_stem:
        f.write(struct.pack("<7i", b.version, b.base_channels, b.n_bands,
                            b.n_classes, b.upsampler, 1, 1))
        _w_conv(f, b.stem_conv); _w_act(f, b.stem_act)
    else:
        f.write(struct.pack("<5i", b.version, b.base_channels, b.n_bands,
                            b.n_classes, b.upsampler))
    for i in range(4):
        _w_conv(f, b.enc_conv1[i]); _w_act(f, b.enc_act1[i])
        _w_conv(f, b.enc_conv2[i]); _w_act(f, b.enc_act2_skip[i])
        _w_act(f, b.enc_act2_down[i])
    _w_conv(f, b.bott_conv1); _w_act(f, b.bott_act1)
    _w_conv(f, b.bott_conv2); _w_act(f, b.bott_act2)
    for i in range(4):
        _w_conv(f, b.dec_conv1[i]); _w_act(f, b.dec_act1[i])
        _w_conv(f, b.dec_conv2[i]); _w_act(f, b.dec_act2[i])
    h = b.head
    f.write(struct.pack("<3i", TAG_HEAD, h.cout, h.cin))
    f.write(np.ascontiguousarray(h.W, "<f4").tobytes())
    f.write(np.ascontiguousarray(h.bias, "<f4").tobytes())
    return f.getvalue()


def write(b: BlobV1, path: str) -> str:
    with open(path, "wb") as fh:
        fh.write(to_bytes(b))
    return path


# ----------------------------------------------------------------- reader --
class _Rd:
    def __init__(self, data: bytes):
        self.d = memoryview(data)
        self.o = 0

    def take(self, n: int) -> memoryview:
        if n < 0 or self.o + n > len(self.d):
            raise BlobError("short read")
        v = self.d[self.o:self.o + n]
        self.o += n
        return v

    def ints(self, n: int):
        return struct.unpack(f"<{n}i", self.take(4 * n))

    def arr(self, dtype: str, count: int) -> np.ndarray:
        dt = np.dtype(dtype)
        return np.frombuffer(self.take(dt.itemsize * count), dt).copy()


def _r_conv(r: _Rd) -> Conv:
    tag, cout, cin, kh, kw, pad, stride = r.ints(7)
    if tag == TAG_CONV_BIN:
        (nwords,) = r.ints(1)
        if cout < 0 or nwords < 0:
            raise BlobError("bad conv dims")
        packed = r.arr("<u8", cout * nwords).reshape(cout, nwords)
        return Conv(TAG_CONV_BIN, cout, cin, kh, kw, pad, stride, packed=packed)
    if tag == TAG_CONV_REAL:
        if min(cout, cin, kh, kw) < 0:
            raise BlobError("bad conv dims")
        wsign = r.arr("i1", cout * cin * kh * kw).reshape(cout, cin, kh, kw)
        alpha = r.arr("<f4", cout)
        return Conv(TAG_CONV_REAL, cout, cin, kh, kw, pad, stride,
                    wsign=wsign, alpha=alpha)
    raise BlobError(f"bad conv tag {tag}")


def _r_act(r: _Rd) -> Act:
    tag, kind, c = r.ints(3)
    if tag != TAG_ACT:
        raise BlobError(f"bad act tag {tag}")
    if c < 0:
        raise BlobError("bad act channel count")
    if kind == 0:
        ty, t, lo, hi = (r.arr("<i4", c) for _ in range(4))
        return Act(0, c, type=ty, t=t, lo=lo, hi=hi)
    A, B, s, rs = (r.arr("<f4", c) for _ in range(4))
    return Act(kind, c, A=A, B=B, slope=s, rsign=rs)


def from_bytes(data: bytes, strict: bool = True) -> BlobV1:
    """Parse a v1 or v2 blob.  strict=True also rejects other versions and
    upsampler != 0 (the nearest-upsampler engines are the only ones)."""
    r = _Rd(data)
    if bytes(r.take(4)) != MAGIC:
        raise BlobError("bad magic")
    version, base, nb, nc, ups = r.ints(5)
    if strict and version not in (VERSION, VERSION_STEM):
        raise BlobError(f"unsupported blob version {version}")
    if strict and ups != UPSAMPLER_NEAREST:
        raise BlobError(f"unsupported upsampler {ups}")
    b = BlobV1(base_channels=base, n_bands=nb, n_classes=nc, upsampler=ups,
               version=version)
    if version == VERSION_STEM:
        has_stem, n_stem = r.ints(2)
        if (has_stem, n_stem) != (1, 1):
            raise BlobError("only has_stem=1, n_stem_layers=1 supported")
        b.stem_conv = _r_conv(r); b.stem_act = _r_act(r)
    for _ in range(4):
        b.enc_conv1.append(_r_conv(r)); b.enc_act1.append(_r_act(r))
        b.enc_conv2.append(_r_conv(r)); b.enc_act2_skip.append(_r_act(r))
        b.enc_act2_down.append(_r_act(r))
    b.bott_conv1 = _r_conv(r); b.bott_act1 = _r_act(r)
    b.bott_conv2 = _r_conv(r); b.bott_act2 = _r_act(r)
    for _ in range(4):
        b.dec_conv1.append(_r_conv(r)); b.dec_act1.append(_r_act(r))
        b.dec_conv2.append(_r_conv(r)); b.dec_act2.append(_r_act(r))
    tag, hco, hci = r.ints(3)
    if tag != TAG_HEAD:
        raise BlobError(f"bad head tag {tag}")
    W = r.arr("<f4", hco * hci).reshape(hco, hci)
    bias = r.arr("<f4", hco)
    b.head = Head(hco, hci, W, bias)
    if r.o != len(r.d):
        raise BlobError("trailing bytes in blob")
    return b


def read(path: str, strict: bool = True) -> BlobV1:
    with open(path, "rb") as fh:
        return from_bytes(fh.read(), strict=strict)
