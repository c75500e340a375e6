"""ctypes bindings for libbnn_hip.so, the gfx950 engine (include/bnn_model.h,
include/bnn_model_stem.h).

This is the Python mirror of the reference's C interface for the v1 path:
`Engine.load` / `forward` / `free` wrap bnn_load / bnn_forward / bnn_free
(csrc/bnn_model.h:57-60), `StemEngine` the v2 spectral-stem model's
bnn_stem_load / bnn_stem_forward / bnn_stem_free
(csrc/bnn_model_stem.h:61-64), and the kernel functions keep the reference's
names, argument order and batch-1 layouts (csrc/bnn_model.h:7-23), exactly as
the reference's ctypes harnesses bind them (python/verify/bconv_harness.py:36-47,
forward_driver.py:55-66).  Every call runs on the GPU.  There is no CPU
fallback: a missing library or a missing GPU raises.

With PyTorch in the same process, import torch before the first call here:
torch bundles a HIP runtime with the same soname as /opt/rocm's, and the
library must bind to the one already loaded rather than start a second.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Dict, Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libbnn_hip.so")
CLI_PATH = os.path.join(LIB_DIR, "bnn_infer")
CLI_STEM_PATH = os.path.join(LIB_DIR, "bnn_infer_stem")
HEADER = os.path.join(os.path.dirname(HERE), "include", "bnn_model.h")
HEADER_STEM = os.path.join(os.path.dirname(HERE), "include", "bnn_model_stem.h")
HEADER_REACT = os.path.join(os.path.dirname(HERE), "include", "bnn_model_react.h")
CLI_REACT_PATH = os.path.join(LIB_DIR, "bnn_infer_react")

BNN_OK, BNN_EBLOB, BNN_EARG, BNN_EHIP = 0, 1, 2, 3

_i8 = C.POINTER(C.c_int8)
_i32 = C.POINTER(C.c_int32)
_u32 = C.POINTER(C.c_uint32)
_u64 = C.POINTER(C.c_uint64)
_f32 = C.POINTER(C.c_float)
_u8 = C.POINTER(C.c_uint8)
_ci = C.c_int
_vp = C.c_void_p

STAGE_CB = C.CFUNCTYPE(None, _vp, C.c_char_p, _ci, _ci, _ci, _ci, _ci, _vp)
_DT = {0: np.int8, 1: np.int32, 2: np.float32}


class BnnError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


_LIB: Optional[C.CDLL] = None


def lib() -> C.CDLL:
    """Load libbnn_hip.so (built by __graft_entry__.build()); raise if absent."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built: run __graft_entry__.build() "
                          "(the engine has no CPU fallback)")
    L = C.CDLL(LIB_PATH)
    L.bnn_last_error.restype = C.c_char_p
    L.bnn_blob_check.argtypes = [C.c_char_p]
    L.bnn_load_status.argtypes = [C.c_char_p, C.POINTER(_vp)]
    L.bnn_free.argtypes = [_vp]
    L.bnn_forward.argtypes = [_vp, _f32, _ci, _ci, _f32]
    L.bnn_forward_batch.argtypes = [_vp, _f32, _ci, _ci, _ci, _f32]
    L.bnn_forward_device.argtypes = [_vp, _vp, _ci, _ci, _ci, _vp, _vp]
    L.bnn_forward_device_noalloc.argtypes = [_vp, _vp, _ci, _ci, _ci, _vp, _vp]
    L.bnn_cert_stats.argtypes = [_vp, C.POINTER(C.c_ulonglong), C.POINTER(C.c_ulonglong)]
    L.bnn_forward_debug.argtypes = [_vp, _f32, _ci, _ci, _ci, _f32, STAGE_CB, _vp]
    L.bnn_forward_patched.argtypes = [_vp, _f32, _ci, _ci, _f32, _ci]
    L.bnn_forward_patched_device.argtypes = [_vp, _vp, _ci, _ci, _vp, _ci, _vp]
    L.bnn_stream.argtypes = [_vp]
    L.bnn_stream.restype = _vp
    # v2 (spectral stem): the same signatures on a StemModel*
    L.bnn_stem_blob_check.argtypes = [C.c_char_p]
    L.bnn_stem_load_status.argtypes = [C.c_char_p, C.POINTER(_vp)]
    L.bnn_stem_free.argtypes = [_vp]
    L.bnn_stem_forward.argtypes = [_vp, _f32, _ci, _ci, _f32]
    L.bnn_stem_forward_batch.argtypes = [_vp, _f32, _ci, _ci, _ci, _f32]
    L.bnn_stem_forward_device.argtypes = [_vp, _vp, _ci, _ci, _ci, _vp, _vp]
    L.bnn_stem_forward_debug.argtypes = [_vp, _f32, _ci, _ci, _ci, _f32, STAGE_CB, _vp]
    L.bnn_stem_forward_patched.argtypes = [_vp, _f32, _ci, _ci, _f32, _ci]
    L.bnn_stem_forward_patched_device.argtypes = [_vp, _vp, _ci, _ci, _vp, _ci, _vp]
    L.bnn_stem_stream.argtypes = [_vp]
    L.bnn_stem_stream.restype = _vp
    # v3 (ReActNet real highway), include/bnn_model_react.h
    L.bnn_react_blob_check.argtypes = [C.c_char_p]
    L.bnn_react_load_status.argtypes = [C.c_char_p, C.POINTER(_vp)]
    L.bnn_free_react.argtypes = [_vp]
    L.bnn_forward_react.argtypes = [_vp, _f32, _ci, _ci, _f32]
    L.bnn_react_forward_batch.argtypes = [_vp, _f32, _ci, _ci, _ci, _f32]
    L.bnn_react_forward_device.argtypes = [_vp, _vp, _ci, _ci, _ci, _vp, _vp]
    L.bnn_react_forward_debug.argtypes = [_vp, _f32, _ci, _ci, _ci, _f32, STAGE_CB, _vp]
    L.bnn_react_forward_patched.argtypes = [_vp, _f32, _ci, _ci, _f32, _ci]
    L.bnn_react_forward_patched_device.argtypes = [_vp, _vp, _ci, _ci, _vp, _ci, _vp]
    L.bnn_react_stream.argtypes = [_vp]
    L.bnn_react_stream.restype = _vp
    L.bnn_prof_enable.argtypes = [_ci]
    L.bnn_prof_count.restype = _ci
    L.bnn_prof_get.argtypes = [_ci, C.c_char_p, _ci, C.c_char_p, _ci, C.POINTER(C.c_double),
                               C.POINTER(C.c_double)]
    L.prof_reset.argtypes = []
    L.prof_now.restype = C.c_double
    L.bnn_layer_create.argtypes = [_u64, _ci, _ci] + [_i32] * 8
    L.bnn_layer_create.restype = _vp
    L.bnn_layer_free.argtypes = [_vp]
    L.bnn_layer_P_device.argtypes = [_vp, _vp, _ci, _ci, _ci, _vp, _vp]
    L.bnn_layer_fold_pool_device.argtypes = [_vp, _vp, _ci, _ci, _ci, _vp, _vp, _vp]
    L.bnn_pack_act_device.argtypes = [_vp, _vp, _ci, _ci, _ci, _ci, _vp]
    L.bnn_fold_canon.argtypes = [_i32, _i32, _i32, _i32, _ci, _i32, _u32, _u8]
    # reference kernel ABI
    for nm in ("bconv_xnor", "bconv_xnor_packed", "bconv_dispatch"):
        getattr(L, nm).argtypes = [_i8, _u64, _i32] + [_ci] * 8
    L.bconv_naive_int.argtypes = [_i8, _i8, _i32] + [_ci] * 8
    L.pack_weights.argtypes = [_i8, _u64, _ci, _ci, _ci, _ci]
    L.conv_realin_naive.argtypes = [_f32, _i8, _f32, _f32] + [_ci] * 8
    L.maxpool_P.argtypes = [_i32, _i32, _ci, _ci, _ci, _ci, _ci]
    L.apply_fold_int.argtypes = [_i32, _i8, _ci, _ci, _ci, _i32, _i32, _i32, _i32]
    L.apply_fold_real.argtypes = [_f32, _i8, _ci, _ci, _ci, _f32, _f32, _f32, _f32]
    L.head_1x1.argtypes = [_f32, _f32, _f32, _f32, _ci, _ci, _ci, _ci]
    _LIB = L
    return L


def last_error() -> str:
    return lib().bnn_last_error().decode()


def _check(rc: int) -> None:
    if rc != BNN_OK:
        raise BnnError(rc, last_error())


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def blob_check(path: str) -> None:
    """Parse and validate a v1 blob on the host only; raises BnnError."""
    _check(lib().bnn_blob_check(path.encode()))


def stem_blob_check(path: str) -> None:
    """Parse and validate a v2 (spectral-stem) blob on the host only."""
    _check(lib().bnn_stem_blob_check(path.encode()))


def header_symbols(path: str = HEADER):
    """Function names declared in a header (default include/bnn_model.h)."""
    import re
    txt = open(path).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    txt = re.sub(r"\btypedef\b[^;]*;", "", txt)
    txt = re.sub(r"^\s*#.*$", "", txt, flags=re.M)
    return sorted(set(re.findall(r"\b([A-Za-z_]\w*)\s*\([^;{()]*(?:\([^()]*\)[^;{()]*)*\)\s*;", txt))
                  - {"if", "sizeof"})


class Engine:
    """A loaded v1 model on the GPU (the reference's Model*)."""

    _api = "bnn_"  # entry-point prefix: bnn_load_status, bnn_forward_batch, ...

    def __init__(self, path: str):
        h = _vp()
        _check(self._fn("load_status")(path.encode(), C.byref(h)))
        self.h = h
        hdr = (C.c_int * 5).from_address(h.value)
        self.version, self.base, self.n_bands, self.n_classes, self.upsampler = list(hdr)

    def _fn(self, name: str):
        return getattr(lib(), self._api + name)

    def close(self) -> None:
        if getattr(self, "h", None):
            self._fn("free")(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, x: np.ndarray) -> np.ndarray:
        """One patch [n_bands,H,W] -> [n_classes,H,W] (the reference's bnn_forward)."""
        return self.forward_batch(np.asarray(x)[None])[0]

    def forward_batch(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        N, nb, H, W = x.shape
        out = np.empty((N, self.n_classes, H, W), np.float32)
        _check(self._fn("forward_batch")(self.h, _p(x, _f32), N, H, W, _p(out, _f32)))
        return out

    def forward_batch_ptr(self, x_ptr: int, N: int, H: int, W: int, out_ptr: int) -> None:
        """bnn_forward_batch on caller-owned host buffers given by address
        (e.g. pinned memory): the copies in and out are part of the call."""
        _check(self._fn("forward_batch")(self.h, C.cast(C.c_void_p(x_ptr), _f32), N, H, W,
                                         C.cast(C.c_void_p(out_ptr), _f32)))

    def forward_device(self, d_in: int, N: int, H: int, W: int, d_out: int,
                       stream: Optional[int] = None) -> None:
        _check(self._fn("forward_device")(self.h, _vp(d_in), N, H, W, _vp(d_out),
                                          _vp(stream or None)))

    def forward_device_noalloc(self, d_in: int, N: int, H: int, W: int, d_out: int,
                               stream: Optional[int] = None) -> None:
        """bnn_forward_device with no device allocation (v1 models only): the
        inter-layer tensors live in the library's fixed per-GPU scratch array."""
        _check(lib().bnn_forward_device_noalloc(self.h, _vp(d_in), N, H, W, _vp(d_out),
                                                _vp(stream or None)))

    def cert_stats(self) -> tuple:
        """(undecided, outputs) of the certified first conv since the last
        call (bnn_cert_stats): the outputs it recomputed in the reference's
        order, and all it made.  Waits for the model's GPU."""
        u, o = C.c_ulonglong(0), C.c_ulonglong(0)
        _check(lib().bnn_cert_stats(self.h, C.byref(u), C.byref(o)))
        return int(u.value), int(o.value)

    def forward_patched(self, cube: np.ndarray, P: int = 32) -> np.ndarray:
        """Scene [n_bands, H, W] -> logit map [n_classes, H, W] by independent
        P x P patches, edge patches zero past the scene (bnn_forward_patched)."""
        cube = np.ascontiguousarray(cube, np.float32)
        nb, H, W = cube.shape
        out = np.empty((self.n_classes, H, W), np.float32)
        _check(self._fn("forward_patched")(self.h, _p(cube, _f32), H, W, _p(out, _f32), P))
        return out

    def forward_patched_device(self, d_cube: int, H: int, W: int, d_map: int, P: int = 32,
                               stream: Optional[int] = None) -> None:
        _check(self._fn("forward_patched_device")(self.h, _vp(d_cube), H, W, _vp(d_map), P,
                                                  _vp(stream or None)))

    def stream(self) -> int:
        return self._fn("stream")(self.h)

    def forward_debug(self, x: np.ndarray):
        """Forward with every intermediate stage returned as numpy arrays
        (binary stages as int8 +-1 [N,C,H,W], P as int32, the first real
        conv's output -- enc1.conv1, or stem.conv for v2 -- as f32)."""
        x = np.ascontiguousarray(x, np.float32)
        N, nb, H, W = x.shape
        out = np.empty((N, self.n_classes, H, W), np.float32)
        got: Dict[str, np.ndarray] = {}

        def cb(_ctx, name, dtype, n, c, h, w, data):
            cnt = n * c * h * w
            ct = np.ctypeslib.as_ctypes_type(_DT[dtype])
            arr = np.ctypeslib.as_array(C.cast(data, C.POINTER(ct)), shape=(cnt,))
            got[name.decode()] = arr.copy().reshape(n, c, h, w)

        _check(self._fn("forward_debug")(self.h, _p(x, _f32), N, H, W, _p(out, _f32),
                                         STAGE_CB(cb), None))
        return out, got


class StemEngine(Engine):
    """A loaded v2 spectral-stem model on the GPU (the reference's
    StemModel*, csrc/bnn_model_stem.h:44-64); the same methods as Engine."""

    _api = "bnn_stem_"

    def __init__(self, path: str):
        super().__init__(path)
        # has_stem, n_stem_layers, then the stem ConvS (8-byte aligned) at 32
        ints = (C.c_int * 10).from_address(self.h.value)
        self.has_stem, self.n_stem_layers = ints[5], ints[6]
        self.stem_channels = ints[9]


class ReactEngine(Engine):
    """A loaded v3 (ReActNet real-highway) model on the GPU (the reference's
    ModelR*, csrc/bnn_model_react.h:82-98); the same methods as Engine.
    forward_debug returns the stages include/bnn_model_react.h lists."""

    _api = "bnn_react_"

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().bnn_free_react(self.h)
            self.h = None


def react_blob_check(path: str) -> None:
    """Parse and validate a v3 (ReActNet) blob on the host only."""
    _check(lib().bnn_react_blob_check(path.encode()))


# ---------------------------------------------------------------- profiler --
def prof_enable(on: bool) -> None:
    lib().bnn_prof_enable(int(on))


def prof_reset() -> None:
    lib().prof_reset()


def prof_records():
    L = lib()
    recs = []
    lab = C.create_string_buffer(64)
    op = C.create_string_buffer(32)
    ms = C.c_double()
    work = C.c_double()
    for i in range(L.bnn_prof_count()):
        _check(L.bnn_prof_get(i, lab, 64, op, 32, C.byref(ms), C.byref(work)))
        recs.append((lab.value.decode(), op.value.decode(), ms.value, work.value))
    return recs


# --------------------------------------------------------- isolated layers --
class ConvLayer:
    """One binary 3x3 conv (+ optional rules) resident on the GPU."""

    def __init__(self, packed_w: np.ndarray, cin: int, cout: int, fold1=None, fold2=None):
        self._keep = []
        args = []
        for f in (fold1, fold2):
            if f is None:
                args += [None] * 4
            else:
                arrs = [np.ascontiguousarray(v, np.int32) for v in f]
                self._keep += arrs
                args += [_p(v, _i32) for v in arrs]
        pw = np.ascontiguousarray(packed_w, np.uint64)
        h = lib().bnn_layer_create(_p(pw, _u64), cin, cout, *args)
        if not h:
            raise BnnError(BNN_EARG, last_error())
        self.h = h
        self.cin, self.cout = cin, cout

    def close(self):
        if getattr(self, "h", None):
            lib().bnn_layer_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def P_device(self, d_act: int, N: int, H: int, W: int, d_P: int, stream: Optional[int] = None):
        _check(lib().bnn_layer_P_device(self.h, _vp(d_act), N, H, W, _vp(d_P),
                                        _vp(stream or None)))

    def fold_pool_device(self, d_act: int, N: int, H: int, W: int, d_skip: Optional[int],
                         d_down: int, stream: Optional[int] = None):
        _check(lib().bnn_layer_fold_pool_device(self.h, _vp(d_act), N, H, W,
                                                _vp(d_skip) if d_skip else None, _vp(d_down),
                                                _vp(stream or None)))


def pack_act_device(d_a: int, d_out: int, N: int, Cc: int, H: int, W: int,
                    stream: Optional[int] = None) -> None:
    _check(lib().bnn_pack_act_device(_vp(d_a), _vp(d_out), N, Cc, H, W,
                                     _vp(stream or None)))


def fold_canon(ty, t, lo, hi):
    arrs = [np.ascontiguousarray(v, np.int32) for v in (ty, t, lo, hi)]
    c = len(arrs[0])
    olo = np.zeros(c, np.int32)
    owid = np.zeros(c, np.uint32)
    oinv = np.zeros(c, np.uint8)
    lib().bnn_fold_canon(*[_p(v, _i32) for v in arrs], c, _p(olo, _i32), _p(owid, _u32), _p(oinv, _u8))
    return olo, owid, oinv


# ------------------------------------------------ reference kernel ABI -----
def _od(n, k, pad, stride):
    return (n + 2 * pad - k) // stride + 1


def bconv(a, packed_w, cout, kh=3, kw=3, pad=1, stride=1, fn="bconv_dispatch"):
    a = np.ascontiguousarray(a, np.int8)
    pw = np.ascontiguousarray(packed_w, np.uint64)
    cin, H, W = a.shape
    P = np.zeros((cout, _od(H, kh, pad, stride), _od(W, kw, pad, stride)), np.int32)
    getattr(lib(), fn)(_p(a, _i8), _p(pw, _u64), _p(P, _i32), cin, H, W, cout, kh, kw, pad, stride)
    return P


def bconv_naive_int(a, wsign, pad=1, stride=1):
    a = np.ascontiguousarray(a, np.int8)
    w = np.ascontiguousarray(wsign, np.int8)
    cin, H, W = a.shape
    cout, _, kh, kw = w.shape
    P = np.zeros((cout, _od(H, kh, pad, stride), _od(W, kw, pad, stride)), np.int32)
    lib().bconv_naive_int(_p(a, _i8), _p(w, _i8), _p(P, _i32), cin, H, W, cout, kh, kw, pad, stride)
    return P


def pack_weights(wsign):
    w = np.ascontiguousarray(wsign, np.int8)
    co, ci, kh, kw = w.shape
    out = np.zeros((co, (ci * kh * kw + 63) // 64), np.uint64)
    lib().pack_weights(_p(w, _i8), _p(out, _u64), co, ci, kh, kw)
    return out


def conv_realin(x, wsign, alpha, pad=1, stride=1):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(wsign, np.int8)
    al = np.ascontiguousarray(alpha, np.float32)
    cin, H, W = x.shape
    cout, _, kh, kw = w.shape
    out = np.zeros((cout, _od(H, kh, pad, stride), _od(W, kw, pad, stride)), np.float32)
    lib().conv_realin_naive(_p(x, _f32), _p(w, _i8), _p(al, _f32), _p(out, _f32), cin, H, W, cout, kh, kw,
                            pad, stride)
    return out


def maxpool_P(P, k=2, stride=2):
    P = np.ascontiguousarray(P, np.int32)
    c, H, W = P.shape
    out = np.zeros((c, (H - k) // stride + 1, (W - k) // stride + 1), np.int32)
    lib().maxpool_P(_p(P, _i32), _p(out, _i32), c, H, W, k, stride)
    return out


def apply_fold_int(P, ty, t, lo, hi):
    P = np.ascontiguousarray(P, np.int32)
    c, H, W = P.shape
    out = np.zeros(P.shape, np.int8)
    arrs = [np.ascontiguousarray(v, np.int32) for v in (ty, t, lo, hi)]
    lib().apply_fold_int(_p(P, _i32), _p(out, _i8), c, H, W, *[_p(v, _i32) for v in arrs])
    return out


def apply_fold_real(x, A, B, slope, rsign):
    x = np.ascontiguousarray(x, np.float32)
    c, H, W = x.shape
    out = np.zeros(x.shape, np.int8)
    arrs = [np.ascontiguousarray(v, np.float32) for v in (A, B, slope, rsign)]
    lib().apply_fold_real(_p(x, _f32), _p(out, _i8), c, H, W, *[_p(v, _f32) for v in arrs])
    return out


def head_1x1(a, Wt, bias):
    a = np.ascontiguousarray(a, np.float32)
    Wt = np.ascontiguousarray(Wt, np.float32)
    b = np.ascontiguousarray(bias, np.float32)
    cin, H, W = a.shape
    out = np.zeros((Wt.shape[0], H, W), np.float32)
    lib().head_1x1(_p(a, _f32), _p(Wt, _f32), _p(b, _f32), _p(out, _f32), cin, H, W, Wt.shape[0])
    return out


# ------------------------------------------------------------ bit helpers --
def pack_bits_nhwc(a: np.ndarray) -> np.ndarray:
    """int8 +-1 [N,C,H,W] -> uint32 [N,H,W,ceil(C/32)] (bit = a > 0)."""
    a = np.asarray(a)
    N, Cc, H, W = a.shape
    cw = (Cc + 31) // 32
    bits = np.zeros((N, H, W, cw * 32), np.uint8)
    bits[..., :Cc] = (a > 0).transpose(0, 2, 3, 1)
    by = np.packbits(bits.reshape(N, H, W, cw * 4, 8), axis=-1, bitorder="little")
    return by.reshape(N, H, W, cw * 4).view("<u4").reshape(N, H, W, cw).copy()


def unpack_bits_nhwc(words: np.ndarray, Cc: int) -> np.ndarray:
    """uint32 [N,H,W,cw] -> int8 +-1 [N,C,H,W]."""
    w = np.ascontiguousarray(words, "<u4")
    N, H, W, cw = w.shape
    bits = np.unpackbits(w.view(np.uint8).reshape(N, H, W, cw * 4), axis=-1, bitorder="little")
    return np.where(bits[..., :Cc] > 0, 1, -1).astype(np.int8).transpose(0, 3, 1, 2).copy()
