"""ctypes bindings for the CPU checker. TEST INFRASTRUCTURE ONLY.

`Oracle` wraps liboracle.so, the clean-room C restatement of the reference v1
forward (oracle/bnn_oracle.c).  `RefC` wraps oracle/_ref/libbnnref.so, the
reference's own C sources compiled by `make -C oracle ref`; it exists only
where /root/reference was present at build time (or the built file travelled
with the tree), and every user of it must treat it as optional.

Arrays are numpy, batch-1 row-major exactly as the C signatures take them.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from typing import Dict, Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libbnnref.so")
REF_CLI = os.path.join(HERE, "_ref", "bnn_infer")
REF_CLI_STEM = os.path.join(HERE, "_ref", "bnn_infer_stem")

_i8 = C.POINTER(C.c_int8)
_i32 = C.POINTER(C.c_int32)
_u64 = C.POINTER(C.c_uint64)
_f32 = C.POINTER(C.c_float)
_ci = C.c_int

STAGE_CB = C.CFUNCTYPE(None, C.c_void_p, C.c_char_p, C.c_int, C.c_int, C.c_int,
                       C.c_int, C.c_void_p)
_DT = {0: np.int8, 1: np.int32, 2: np.float32}


def _p(a: np.ndarray, ptype):
    return a.ctypes.data_as(ptype)


def build(force: bool = False) -> None:
    if force or not os.path.exists(LIB):
        subprocess.run(["make", "-s", "-C", HERE], check=True)


def _out_dim(n, k, pad, stride):
    return (n + 2 * pad - k) // stride + 1


class Oracle:
    def __init__(self, path: str = LIB):
        if not os.path.exists(path):
            build()
        L = self.lib = C.CDLL(path)
        L.orc_parse.argtypes = [C.c_char_p, C.c_size_t, _ci, C.POINTER(C.c_void_p), C.c_char_p, _ci]
        L.orc_free.argtypes = [C.c_void_p]
        L.orc_forward.argtypes = [C.c_void_p, _f32, _ci, _ci, _f32, STAGE_CB, C.c_void_p]
        L.orc_forward_batch.argtypes = [C.c_void_p, _f32, _ci, _ci, _ci, _f32]
        L.orc_forward_batch_par.argtypes = [C.c_void_p, _f32, _ci, _ci, _ci, _f32]
        L.orc_pack_kidx.argtypes = [_i8, _u64, _ci, _ci, _ci, _ci]
        for nm in ("orc_bconv_dense", "orc_bconv_chan", "orc_bconv"):
            getattr(L, nm).argtypes = [_i8, _u64, _i32] + [_ci] * 8
        L.orc_bconv_naive.argtypes = [_i8, _i8, _i32] + [_ci] * 8
        L.orc_conv_real.argtypes = [_f32, _i8, _f32, _f32] + [_ci] * 8
        L.orc_fold_int.argtypes = [_i32, _i8, _ci, _ci, _ci, _i32, _i32, _i32, _i32]
        L.orc_fold_real.argtypes = [_f32, _i8, _ci, _ci, _ci, _f32, _f32, _f32, _f32]
        L.orc_maxpool.argtypes = [_i32, _i32, _ci, _ci, _ci, _ci, _ci]
        L.orc_head.argtypes = [_f32, _f32, _f32, _f32, _ci, _ci, _ci, _ci]
        L.orc_up_cat.argtypes = [_i8, _ci, _ci, _ci, _i8, _ci, _ci, _ci, _i8]

    # ---- model ----
    def parse(self, data: bytes, strict: bool = True):
        h = C.c_void_p()
        err = C.create_string_buffer(256)
        rc = self.lib.orc_parse(data, len(data), int(strict), C.byref(h), err, 256)
        if rc:
            raise ValueError(err.value.decode())
        return OracleModel(self, h)

    # ---- kernels ----
    def pack_kidx(self, wsign):
        w = np.ascontiguousarray(wsign, np.int8)
        co, ci, kh, kw = w.shape
        out = np.zeros((co, (ci * kh * kw + 63) // 64), np.uint64)
        self.lib.orc_pack_kidx(_p(w, _i8), _p(out, _u64), co, ci, kh, kw)
        return out

    def bconv(self, a, bits, cout, kh=3, kw=3, pad=1, stride=1, kind="dispatch"):
        a = np.ascontiguousarray(a, np.int8)
        bits = np.ascontiguousarray(bits, np.uint64)
        cin, H, W = a.shape
        P = np.zeros((cout, _out_dim(H, kh, pad, stride), _out_dim(W, kw, pad, stride)), np.int32)
        fn = {"dispatch": "orc_bconv", "dense": "orc_bconv_dense", "chan": "orc_bconv_chan"}[kind]
        getattr(self.lib, fn)(_p(a, _i8), _p(bits, _u64), _p(P, _i32), cin, H, W, cout, kh, kw, pad, stride)
        return P

    def bconv_naive(self, a, wsign, pad=1, stride=1):
        a = np.ascontiguousarray(a, np.int8)
        w = np.ascontiguousarray(wsign, np.int8)
        cin, H, W = a.shape
        cout, _, kh, kw = w.shape
        P = np.zeros((cout, _out_dim(H, kh, pad, stride), _out_dim(W, kw, pad, stride)), np.int32)
        self.lib.orc_bconv_naive(_p(a, _i8), _p(w, _i8), _p(P, _i32), cin, H, W, cout, kh, kw, pad, stride)
        return P

    def conv_real(self, x, wsign, alpha, pad=1, stride=1):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(wsign, np.int8)
        al = np.ascontiguousarray(alpha, np.float32)
        cin, H, W = x.shape
        cout, _, kh, kw = w.shape
        out = np.zeros((cout, _out_dim(H, kh, pad, stride), _out_dim(W, kw, pad, stride)), np.float32)
        self.lib.orc_conv_real(_p(x, _f32), _p(w, _i8), _p(al, _f32), _p(out, _f32),
                               cin, H, W, cout, kh, kw, pad, stride)
        return out

    def fold_int(self, P, ty, t, lo, hi):
        P = np.ascontiguousarray(P, np.int32)
        c, H, W = P.shape
        out = np.zeros(P.shape, np.int8)
        arrs = [np.ascontiguousarray(v, np.int32) for v in (ty, t, lo, hi)]
        self.lib.orc_fold_int(_p(P, _i32), _p(out, _i8), c, H, W, *[_p(v, _i32) for v in arrs])
        return out

    def fold_real(self, x, A, B, slope, rsign):
        x = np.ascontiguousarray(x, np.float32)
        c, H, W = x.shape
        out = np.zeros(x.shape, np.int8)
        arrs = [np.ascontiguousarray(v, np.float32) for v in (A, B, slope, rsign)]
        self.lib.orc_fold_real(_p(x, _f32), _p(out, _i8), c, H, W, *[_p(v, _f32) for v in arrs])
        return out

    def maxpool(self, P, k=2, stride=2):
        P = np.ascontiguousarray(P, np.int32)
        c, H, W = P.shape
        out = np.zeros((c, (H - k) // stride + 1, (W - k) // stride + 1), np.int32)
        self.lib.orc_maxpool(_p(P, _i32), _p(out, _i32), c, H, W, k, stride)
        return out

    def head(self, a, Wt, bias):
        a = np.ascontiguousarray(a, np.float32)
        Wt = np.ascontiguousarray(Wt, np.float32)
        b = np.ascontiguousarray(bias, np.float32)
        cin, H, W = a.shape
        out = np.zeros((Wt.shape[0], H, W), np.float32)
        self.lib.orc_head(_p(a, _f32), _p(Wt, _f32), _p(b, _f32), _p(out, _f32), cin, H, W, Wt.shape[0])
        return out

    def up_cat(self, skip, x):
        s = np.ascontiguousarray(skip, np.int8)
        x = np.ascontiguousarray(x, np.int8)
        sC, sH, sW = s.shape
        xC, hH, hW = x.shape
        out = np.zeros((sC + xC, sH, sW), np.int8)
        self.lib.orc_up_cat(_p(s, _i8), sC, sH, sW, _p(x, _i8), xC, hH, hW, _p(out, _i8))
        return out


class OracleModel:
    def __init__(self, orc: Oracle, handle):
        self.orc = orc
        self.h = handle

    def __del__(self):
        try:
            if self.h:
                self.orc.lib.orc_free(self.h)
                self.h = None
        except Exception:
            pass

    def _dims(self):
        # n_bands / n_classes are the 3rd/4th int of orc_model
        hdr = (C.c_int * 5).from_address(self.h.value)
        return hdr[2], hdr[3]

    def forward(self, x: np.ndarray, stages: bool = False):
        """x [n_bands,H,W] -> logits [n_classes,H,W] (+ dict of every stage)."""
        x = np.ascontiguousarray(x, np.float32)
        nb, H, W = x.shape
        _, ncls = self._dims()
        logits = np.zeros((ncls, H, W), np.float32)
        got: Dict[str, np.ndarray] = {}

        def cb(_ctx, name, dtype, c, h, w, data):
            n = c * h * w
            arr = np.ctypeslib.as_array(C.cast(data, C.POINTER(np.ctypeslib.as_ctypes_type(_DT[dtype]))),
                                        shape=(n,)).copy().reshape(c, h, w)
            got[name.decode()] = arr

        cbf = STAGE_CB(cb) if stages else STAGE_CB()
        rc = self.orc.lib.orc_forward(self.h, _p(x, _f32), H, W, _p(logits, _f32), cbf, None)
        if rc:
            raise ValueError("oracle forward rejected the model/shape")
        return (logits, got) if stages else logits

    def forward_batch(self, x: np.ndarray, parallel: bool = True) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        N, nb, H, W = x.shape
        _, ncls = self._dims()
        out = np.zeros((N, ncls, H, W), np.float32)
        fn = self.orc.lib.orc_forward_batch_par if parallel else self.orc.lib.orc_forward_batch
        if fn(self.h, _p(x, _f32), N, H, W, _p(out, _f32)):
            raise ValueError("oracle forward rejected the model/shape")
        return out


# ------------------------------------------------------------ reference C --
def ref_available() -> bool:
    return os.path.exists(REF_LIB)


class RefC:
    """The reference's own C kernels and engine, built from its sources.

    bnn_load() exits the process on a malformed blob (csrc/bnn_model.c:17-24),
    so only well-formed blobs may be given to it."""

    def __init__(self, path: str = REF_LIB):
        L = self.lib = C.CDLL(path)
        L.bnn_load.argtypes = [C.c_char_p]
        L.bnn_load.restype = C.c_void_p
        L.bnn_free.argtypes = [C.c_void_p]
        L.bnn_forward.argtypes = [C.c_void_p, _f32, _ci, _ci, _f32]
        L.pack_weights.argtypes = [_i8, _u64, _ci, _ci, _ci, _ci]
        for nm in ("bconv_xnor", "bconv_xnor_packed", "bconv_dispatch"):
            getattr(L, nm).argtypes = [_i8, _u64, _i32] + [_ci] * 8
        L.bconv_naive_int.argtypes = [_i8, _i8, _i32] + [_ci] * 8
        L.conv_realin_naive.argtypes = [_f32, _i8, _f32, _f32] + [_ci] * 8
        L.apply_fold_int.argtypes = [_i32, _i8, _ci, _ci, _ci, _i32, _i32, _i32, _i32]
        L.apply_fold_real.argtypes = [_f32, _i8, _ci, _ci, _ci, _f32, _f32, _f32, _f32]
        L.maxpool_P.argtypes = [_i32, _i32, _ci, _ci, _ci, _ci, _ci]
        L.head_1x1.argtypes = [_f32, _f32, _f32, _f32, _ci, _ci, _ci, _ci]
        # v2 engine (csrc/bnn_model_stem.h:61-64)
        L.bnn_stem_load.argtypes = [C.c_char_p]
        L.bnn_stem_load.restype = C.c_void_p
        L.bnn_stem_free.argtypes = [C.c_void_p]
        L.bnn_stem_forward.argtypes = [C.c_void_p, _f32, _ci, _ci, _f32]

    def stem_load(self, path: str):
        """bnn_stem_load: (handle, n_bands, n_classes); exits on a bad blob"""
        h = self.lib.bnn_stem_load(path.encode())
        hdr = (C.c_int * 7).from_address(h)
        return h, hdr[2], hdr[3]

    def stem_forward(self, handle, x: np.ndarray, n_classes: int) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        _, H, W = x.shape
        out = np.zeros((n_classes, H, W), np.float32)
        self.lib.bnn_stem_forward(C.c_void_p(handle), _p(x, _f32), H, W, _p(out, _f32))
        return out

    def stem_free(self, handle):
        self.lib.bnn_stem_free(C.c_void_p(handle))

    def load(self, path: str):
        h = self.lib.bnn_load(path.encode())
        hdr = (C.c_int * 5).from_address(h)
        return h, hdr[2], hdr[3]

    def forward(self, handle, x: np.ndarray, n_classes: int) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        _, H, W = x.shape
        out = np.zeros((n_classes, H, W), np.float32)
        self.lib.bnn_forward(C.c_void_p(handle), _p(x, _f32), H, W, _p(out, _f32))
        return out

    def free(self, handle):
        self.lib.bnn_free(C.c_void_p(handle))

    def bconv(self, a, bits, cout, kh=3, kw=3, pad=1, stride=1, kind="dispatch"):
        a = np.ascontiguousarray(a, np.int8)
        bits = np.ascontiguousarray(bits, np.uint64)
        cin, H, W = a.shape
        P = np.zeros((cout, _out_dim(H, kh, pad, stride), _out_dim(W, kw, pad, stride)), np.int32)
        fn = {"dispatch": "bconv_dispatch", "dense": "bconv_xnor", "chan": "bconv_xnor_packed"}[kind]
        getattr(self.lib, fn)(_p(a, _i8), _p(bits, _u64), _p(P, _i32), cin, H, W, cout, kh, kw, pad, stride)
        return P

    def bconv_naive(self, a, wsign, pad=1, stride=1):
        a = np.ascontiguousarray(a, np.int8)
        w = np.ascontiguousarray(wsign, np.int8)
        cin, H, W = a.shape
        cout, _, kh, kw = w.shape
        P = np.zeros((cout, _out_dim(H, kh, pad, stride), _out_dim(W, kw, pad, stride)), np.int32)
        self.lib.bconv_naive_int(_p(a, _i8), _p(w, _i8), _p(P, _i32), cin, H, W, cout, kh, kw, pad, stride)
        return P

    def pack_weights(self, wsign):
        w = np.ascontiguousarray(wsign, np.int8)
        co, ci, kh, kw = w.shape
        out = np.zeros((co, (ci * kh * kw + 63) // 64), np.uint64)
        self.lib.pack_weights(_p(w, _i8), _p(out, _u64), co, ci, kh, kw)
        return out

    def conv_real(self, x, wsign, alpha, pad=1, stride=1):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(wsign, np.int8)
        al = np.ascontiguousarray(alpha, np.float32)
        cin, H, W = x.shape
        cout, _, kh, kw = w.shape
        out = np.zeros((cout, _out_dim(H, kh, pad, stride), _out_dim(W, kw, pad, stride)), np.float32)
        self.lib.conv_realin_naive(_p(x, _f32), _p(w, _i8), _p(al, _f32), _p(out, _f32),
                                   cin, H, W, cout, kh, kw, pad, stride)
        return out

    def fold_int(self, P, ty, t, lo, hi):
        P = np.ascontiguousarray(P, np.int32)
        c, H, W = P.shape
        out = np.zeros(P.shape, np.int8)
        arrs = [np.ascontiguousarray(v, np.int32) for v in (ty, t, lo, hi)]
        self.lib.apply_fold_int(_p(P, _i32), _p(out, _i8), c, H, W, *[_p(v, _i32) for v in arrs])
        return out

    def fold_real(self, x, A, B, slope, rsign):
        x = np.ascontiguousarray(x, np.float32)
        c, H, W = x.shape
        out = np.zeros(x.shape, np.int8)
        arrs = [np.ascontiguousarray(v, np.float32) for v in (A, B, slope, rsign)]
        self.lib.apply_fold_real(_p(x, _f32), _p(out, _i8), c, H, W, *[_p(v, _f32) for v in arrs])
        return out

    def maxpool(self, P, k=2, stride=2):
        P = np.ascontiguousarray(P, np.int32)
        c, H, W = P.shape
        out = np.zeros((c, (H - k) // stride + 1, (W - k) // stride + 1), np.int32)
        self.lib.maxpool_P(_p(P, _i32), _p(out, _i32), c, H, W, k, stride)
        return out

    def head(self, a, Wt, bias):
        a = np.ascontiguousarray(a, np.float32)
        Wt = np.ascontiguousarray(Wt, np.float32)
        b = np.ascontiguousarray(bias, np.float32)
        cin, H, W = a.shape
        out = np.zeros((Wt.shape[0], H, W), np.float32)
        self.lib.head_1x1(_p(a, _f32), _p(Wt, _f32), _p(b, _f32), _p(out, _f32), cin, H, W, Wt.shape[0])
        return out


# ------------------------------------------------------------- v3 oracle --
REACT_REF_LIB = os.path.join(HERE, "_ref", "libreactref.so")
REACT_REF_CLI = os.path.join(HERE, "_ref", "bnn_infer_react")
_i16 = C.POINTER(C.c_int16)


class ReactOracle:
    """The clean-room v3 (ReActNet) restatement in liboracle.so
    (oracle/bnn_oracle_react.c)."""

    def __init__(self, path: str = LIB):
        if not os.path.exists(path):
            build()
        L = self.lib = C.CDLL(path)
        L.orr_parse.argtypes = [C.c_char_p, C.c_size_t, C.POINTER(C.c_void_p), C.c_char_p, _ci]
        L.orr_free.argtypes = [C.c_void_p]
        L.orr_forward.argtypes = [C.c_void_p, _f32, _ci, _ci, _f32, STAGE_CB, C.c_void_p]
        L.orr_forward_patched.argtypes = [C.c_void_p, _f32, _ci, _ci, _f32, _ci]
        L.orr_forward_batch_par.argtypes = [C.c_void_p, _f32, _ci, _ci, _ci, _f32]
        L.orr_proj.argtypes = [_f32, _f32, _f32, _ci, _ci, _ci]
        L.orr_conv3.argtypes = [_f32, _i8, _f32, _f32, _ci, _ci, _ci, _ci]
        L.orr_epi_int.argtypes = [_i32, _f32, _f32, _ci, _ci, _f32, _f32, _f32, _f32]
        L.orr_epi_real.argtypes = [_f32, _f32, _f32, _ci, _ci, _f32, _f32, _f32, _f32]
        L.orr_tap.argtypes = [_f32, _i8, _ci, _ci, _f32]
        L.orr_epi_plain.argtypes = [C.c_void_p, _ci, _f32, _f32, _ci, _ci, _f32, _f32, _f32, _f32]
        L.orr_maxpool_real.argtypes = [_f32, _f32, _ci, _ci, _ci]
        L.orr_up_cat.argtypes = [_f32, _ci, _ci, _ci, _f32, _ci, _ci, _ci, _f32]
        L.orr_head.argtypes = [_f32, _f32, _f32, _f32, _ci, _ci, _ci]

    def parse(self, data: bytes):
        h = C.c_void_p()
        err = C.create_string_buffer(256)
        if self.lib.orr_parse(data, len(data), C.byref(h), err, 256):
            raise ValueError(err.value.decode())
        return ReactOracleModel(self, h)

    # ---- kernels ([C,H,W] float / int arrays, batch 1) ----
    def proj(self, x, Wm):
        x = np.ascontiguousarray(x, np.float32)
        Wm = np.ascontiguousarray(Wm, np.float32)
        cin, H, W = x.shape
        out = np.zeros((Wm.shape[0], H, W), np.float32)
        self.lib.orr_proj(_p(x, _f32), _p(Wm, _f32), _p(out, _f32), cin, H * W, Wm.shape[0])
        return out

    def conv3(self, x, wsign, alpha):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(wsign, np.int8)
        al = np.ascontiguousarray(alpha, np.float32)
        cin, H, W = x.shape
        out = np.zeros((w.shape[0], H, W), np.float32)
        self.lib.orr_conv3(_p(x, _f32), _p(w, _i8), _p(al, _f32), _p(out, _f32), cin, H, W, w.shape[0])
        return out

    def epi(self, acc, res, A, B, move1, prelu_w):
        res = np.ascontiguousarray(res, np.float32)
        c = res.shape[0]
        out = np.zeros(res.shape, np.float32)
        prm = [_p(np.ascontiguousarray(v, np.float32), _f32) for v in (A, B, move1, prelu_w)]
        if np.asarray(acc).dtype.kind == "i":
            P = np.ascontiguousarray(acc, np.int32)
            self.lib.orr_epi_int(_p(P, _i32), _p(res, _f32), _p(out, _f32), c, res[0].size, *prm)
        else:
            x = np.ascontiguousarray(acc, np.float32)
            self.lib.orr_epi_real(_p(x, _f32), _p(res, _f32), _p(out, _f32), c, res[0].size, *prm)
        return out

    def epi_plain(self, acc, res, A, B, move1, prelu_w):
        """the react_epilogue_int / _real order (t = A*acc + B + res + move1)"""
        res = np.ascontiguousarray(res, np.float32)
        is_int = np.asarray(acc).dtype.kind == "i"
        a = np.ascontiguousarray(acc, np.int32 if is_int else np.float32)
        out = np.zeros(res.shape, np.float32)
        prm = [_p(np.ascontiguousarray(v, np.float32), _f32) for v in (A, B, move1, prelu_w)]
        self.lib.orr_epi_plain(a.ctypes.data, int(is_int), _p(res, _f32), _p(out, _f32), res.shape[0],
                               res[0].size, *prm)
        return out

    def tap(self, x, rsign):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(x.shape, np.int8)
        self.lib.orr_tap(_p(x, _f32), _p(out, _i8), x.shape[0], x[0].size,
                         _p(np.ascontiguousarray(rsign, np.float32), _f32))
        return out

    def maxpool_real(self, x):
        x = np.ascontiguousarray(x, np.float32)
        c, H, W = x.shape
        out = np.zeros((c, H // 2, W // 2), np.float32)
        self.lib.orr_maxpool_real(_p(x, _f32), _p(out, _f32), c, H, W)
        return out

    def up_cat(self, skip, x):
        s = np.ascontiguousarray(skip, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        sC, sH, sW = s.shape
        xC, hH, hW = x.shape
        out = np.zeros((sC + xC, sH, sW), np.float32)
        self.lib.orr_up_cat(_p(s, _f32), sC, sH, sW, _p(x, _f32), xC, hH, hW, _p(out, _f32))
        return out

    def head(self, a, Wm, bias):
        a = np.ascontiguousarray(a, np.float32)
        Wm = np.ascontiguousarray(Wm, np.float32)
        cin, H, W = a.shape
        out = np.zeros((Wm.shape[0], H, W), np.float32)
        self.lib.orr_head(_p(a, _f32), _p(Wm, _f32), _p(np.ascontiguousarray(bias, np.float32), _f32),
                          _p(out, _f32), cin, H * W, Wm.shape[0])
        return out


class ReactOracleModel:
    def __init__(self, orc: ReactOracle, handle):
        self.orc = orc
        self.h = handle

    def __del__(self):
        try:
            if self.h:
                self.orc.lib.orr_free(self.h)
                self.h = None
        except Exception:
            pass

    def _dims(self):
        hdr = (C.c_int * 5).from_address(self.h.value)
        return hdr[2], hdr[3]

    def forward(self, x: np.ndarray, stages: bool = False):
        """x [n_bands,H,W] -> logits [n_classes,H,W] (+ dict of every stage)."""
        x = np.ascontiguousarray(x, np.float32)
        _, H, W = x.shape
        logits = np.zeros((self._dims()[1], H, W), np.float32)
        got: Dict[str, np.ndarray] = {}

        def cb(_ctx, name, dtype, c, h, w, data):
            arr = np.ctypeslib.as_array(C.cast(data, C.POINTER(np.ctypeslib.as_ctypes_type(_DT[dtype]))),
                                        shape=(c * h * w,)).copy().reshape(c, h, w)
            got[name.decode()] = arr

        cbf = STAGE_CB(cb) if stages else STAGE_CB()
        if self.orc.lib.orr_forward(self.h, _p(x, _f32), H, W, _p(logits, _f32), cbf, None):
            raise ValueError("oracle forward rejected the model/shape")
        return (logits, got) if stages else logits

    def forward_batch(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        N, _, H, W = x.shape
        out = np.zeros((N, self._dims()[1], H, W), np.float32)
        if self.orc.lib.orr_forward_batch_par(self.h, _p(x, _f32), N, H, W, _p(out, _f32)):
            raise ValueError("oracle forward rejected the model/shape")
        return out

    def forward_patched(self, cube: np.ndarray, P: int) -> np.ndarray:
        cube = np.ascontiguousarray(cube, np.float32)
        _, H, W = cube.shape
        out = np.zeros((self._dims()[1], H, W), np.float32)
        if self.orc.lib.orr_forward_patched(self.h, _p(cube, _f32), H, W, _p(out, _f32), P):
            raise ValueError("oracle forward rejected the model/shape")
        return out


def react_ref_available() -> bool:
    return os.path.exists(REACT_REF_LIB)


class RefReact:
    """The reference's v3 engine and kernels built from its sources
    (oracle/_ref/libreactref.so).  bnn_load_react() exits the process on a
    malformed blob (csrc/bnn_model_react.c:36-38), so only well-formed blobs
    may be given to it."""

    def __init__(self, path: str = REACT_REF_LIB):
        L = self.lib = C.CDLL(path)
        L.bnn_load_react.argtypes = [C.c_char_p]
        L.bnn_load_react.restype = C.c_void_p
        L.bnn_free_react.argtypes = [C.c_void_p]
        L.bnn_forward_react.argtypes = [C.c_void_p, _f32, _ci, _ci, _f32]
        L.bnn_forward_react_patched.argtypes = [C.c_void_p, _f32, _ci, _ci, _f32, _ci]
        L.react_proj_blk.argtypes = [_f32, _f32, _f32, _ci, _ci, _ci, _ci]
        L.react_proj_1x1.argtypes = [_f32, _f32, _f32, _ci, _ci, _ci, _ci]
        L.react_conv3_blk.argtypes = [_f32, _i8, _f32, _f32, _ci, _ci, _ci, _ci]
        L.react_epilogue_int_i16.argtypes = [_i16, _f32, _f32, _ci, _ci, _ci, _f32, _f32, _f32, _f32]
        L.react_epilogue_int.argtypes = [_i32, _f32, _f32, _ci, _ci, _ci, _f32, _f32, _f32, _f32]
        L.react_epilogue_real.argtypes = [_f32, _f32, _f32, _ci, _ci, _ci, _f32, _f32, _f32, _f32]
        L.react_epilogue_real_v2.argtypes = [_f32, _f32, _f32, _ci, _ci, _ci, _f32, _f32, _f32, _f32]
        L.react_tap.argtypes = [_f32, _i8, _ci, _ci, _ci, _f32]
        L.maxpool_real_v2.argtypes = [_f32, _f32, _ci, _ci, _ci, _ci, _ci]
        L.maxpool_P_i16.argtypes = [_i16, _i16, _ci, _ci, _ci, _ci, _ci]
        L.head_1x1_v2.argtypes = [_f32, _f32, _f32, _f32, _ci, _ci, _ci, _ci]
        L.bconv_blk_b4p4_i16.argtypes = [_i8, _u64, _i16] + [_ci] * 8

    def load(self, path: str):
        """(handle, n_bands, n_classes); exits on a bad blob"""
        h = self.lib.bnn_load_react(path.encode())
        hdr = (C.c_int * 5).from_address(h)
        return h, hdr[2], hdr[3]

    def free(self, handle):
        self.lib.bnn_free_react(C.c_void_p(handle))

    def forward(self, handle, x: np.ndarray, n_classes: int) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        _, H, W = x.shape
        out = np.zeros((n_classes, H, W), np.float32)
        self.lib.bnn_forward_react(C.c_void_p(handle), _p(x, _f32), H, W, _p(out, _f32))
        return out

    def forward_patched(self, handle, cube: np.ndarray, n_classes: int, P: int) -> np.ndarray:
        cube = np.ascontiguousarray(cube, np.float32)
        _, H, W = cube.shape
        out = np.zeros((n_classes, H, W), np.float32)
        self.lib.bnn_forward_react_patched(C.c_void_p(handle), _p(cube, _f32), H, W, _p(out, _f32), P)
        return out

    def proj(self, x, Wm, blk: bool = True):
        x = np.ascontiguousarray(x, np.float32)
        Wm = np.ascontiguousarray(Wm, np.float32)
        cin, H, W = x.shape
        out = np.zeros((Wm.shape[0], H, W), np.float32)
        fn = self.lib.react_proj_blk if blk else self.lib.react_proj_1x1
        fn(_p(x, _f32), _p(Wm, _f32), _p(out, _f32), cin, H, W, Wm.shape[0])
        return out

    def conv3(self, x, wsign, alpha):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(wsign, np.int8)
        cin, H, W = x.shape
        out = np.zeros((w.shape[0], H, W), np.float32)
        self.lib.react_conv3_blk(_p(x, _f32), _p(w, _i8), _p(np.ascontiguousarray(alpha, np.float32), _f32),
                                 _p(out, _f32), cin, H, W, w.shape[0])
        return out

    def epi(self, acc, res, A, B, move1, prelu_w):
        res = np.ascontiguousarray(res, np.float32)
        c, H, W = res.shape
        out = np.zeros(res.shape, np.float32)
        prm = [_p(np.ascontiguousarray(v, np.float32), _f32) for v in (A, B, move1, prelu_w)]
        if np.asarray(acc).dtype.kind == "i":
            P = np.ascontiguousarray(acc, np.int16)
            self.lib.react_epilogue_int_i16(_p(P, _i16), _p(res, _f32), _p(out, _f32), c, H, W, *prm)
        else:
            x = np.ascontiguousarray(acc, np.float32)
            self.lib.react_epilogue_real_v2(_p(x, _f32), _p(res, _f32), _p(out, _f32), c, H, W, *prm)
        return out

    def epi_plain(self, acc, res, A, B, move1, prelu_w):
        res = np.ascontiguousarray(res, np.float32)
        c, H, W = res.shape
        out = np.zeros(res.shape, np.float32)
        prm = [_p(np.ascontiguousarray(v, np.float32), _f32) for v in (A, B, move1, prelu_w)]
        if np.asarray(acc).dtype.kind == "i":
            P = np.ascontiguousarray(acc, np.int32)
            self.lib.react_epilogue_int(_p(P, _i32), _p(res, _f32), _p(out, _f32), c, H, W, *prm)
        else:
            x = np.ascontiguousarray(acc, np.float32)
            self.lib.react_epilogue_real(_p(x, _f32), _p(res, _f32), _p(out, _f32), c, H, W, *prm)
        return out

    def tap(self, x, rsign):
        x = np.ascontiguousarray(x, np.float32)
        c, H, W = x.shape
        out = np.zeros(x.shape, np.int8)
        self.lib.react_tap(_p(x, _f32), _p(out, _i8), c, H, W, _p(np.ascontiguousarray(rsign, np.float32), _f32))
        return out

    def maxpool_real(self, x):
        x = np.ascontiguousarray(x, np.float32)
        c, H, W = x.shape
        out = np.zeros((c, H // 2, W // 2), np.float32)
        self.lib.maxpool_real_v2(_p(x, _f32), _p(out, _f32), c, H, W, 2, 2)
        return out

    def maxpool_P(self, P):
        P = np.ascontiguousarray(P, np.int16)
        c, H, W = P.shape
        out = np.zeros((c, H // 2, W // 2), np.int16)
        self.lib.maxpool_P_i16(_p(P, _i16), _p(out, _i16), c, H, W, 2, 2)
        return out

    def head(self, a, Wm, bias):
        a = np.ascontiguousarray(a, np.float32)
        Wm = np.ascontiguousarray(Wm, np.float32)
        cin, H, W = a.shape
        out = np.zeros((Wm.shape[0], H, W), np.float32)
        self.lib.head_1x1_v2(_p(a, _f32), _p(Wm, _f32), _p(np.ascontiguousarray(bias, np.float32), _f32),
                             _p(out, _f32), cin, H, W, Wm.shape[0])
        return out

    def bconv(self, a, bits, cout):
        a = np.ascontiguousarray(a, np.int8)
        bits = np.ascontiguousarray(bits, np.uint64)
        cin, H, W = a.shape
        P = np.zeros((cout, H, W), np.int16)
        self.lib.bconv_blk_b4p4_i16(_p(a, _i8), _p(bits, _u64), _p(P, _i16), cin, H, W, cout, 3, 3, 1, 1)
        return P
