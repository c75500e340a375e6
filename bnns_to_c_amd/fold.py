"""weights.blob from trained parameters: the exporter's folding on numpy.

The reference builds a blob from a torch model of the training repo
(python/bnn2c/blob.py:159-245, python/bnn2c/export.py): every activation
chain after a conv (BatchNorm, RPReLU move1 bias, PReLU, RSign bias, sign)
is folded per output channel, into an integer rule on the XNOR accumulator
P where the conv input is binary, or into the real-fold parameters
A, B, slope, rsign where it is real (the first conv, or the v2 stem).  This
module does the same from plain arrays, so a blob can be written without
the training repo:

  chain_affine   forward_driver.py:100-112 (scale, shift, defaults)
  presign        derive_thresholds.py:104-117 (r as a function of P)
  derive_rule    derive_thresholds.py:131-155 (flips over achievable P)
  fold_act       forward_driver.py:113-140 (rule codes, real-fold arrays)
  conv records   blob.py:64-88 and export.py:52-67 (zero weights snapped)
  blob_from_params  blob.py:165-200 (v1) and blob.py:204-245 (v2)

Parameters come as a flat mapping of numpy arrays named after the model's
modules (see PARAMS below); `python -m bnns_to_c_amd.fold params.npz
out.blob` writes a blob from an .npz of them.
"""
from __future__ import annotations

import sys
from typing import Dict, Mapping, Optional, Tuple

import numpy as np

from . import blob as B

RULE_CODE = {"const": B.RULE_CONST, "ge": B.RULE_GE, "lt": B.RULE_LT,
             "band_in": B.RULE_BAND_IN, "band_out": B.RULE_BAND_OUT}

# exact-zero binary weights are set to this before export (export.py:52-67)
SNAP_EPS = 1e-6
BN_EPS = 1e-5

PARAMS = """
Parameter names (float32 arrays; C = the chain's channels):
  <conv>.weight            [Cout, Cin, kh, kw]  convs: enc1..4.conv1/conv2,
                           bottleneck.conv1/conv2, dec4..1.conv1/conv2, and
                           stem.conv for a v2 model; <conv>.padding and
                           <conv>.stride (int, default 1/1 for 3x3, 0/1 for
                           1x1) are optional
  <act>.bn.weight, .bn.bias, .bn.running_mean, .bn.running_var  [C]
  <act>.bn.eps             scalar, default 1e-5
  <act>.move1, <act>.prelu, <act>.rsign  [C], optional (0, 1, 0)
                           acts: enc1..4.act1/act2_skip/act2_down,
                           bottleneck.act1/act2, dec4..1.act1/act2, stem.act
  outc.weight [n_classes, Cin, 1, 1], outc.bias [n_classes] (optional)
"""


# ------------------------------------------------------------ the fold --
def chain_affine(p: Mapping[str, np.ndarray], act: str, c: int):
    """Per-channel float32 scale, shift, move1, slope, rsign of one chain
    (python/verify/forward_driver.py:100-112: scale = g / sqrt(v + eps),
    shift = b - scale * m; absent RPReLU / PReLU / RSign give 0 / 1 / 0)."""
    def arr(name, default):
        v = p.get(f"{act}.{name}")
        if v is None:
            return np.full(c, default, np.float32)
        v = np.asarray(v, np.float32).reshape(-1)
        if v.shape[0] != c:
            raise ValueError(f"{act}.{name}: {v.shape[0]} values for {c} channels")
        return v
    g = arr("bn.weight", 1.0)
    b = arr("bn.bias", 0.0)
    m = arr("bn.running_mean", 0.0)
    v = arr("bn.running_var", 1.0)
    eps = float(np.asarray(p.get(f"{act}.bn.eps", BN_EPS)))
    scale = g / np.sqrt(v + eps)
    shift = b - scale * m
    return scale, shift, arr("move1", 0.0), arr("prelu", 1.0), arr("rsign", 0.0)


def presign(P: np.ndarray, k: int, alpha, scale, shift, move1, slope, rsign) -> np.ndarray:
    """r(P) of channel k: x = alpha*P; z = scale*x + (shift + move1);
    z<0 -> slope*z; r = z + rsign (derive_thresholds.py:104-117), float64
    arithmetic on float32 parameters as there."""
    x = alpha[k] * np.asarray(P, np.float64)
    z = scale[k] * x + (shift[k] + move1[k])
    z = np.where(z >= 0.0, z, slope[k] * z)
    return z + rsign[k]


def derive_rule(k: int, N: int, alpha, scale, shift, move1, slope, rsign) -> Tuple[str, int, int, int]:
    """The rule of channel k as (kind, t, lo, hi): tabulate bit = r(P) > 0
    over every achievable P (-N..N step 2) and read the flips
    (derive_thresholds.py:131-155): none -> const (t = +1 / -1), one ->
    ge / lt at the first P of the new segment, two -> band_in / band_out."""
    Pv = np.arange(-N, N + 1, 2, dtype=np.int64)
    bits = presign(Pv.astype(np.float64), k, alpha, scale, shift, move1, slope, rsign) > 0.0
    flips = np.nonzero(bits[1:] != bits[:-1])[0]
    if len(flips) == 0:
        return "const", (1 if bits[0] else -1), 0, 0
    if len(flips) == 1:
        t = int(Pv[flips[0] + 1])
        return ("ge" if bits[flips[0] + 1] else "lt"), t, 0, 0
    if len(flips) == 2:
        lo, hi = int(Pv[flips[0] + 1]), int(Pv[flips[1] + 1])
        return ("band_in" if bits[flips[0] + 1] else "band_out"), 0, lo, hi
    raise ValueError(f"channel {k}: {len(flips)} sign changes over P; a blob rule holds at most 2")


def apply_rule(P: np.ndarray, kind: str, t: int, lo: int, hi: int) -> np.ndarray:
    """bool bits of a rule on integer P (derive_thresholds.py:158-173)."""
    P = np.asarray(P)
    if kind == "const":
        return np.full(P.shape, t > 0)
    if kind == "ge":
        return P >= t
    if kind == "lt":
        return P < t
    if kind == "band_in":
        return (P >= lo) & (P < hi)
    if kind == "band_out":
        return (P < lo) | (P >= hi)
    raise ValueError(kind)


def fold_act(p: Mapping[str, np.ndarray], act: str, c: int, alpha: np.ndarray, N: int, real: bool) -> B.Act:
    """One ACT record (forward_driver.py:113-140): the real fold keeps
    A = scale, B = shift + move1 (float32), slope, rsign; the integer fold
    stores one derived rule per channel."""
    scale, shift, move1, slope, rsign = chain_affine(p, act, c)
    if real:
        return B.Act(1, c, A=scale.astype(np.float32), B=(shift + move1).astype(np.float32),
                     slope=slope.astype(np.float32), rsign=rsign.astype(np.float32))
    ty = np.zeros(c, np.int32)
    tt = np.zeros(c, np.int32)
    lo = np.zeros(c, np.int32)
    hi = np.zeros(c, np.int32)
    for k in range(c):
        kind, t, l, h = derive_rule(k, N, alpha, scale, shift, move1, slope, rsign)
        ty[k], tt[k], lo[k], hi[k] = RULE_CODE[kind], t, l, h
    return B.Act(0, c, type=ty, t=tt, lo=lo, hi=hi)


# ----------------------------------------------------------------- convs --
def snapped(w: np.ndarray) -> np.ndarray:
    """Exact-zero weights set to +1e-6 (export.py:52-67: XNOR cannot hold 0)."""
    w = np.array(w, np.float32, copy=True)
    w[w == 0] = np.float32(SNAP_EPS)
    return w


def conv_alpha(w: np.ndarray) -> np.ndarray:
    """mean |w| per output channel as the exporter takes it from the module
    (derive_thresholds.py:79-83, a torch float32 mean); numpy's float32 mean
    where torch is absent."""
    try:
        import torch
        return torch.from_numpy(np.ascontiguousarray(w, np.float32)).abs().mean(dim=(1, 2, 3)).numpy()
    except ImportError:
        return np.abs(w).mean(axis=(1, 2, 3), dtype=np.float32)


def _geom(p, name, k):
    pad = int(np.asarray(p.get(f"{name}.padding", 1 if k == 3 else 0)))
    stride = int(np.asarray(p.get(f"{name}.stride", 1)))
    return pad, stride


def conv_bin(p: Mapping[str, np.ndarray], name: str) -> Tuple[B.Conv, np.ndarray]:
    """Binary CONV record: signs w >= 0 -> +1 packed in kidx order
    (blob.py:64-77), and the alpha the rule derivation uses."""
    w = snapped(p[f"{name}.weight"])
    cout, cin, kh, kw = w.shape
    pad, stride = _geom(p, name, kh)
    wsign = np.where(w >= 0, 1, -1).astype(np.int8)
    return B.Conv(B.TAG_CONV_BIN, cout, cin, kh, kw, pad, stride, packed=B.pack_kidx(wsign)), conv_alpha(w)


def conv_real(p: Mapping[str, np.ndarray], name: str) -> B.Conv:
    """Real-input CONV record: sign(w) and alpha = mean |w| (blob.py:80-88)."""
    w = snapped(p[f"{name}.weight"])
    cout, cin, kh, kw = w.shape
    pad, stride = _geom(p, name, kh)
    return B.Conv(B.TAG_CONV_REAL, cout, cin, kh, kw, pad, stride, wsign=np.sign(w).astype(np.int8),
                  alpha=np.abs(w).mean(axis=(1, 2, 3)).astype(np.float32))


# ------------------------------------------------------------------ blob --
def blob_from_params(p: Mapping[str, np.ndarray], n_bands: Optional[int] = None) -> B.BlobV1:
    """The v1 blob (blob.py:165-200), or v2 when stem.conv.weight is given
    (blob.py:204-245: real stem and its real fold, then a binary enc1)."""
    stem = "stem.conv.weight" in p
    first = "stem.conv" if stem else "enc1.conv1"
    nb = int(np.asarray(p[f"{first}.weight"]).shape[1]) if n_bands is None else n_bands
    W = np.asarray(p["outc.weight"], np.float32)
    ncls, hcin = W.shape[0], W.shape[1]
    b = B.BlobV1(base_channels=int(np.asarray(p["enc1.conv1.weight"]).shape[0]), n_bands=nb, n_classes=ncls,
                 version=B.VERSION_STEM if stem else B.VERSION)

    def bin_with(conv, acts):
        c, alpha = conv_bin(p, conv)
        N = c.cin * c.kh * c.kw
        return c, [fold_act(p, a, c.cout, alpha, N, real=False) for a in acts]

    if stem:
        sc = conv_real(p, "stem.conv")
        b.stem_conv = sc
        b.stem_act = fold_act(p, "stem.act", sc.cout, sc.alpha, 0, real=True)
    for i, st in enumerate(B.ENC):
        if i == 0 and not stem:
            c1 = conv_real(p, f"{st}.conv1")
            a1 = fold_act(p, f"{st}.act1", c1.cout, c1.alpha, 0, real=True)
        else:
            c1, (a1,) = bin_with(f"{st}.conv1", [f"{st}.act1"])
        c2, (sk, dn) = bin_with(f"{st}.conv2", [f"{st}.act2_skip", f"{st}.act2_down"])
        b.enc_conv1.append(c1); b.enc_act1.append(a1)
        b.enc_conv2.append(c2); b.enc_act2_skip.append(sk); b.enc_act2_down.append(dn)
    b.bott_conv1, (b.bott_act1,) = bin_with("bottleneck.conv1", ["bottleneck.act1"])
    b.bott_conv2, (b.bott_act2,) = bin_with("bottleneck.conv2", ["bottleneck.act2"])
    for st in B.DEC:
        c1, (a1,) = bin_with(f"{st}.conv1", [f"{st}.act1"])
        c2, (a2,) = bin_with(f"{st}.conv2", [f"{st}.act2"])
        b.dec_conv1.append(c1); b.dec_act1.append(a1)
        b.dec_conv2.append(c2); b.dec_act2.append(a2)
    bias = p.get("outc.bias")
    b.head = B.Head(ncls, hcin, W[:, :, 0, 0].copy() if W.ndim == 4 else W.copy(),
                    np.zeros(ncls, np.float32) if bias is None else np.asarray(bias, np.float32).copy())
    return b


def main(argv) -> int:
    if len(argv) != 3:
        print(f"usage: python -m bnns_to_c_amd.fold params.npz out.blob\n{PARAMS}", file=sys.stderr)
        return 2
    with np.load(argv[1], allow_pickle=False) as z:
        p: Dict[str, np.ndarray] = {k: z[k] for k in z.files}
    b = blob_from_params(p)
    B.write(b, argv[2])
    print(f"wrote {argv[2]} (v{b.version}, base {b.base_channels}, {b.n_bands} bands, "
          f"{b.n_classes} classes)")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
