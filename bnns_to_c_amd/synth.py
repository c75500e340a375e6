"""Seeded synthetic blobs and inputs for the v1 Bi-Real UNet.

The topology is the dual-skip UNet the v1 engine assembles
(csrc/bnn_model.c:150-253; widths as in csrc/bench_bconv.c:57-67 and
python/bnn2c/blob_react.py:52-58): with base width c,

    enc1 conv1 n_bands->c (real input), conv2 c->c
    enc2 c->2c, 2c->2c      enc3 2c->4c, 4c->4c      enc4 4c->8c, 8c->8c
    bott 8c->16c, 16c->16c
    dec4 (8c+16c)->8c, 8c->8c   dec3 (4c+8c)->4c, 4c->4c
    dec2 (2c+4c)->2c, 2c->2c    dec1 (c+2c)->c, c->c
    head c->n_classes (fp32 1x1)

Random parameters follow the benchmark recipe: binary weights are
Bernoulli(0.5) sign bits; each integer fold is a per-channel threshold
t ~ U[-fan_in/4, fan_in/4] with a Bernoulli(0.5) ge/lt flag; head weights
~ N(0, 0.05).  Choices the recipe leaves open, fixed here and recorded with
every fixture: real first-conv weights w ~ N(0, 1/sqrt(fan_in)) giving
wsign = sign(w) (0 -> +1) and alpha = mean|w|; real fold A ~ U(0.5, 1.5),
B ~ N(0, 0.1), slope ~ U(-0.5, 0.5), rsign ~ N(0, 0.1); head bias ~ N(0, 0.05).

`make_blob_v2` builds the spectral-stem variant (blob version 2).

`coverage=True` draws every integer rule type (const, ge, lt, band_in,
band_out and an unknown code, which the C fold maps to -1;
csrc/bnn_fold.c:49-56) so the fold paths the recipe never reaches are
exercised.
"""
from __future__ import annotations

import numpy as np

from . import blob as B


def topology(base: int, n_bands: int):
    """[(name, cin, cout)] for the 18 convs in blob order."""
    c = base
    enc = [(n_bands, c), (c, 2 * c), (2 * c, 4 * c), (4 * c, 8 * c)]
    convs = []
    for i, (ci, co) in enumerate(enc):
        convs.append((f"enc{i + 1}.conv1", ci, co))
        convs.append((f"enc{i + 1}.conv2", co, co))
    convs.append(("bott.conv1", 8 * c, 16 * c))
    convs.append(("bott.conv2", 16 * c, 16 * c))
    skips = [8 * c, 4 * c, 2 * c, c]         # dec4..dec1 skip widths
    up = 16 * c
    for j, s in enumerate(skips):
        convs.append((f"dec{4 - j}.conv1", s + up, s))
        convs.append((f"dec{4 - j}.conv2", s, s))
        up = s
    return convs


def _bin_conv(rng, cin, cout):
    wsign = np.where(rng.random((cout, cin, 3, 3)) < 0.5, -1, 1).astype(np.int8)
    return B.Conv(B.TAG_CONV_BIN, cout, cin, 3, 3, 1, 1, packed=B.pack_kidx(wsign))


def _real_conv(rng, cin, cout, k=3):
    fan_in = cin * k * k
    w = rng.normal(0.0, 1.0 / np.sqrt(fan_in), (cout, cin, k, k)).astype(np.float32)
    wsign = np.where(w >= 0, 1, -1).astype(np.int8)
    alpha = np.abs(w).mean(axis=(1, 2, 3)).astype(np.float32)
    pad = 1 if k == 3 else 0
    return B.Conv(B.TAG_CONV_REAL, cout, cin, k, k, pad, 1, wsign=wsign, alpha=alpha)


def _int_act(rng, c, fan_in, coverage):
    q = fan_in // 4
    t = rng.integers(-q, q + 1, size=c).astype(np.int32)
    ge = rng.random(c) < 0.5
    ty = np.where(ge, B.RULE_GE, B.RULE_LT).astype(np.int32)
    lo = np.zeros(c, np.int32)
    hi = np.zeros(c, np.int32)
    if coverage:
        # mix every rule code, including an unknown one (5)
        ty = rng.integers(0, 6, size=c).astype(np.int32)
        s = max(1, int(np.sqrt(fan_in)))
        centre = rng.integers(-s, s + 1, size=c)
        width = rng.integers(0, 2 * s + 1, size=c)
        lo = (centre - width // 2).astype(np.int32)
        hi = (lo + width).astype(np.int32)
        swap = rng.random(c) < 0.1           # occasionally lo >= hi
        lo[swap], hi[swap] = hi[swap] + 1, lo[swap]
        const = ty == B.RULE_CONST
        t[const] = np.where(rng.random(int(const.sum())) < 0.5, 1, -1)
    return B.Act(0, c, type=ty, t=t, lo=lo, hi=hi)


def _real_act(rng, c):
    A = rng.uniform(0.5, 1.5, c).astype(np.float32)
    Bv = rng.normal(0.0, 0.1, c).astype(np.float32)
    slope = rng.uniform(-0.5, 0.5, c).astype(np.float32)
    rsign = rng.normal(0.0, 0.1, c).astype(np.float32)
    return B.Act(1, c, A=A, B=Bv, slope=slope, rsign=rsign)


def make_blob(seed: int = 0, base: int = 16, n_bands: int = 120,
              n_classes: int = 3, coverage: bool = False) -> B.BlobV1:
    rng = np.random.default_rng(seed)
    topo = dict((n, (ci, co)) for n, ci, co in topology(base, n_bands))
    b = B.BlobV1(base_channels=base, n_bands=n_bands, n_classes=n_classes)
    for i in range(4):
        ci, co = topo[f"enc{i + 1}.conv1"]
        if i == 0:
            b.enc_conv1.append(_real_conv(rng, ci, co))
            b.enc_act1.append(_real_act(rng, co))
        else:
            b.enc_conv1.append(_bin_conv(rng, ci, co))
            b.enc_act1.append(_int_act(rng, co, ci * 9, coverage))
        ci2, co2 = topo[f"enc{i + 1}.conv2"]
        b.enc_conv2.append(_bin_conv(rng, ci2, co2))
        b.enc_act2_skip.append(_int_act(rng, co2, ci2 * 9, coverage))
        b.enc_act2_down.append(_int_act(rng, co2, ci2 * 9, coverage))
    for k in ("conv1", "conv2"):
        ci, co = topo[f"bott.{k}"]
        setattr(b, f"bott_{k}", _bin_conv(rng, ci, co))
        setattr(b, f"bott_act{k[-1]}", _int_act(rng, co, ci * 9, coverage))
    for j in range(4):
        st = f"dec{4 - j}"
        ci, co = topo[f"{st}.conv1"]
        b.dec_conv1.append(_bin_conv(rng, ci, co))
        b.dec_act1.append(_int_act(rng, co, ci * 9, coverage))
        ci, co = topo[f"{st}.conv2"]
        b.dec_conv2.append(_bin_conv(rng, ci, co))
        b.dec_act2.append(_int_act(rng, co, ci * 9, coverage))
    W = rng.normal(0.0, 0.05, (n_classes, base)).astype(np.float32)
    bias = rng.normal(0.0, 0.05, n_classes).astype(np.float32)
    b.head = B.Head(n_classes, base, W, bias)
    return b


def make_blob_v2(seed: int = 0, base: int = 16, n_bands: int = 120, n_classes: int = 3,
                 stem: int = 16, coverage: bool = False) -> B.BlobV1:
    """A v2 (spectral-stem) blob: a real-input 1x1 binary-weight stem
    n_bands -> stem with a real fold, then the v1 body with enc1.conv1 binary
    (stem -> base) and an integer enc1.act1 (csrc/bnn_model_stem.c:4-9).
    The stem follows the real first conv's recipe with fan_in = n_bands."""
    rng = np.random.default_rng(seed)
    b = make_blob(seed=seed + 7919, base=base, n_bands=n_bands, n_classes=n_classes, coverage=coverage)
    b.version = B.VERSION_STEM
    b.stem_conv = _real_conv(rng, n_bands, stem, k=1)
    b.stem_act = _real_act(rng, stem)
    b.enc_conv1[0] = _bin_conv(rng, stem, base)
    b.enc_act1[0] = _int_act(rng, base, stem * 9, coverage)
    return b


def make_blob_react(seed: int = 0, base: int = 16, n_bands: int = 120, n_classes: int = 3,
                    coverage: bool = False):
    """A v3 (ReActNet real-highway) blob (python/bnn2c/blob_react.py:8-41).
    Recipe (recorded with every fixture): binary weights Bernoulli(0.5);
    enc1.conv1 as the v1 real first conv; proj W ~ N(0, 1/sqrt(Cin)); int
    epilogues A ~ U(0.5, 1.5)/sqrt(Cin*9) (alpha and the BN scale folded),
    real epilogue A ~ U(0.5, 1.5); B ~ N(0, 0.3), move1 ~ N(0, 0.1),
    prelu_w ~ U(-0.25, 0.5); taps rsign ~ N(0, 0.3); head W ~ N(0, 0.1),
    bias ~ N(0, 0.05).  coverage=True also sets exact zeros: prelu_w = 0
    (negative t gives -0), A = 0, rsign = 0 and B = -move1 on some channels."""
    from . import blob_react as R
    rng = np.random.default_rng(seed)

    def epi(kind, c, cin):
        A = rng.uniform(0.5, 1.5, c).astype(np.float32)
        if kind == R.EPI_INT:
            A = (A / np.float32(np.sqrt(cin * 9))).astype(np.float32)
        Bv = rng.normal(0, 0.3, c).astype(np.float32)
        m = rng.normal(0, 0.1, c).astype(np.float32)
        w = rng.uniform(-0.25, 0.5, c).astype(np.float32)
        if coverage:
            w[rng.random(c) < 0.2] = 0.0
            A[rng.random(c) < 0.1] = 0.0
            z = rng.random(c) < 0.1
            Bv[z] = -m[z]
        return R.Epi(kind, c, A, Bv, m, w)

    def tap(c):
        r = rng.normal(0, 0.3, c).astype(np.float32)
        if coverage:
            r[rng.random(c) < 0.2] = 0.0
        return R.Tap(c, r)

    b = R.BlobV3(base, n_bands, n_classes)
    for name, ci, co, kind in R.arch(base):
        if name == "enc1":
            ci = n_bands
        real = name == "enc1"
        conv1 = _real_conv(rng, ci, co) if real else _bin_conv(rng, ci, co)
        W = rng.normal(0, 1 / np.sqrt(ci), (co, ci)).astype(np.float32)
        blk = R.Block(kind == "down", real, None if real else tap(ci), conv1, R.Proj(co, ci, W),
                      epi(R.EPI_REAL if real else R.EPI_INT, co, ci), tap(co), _bin_conv(rng, co, co),
                      epi(R.EPI_INT, co, co), epi(R.EPI_INT, co, co) if kind == "down" else None)
        if name.startswith("enc"):
            b.enc.append(blk)
        elif name == "bottleneck":
            b.bott = blk
        else:
            b.dec.append(blk)
    W = rng.normal(0.0, 0.1, (n_classes, base)).astype(np.float32)
    bias = rng.normal(0.0, 0.05, n_classes).astype(np.float32)
    b.head = B.Head(n_classes, base, W, bias)
    return b


def make_input(seed: int, n: int, n_bands: int = 120, h: int = 32, w: int = 32) -> np.ndarray:
    """x ~ N(0,1) float32 [n, n_bands, h, w] ([band,row,col] per patch)."""
    rng = np.random.default_rng(seed)
    return rng.standard_normal((n, n_bands, h, w), dtype=np.float32)


def react_rand_cube(n_bands: int, h: int, w: int) -> np.ndarray:
    """The v3 CLI's "rand" cube [n_bands, h, w]: xorshift64 (13, 7, 17) from
    88172645463325252, two uniforms ((s >> 11) + 0.5) / 2^53 per value and
    Box-Muller sqrt(-2 ln u0) cos(2 pi u1) in double, rounded to float
    (csrc/main_react.c:28-40).  Python's math module calls the same libm."""
    import math
    n = n_bands * h * w
    out = np.empty(n, np.float32)
    s = 88172645463325252
    m64 = (1 << 64) - 1
    for i in range(n):
        u = []
        for _ in range(2):
            s ^= (s << 13) & m64
            s ^= s >> 7
            s ^= (s << 17) & m64
            u.append(((s >> 11) + 0.5) / 9007199254740992.0)
        out[i] = math.sqrt(-2.0 * math.log(u[0])) * math.cos(6.283185307179586 * u[1])
    return out.reshape(n_bands, h, w)


# ------------------------------------------------- isolated-kernel configs --
def make_bits(seed: int, n: int, h: int, w: int, c: int) -> np.ndarray:
    """Bernoulli(0.5) +-1 activations int8 [n, c, h, w]."""
    rng = np.random.default_rng(seed)
    return np.where(rng.random((n, c, h, w)) < 0.5, -1, 1).astype(np.int8)


def make_signs(seed: int, cout: int, cin: int, k: int = 3) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return np.where(rng.random((cout, cin, k, k)) < 0.5, -1, 1).astype(np.int8)


def make_rules(seed: int, c: int, fan_in: int, coverage: bool = True):
    """Per-channel integer rules (type, t, lo, hi) as drawn for a blob."""
    a = _int_act(np.random.default_rng(seed), c, fan_in, coverage)
    return a.type, a.t, a.lo, a.hi


def make_thresholds(seed: int, c: int, bound: int):
    """cfg2 fold: t ~ U[-bound, bound], Bernoulli(0.5) ge/lt direction."""
    rng = np.random.default_rng(seed)
    t = rng.integers(-bound, bound + 1, size=c).astype(np.int32)
    ty = np.where(rng.random(c) < 0.5, B.RULE_GE, B.RULE_LT).astype(np.int32)
    z = np.zeros(c, np.int32)
    return ty, t, z, z.copy()


# ------------------------------------------- trained-parameter generator --
def make_params(seed: int = 0, base: int = 8, n_bands: int = 120, n_classes: int = 3,
                stem: int = 0) -> dict:
    """Float parameters in the layout bnns_to_c_amd.fold reads: N(0,1)
    conv weights (a few exact zeros), and per chain a BatchNorm, RPReLU
    move1, PReLU slope and RSign bias drawn so that every rule kind occurs:
    some negative gammas (lt), negative slopes (bands), offsets large
    enough for constants.  stem > 0 adds a v2 stem of that many channels."""
    rng = np.random.default_rng(seed)
    p = {}

    def conv(name, cin, cout, k=3):
        w = rng.standard_normal((cout, cin, k, k)).astype(np.float32)
        w.reshape(-1)[rng.choice(w.size, max(1, w.size // 500), replace=False)] = 0.0
        p[f"{name}.weight"] = w
        return float(np.abs(w).mean()) * np.sqrt(cin * k * k)   # typical |alpha * P|

    def act(name, c, spread):
        g = rng.uniform(0.5, 1.5, c).astype(np.float32)
        g[rng.random(c) < 0.2] *= -1
        p[f"{name}.bn.weight"] = g
        p[f"{name}.bn.bias"] = rng.normal(0, 0.3, c).astype(np.float32)
        m = rng.normal(0, 0.5 * spread, c).astype(np.float32)
        m[rng.random(c) < 0.05] = np.float32(5 * spread)            # saturates: a constant
        p[f"{name}.bn.running_mean"] = m
        p[f"{name}.bn.running_var"] = rng.uniform(0.5, 2.0, c).astype(np.float32) * np.float32(spread * spread)
        p[f"{name}.move1"] = rng.normal(0, 0.1, c).astype(np.float32)
        p[f"{name}.prelu"] = rng.uniform(-0.6, 1.0, c).astype(np.float32)
        p[f"{name}.rsign"] = rng.normal(0, 0.3, c).astype(np.float32)

    if stem:
        s = conv("stem.conv", n_bands, stem, k=1)
        act("stem.act", stem, s)
    acts = {"conv1": ["act1"], "conv2": ["act2"]}
    for name, ci, co in topology(base, n_bands):
        st, cv = name.split(".")
        st = "bottleneck" if st == "bott" else st
        if name == "enc1.conv1" and stem:
            ci = stem
        s = conv(f"{st}.{cv}", ci, co)
        names = ["act2_skip", "act2_down"] if st.startswith("enc") and cv == "conv2" else acts[cv]
        for a in names:
            act(f"{st}.{a}", co, s)
    p["outc.weight"] = rng.normal(0, 0.05, (n_classes, base, 1, 1)).astype(np.float32)
    p["outc.bias"] = rng.normal(0, 0.05, n_classes).astype(np.float32)
    return p
