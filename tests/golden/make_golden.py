"""Write the golden fixtures from the reference C built from its own sources.

    make -C oracle ref && python tests/golden/make_golden.py

Needs oracle/_ref/libbnnref.so and oracle/_ref/bnn_infer (the reference's
csrc/*.c compiled by oracle/Makefile); it never imports the reference's
Python.  For each case (a seeded synthetic blob, seeded input patches,
an H x W) it records:

  * SHA-256 of the blob and input bytes (pins the synthetic generator),
  * logits of every patch from the reference bnn_forward (stored in full),
  * SHA-256 of every intermediate stage, computed by chaining the reference
    kernels (bconv_dispatch, conv_realin_naive, apply_fold_*, maxpool_P,
    head_1x1) the way python/verify/forward_driver.py:205-262 chains them,
    with the nearest up + concat of csrc/bnn_model.c:130-148,
  * the output file of the reference CLI `bnn_infer blob rand out H W`,
  * the same for v2 (spectral-stem) blobs: logits from bnn_stem_forward,
    stage hashes of the chained kernels (stem 1x1 conv, real fold, then a
    binary enc1), and the output of `bnn_infer_stem`.

  * for v3 (ReActNet) blobs: logits from bnn_forward_react, stage hashes of
    the reference's v3 kernels (react_proj_blk, react_conv3_blk, react_tap,
    bconv_blk_b4p4_i16, react_epilogue_*, maxpool_P_i16, maxpool_real_v2,
    head_1x1_v2) chained as csrc/bnn_model_react.c:190-274, 395-438 chains
    them, and the output of `bnn_infer_react` on an input file, streamed and
    patch-wise.

Stage hashes are over the C-order bytes of [C,H,W] arrays: int8 for binary
activations, int32 for P, float32 for enc1.conv1 and logits (v3: float32
for every highway stage, int32 for P although the reference stores int16).
"""
from __future__ import annotations

import hashlib
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from bnns_to_c_amd import blob as B  # noqa: E402
from bnns_to_c_amd import synth  # noqa: E402
from bnns_to_c_amd import blob_react as R  # noqa: E402
from oracle.oracle import REACT_REF_CLI, REF_CLI, REF_CLI_STEM, RefC, RefReact  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

# (name, blob seed, base, coverage, input seed, N, H, W)
CASES = [
    ("base16_s0_32x32", 0, 16, False, 100, 2, 32, 32),
    ("base16_cov_s3_32x32", 3, 16, True, 101, 2, 32, 32),
    ("base8_s5_odd17x23", 5, 8, False, 102, 2, 17, 23),
    ("base16_s7_30x34", 7, 16, False, 103, 1, 30, 34),
    ("base32_s9_16x16", 9, 32, False, 104, 1, 16, 16),
]
CLI_CASES = [("base16_s0_32x32", 0, 16, False, 32, 32), ("base8_s5_odd17x23", 5, 8, False, 17, 23)]
# v2 (spectral stem): (name, blob seed, base, stem width, coverage, input seed, N, H, W);
# logits from the reference bnn_stem_forward (csrc/bnn_model_stem.c:168-255)
STEM_CASES = [
    ("stem16_base16_s1_32x32", 1, 16, 16, False, 110, 2, 32, 32),
    ("stem32_base8_cov_s2_odd17x23", 2, 8, 32, True, 111, 2, 17, 23),
    ("stem24_base16_s3_30x34", 3, 16, 24, False, 112, 1, 30, 34),
]
STEM_CLI_CASES = [("stem16_base16_s1_32x32", 1, 16, 16, False, 32, 32)]
# v3 (ReActNet): (name, blob seed, base, coverage, input seed, N, H, W)
REACT_CASES = [
    ("react16_s0_32x32", 0, 16, False, 120, 2, 32, 32),
    ("react8_cov_s1_odd17x23", 1, 8, True, 121, 2, 17, 23),
    ("react16_cov_s2_32x32", 2, 16, True, 122, 1, 32, 32),
    ("react32_s3_16x16", 3, 32, False, 123, 1, 16, 16),
]
# (name, blob seed, base, input seed, H, W, patch size or 0 for the whole image)
REACT_CLI_CASES = [("react8_s4_36x52_file", 4, 8, 124, 36, 52, 0),
                   ("react16_s5_40x56_patch16", 5, 16, 125, 40, 56, 16),
                   ("react8_s6_32x48_rand", 6, 8, -1, 32, 48, 0)]   # input seed -1: the CLI's "rand" cube


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def up_cat(skip: np.ndarray, x: np.ndarray) -> np.ndarray:
    """csrc/bnn_model.c:130-148: [skip ; nearest-2x(x) at the F.pad offset], 0 elsewhere."""
    sC, sH, sW = skip.shape
    xC, hH, hW = x.shape
    out = np.zeros((sC + xC, sH, sW), np.int8)
    out[:sC] = skip
    uH, uW = 2 * hH, 2 * hW
    oh, ow = max(sH - uH, 0) // 2, max(sW - uW, 0) // 2
    up = np.repeat(np.repeat(x, 2, axis=1), 2, axis=2)[:, :min(uH, sH), :min(uW, sW)]
    out[sC:, oh:oh + up.shape[1], ow:ow + up.shape[2]] = up
    return out


def ref_chain(ref: RefC, b: B.BlobV1, x: np.ndarray):
    """Every stage of one patch through the reference kernels."""
    st = {}

    def fold(P, a):
        return ref.fold_int(P, a.type, a.t, a.lo, a.hi)

    def conv_fold(conv, act, inp, name, aname):
        P = ref.bconv(inp, conv.packed, conv.cout)
        st[f"{name}.P"] = P
        o = fold(P, act)
        st[aname] = o
        return o

    if b.has_stem:
        sc, sa = b.stem_conv, b.stem_act
        r = ref.conv_real(x, sc.wsign, sc.alpha, pad=0)
        st["stem.conv"] = r
        h = ref.fold_real(r, sa.A, sa.B, sa.slope, sa.rsign)
        st["stem.act"] = h
    else:
        c1 = b.enc_conv1[0]
        r = ref.conv_real(x, c1.wsign, c1.alpha)
        st["enc1.conv1"] = r
        a = b.enc_act1[0]
        h = ref.fold_real(r, a.A, a.B, a.slope, a.rsign)
        st["enc1.act1"] = h
    skips = []
    for i in range(4):
        if i or b.has_stem:
            h = conv_fold(b.enc_conv1[i], b.enc_act1[i], h, f"enc{i + 1}.conv1", f"enc{i + 1}.act1")
        c2 = b.enc_conv2[i]
        P = ref.bconv(h, c2.packed, c2.cout)
        st[f"enc{i + 1}.conv2.P"] = P
        s = fold(P, b.enc_act2_skip[i])
        st[f"enc{i + 1}.act2_skip"] = s
        skips.append(s)
        Pd = ref.maxpool(P)
        st[f"enc{i + 1}.pool.P"] = Pd
        h = fold(Pd, b.enc_act2_down[i])
        st[f"enc{i + 1}.act2_down"] = h
    h = conv_fold(b.bott_conv1, b.bott_act1, h, "bott.conv1", "bott.act1")
    h = conv_fold(b.bott_conv2, b.bott_act2, h, "bott.conv2", "bott.act2")
    for j in range(4):
        k = 4 - j
        cat = up_cat(skips[3 - j], h)
        st[f"dec{k}.upcat"] = cat
        h = conv_fold(b.dec_conv1[j], b.dec_act1[j], cat, f"dec{k}.conv1", f"dec{k}.act1")
        h = conv_fold(b.dec_conv2[j], b.dec_act2[j], h, f"dec{k}.conv2", f"dec{k}.act2")
    logits = ref.head(h.astype(np.float32), b.head.W, b.head.bias)
    st["logits"] = logits
    return st


def up_cat_f(skip: np.ndarray, x: np.ndarray) -> np.ndarray:
    """csrc/bnn_model_react.c:280-298: the float concat, 0.0 where the up part is absent."""
    sC, sH, sW = skip.shape
    xC, hH, hW = x.shape
    out = np.zeros((sC + xC, sH, sW), np.float32)
    out[:sC] = skip
    uH, uW = 2 * hH, 2 * hW
    oh, ow = max(sH - uH, 0) // 2, max(sW - uW, 0) // 2
    up = np.repeat(np.repeat(x, 2, axis=1), 2, axis=2)[:, :min(uH, sH), :min(uW, sW)]
    out[sC:, oh:oh + up.shape[1], ow:ow + up.shape[2]] = up
    return out


def react_chain(ref: RefReact, b: R.BlobV3, x: np.ndarray):
    """Every stage of one v3 patch through the reference's v3 kernels."""
    st = {}

    def epi(acc, res, e):
        return ref.epi(acc, res, e.A, e.B, e.move1, e.prelu_w)

    def unit1(k, xin, nm):
        res = ref.proj(xin, k.proj1.W)
        st[f"{nm}.u1.proj"] = res
        a = ref.tap(xin, k.tap1.rsign)
        st[f"{nm}.u1.tap"] = a
        P = ref.bconv(a, k.conv1.packed, k.conv1.cout)
        st[f"{nm}.u1.P"] = P.astype(np.int32)
        h = epi(P, res, k.epi1)
        st[f"{nm}.h1"] = h
        return h

    def unit2_P(k, h1, nm):
        a = ref.tap(h1, k.tap2.rsign)
        st[f"{nm}.u2.tap"] = a
        P = ref.bconv(a, k.conv2.packed, k.conv2.cout)
        st[f"{nm}.u2.P"] = P.astype(np.int32)
        return P

    h = x
    skips = []
    for i, k in enumerate(b.enc):
        nm = f"enc{i + 1}"
        if k.input_real:
            res = ref.proj(h, k.proj1.W)
            st["enc1.u1.proj"] = res
            c = ref.conv3(h, k.conv1.wsign, k.conv1.alpha)
            st["enc1.u1.conv"] = c
            h1 = epi(c, res, k.epi1)
            st["enc1.h1"] = h1
        else:
            h1 = unit1(k, h, nm)
        P = unit2_P(k, h1, nm)
        sk = epi(P, h1, k.epi_a)
        st[f"{nm}.skip"] = sk
        skips.append(sk)
        Pd = ref.maxpool_P(P)
        st[f"{nm}.pool.P"] = Pd.astype(np.int32)
        hd = ref.maxpool_real(h1)
        st[f"{nm}.pool.h"] = hd
        h = epi(Pd, hd, k.epi_b)
        st[f"{nm}.down"] = h
    h1 = unit1(b.bott, h, "bott")
    h = epi(unit2_P(b.bott, h1, "bott"), h1, b.bott.epi_a)
    st["bott.h2"] = h
    for j, k in enumerate(b.dec):
        nm = f"dec{4 - j}"
        cat = up_cat_f(skips[3 - j], h)
        st[f"{nm}.cat"] = cat
        h1 = unit1(k, cat, nm)
        h = epi(unit2_P(k, h1, nm), h1, k.epi_a)
        st[f"{nm}.h2"] = h
    st["logits"] = ref.head(h, b.head.W, b.head.bias)
    return st


def main() -> None:
    ref = RefC()
    meta = {"generator": "tests/golden/make_golden.py",
            "reference_build": "oracle/Makefile `ref`: gcc -O3 -Wall -march=x86-64-v3 -fopenmp",
            "cases": {}, "cli": {}}
    arrays = {}
    with tempfile.TemporaryDirectory() as td:
        for name, seed, base, cov, iseed, N, H, W in CASES:
            b = synth.make_blob(seed=seed, base=base, coverage=cov)
            data = B.to_bytes(b)
            path = os.path.join(td, name + ".blob")
            open(path, "wb").write(data)
            x = synth.make_input(iseed, N, 120, H, W)
            h, _, ncls = ref.load(path)
            logits = np.stack([ref.forward(h, x[n], ncls) for n in range(N)])
            ref.free(h)
            stages = []
            for n in range(N):
                st = ref_chain(ref, b, x[n])
                assert np.array_equal(st["logits"].view(np.uint32), logits[n].view(np.uint32)), \
                    f"{name}: chained reference kernels differ from reference bnn_forward"
                stages.append({k: sha(v) for k, v in st.items()})
            meta["cases"][name] = {"blob_seed": seed, "base": base, "coverage": cov, "input_seed": iseed,
                                   "N": N, "H": H, "W": W, "blob_sha256": hashlib.sha256(data).hexdigest(),
                                   "input_sha256": sha(x), "stages": stages}
            arrays[f"{name}__logits"] = logits
        for name, seed, base, cov, H, W in CLI_CASES:
            b = synth.make_blob(seed=seed, base=base, coverage=cov)
            path = os.path.join(td, name + "_cli.blob")
            open(path, "wb").write(B.to_bytes(b))
            out = os.path.join(td, name + "_cli.bin")
            subprocess.run([REF_CLI, path, "rand", out, str(H), str(W)], check=True,
                           capture_output=True)
            o = np.fromfile(out, np.float32).reshape(-1, H, W)
            meta["cli"][name] = {"blob_seed": seed, "base": base, "coverage": cov, "H": H, "W": W,
                                 "sha256": sha(o)}
            arrays[f"{name}__cli"] = o
        meta["stem_cases"], meta["stem_cli"] = {}, {}
        for name, seed, base, stem, cov, iseed, N, H, W in STEM_CASES:
            b = synth.make_blob_v2(seed=seed, base=base, stem=stem, coverage=cov)
            data = B.to_bytes(b)
            path = os.path.join(td, name + ".blob")
            open(path, "wb").write(data)
            x = synth.make_input(iseed, N, 120, H, W)
            h, _, ncls = ref.stem_load(path)
            logits = np.stack([ref.stem_forward(h, x[n], ncls) for n in range(N)])
            ref.stem_free(h)
            stages = []
            for n in range(N):
                st = ref_chain(ref, b, x[n])
                assert np.array_equal(st["logits"].view(np.uint32), logits[n].view(np.uint32)), \
                    f"{name}: chained reference kernels differ from reference bnn_stem_forward"
                stages.append({k: sha(v) for k, v in st.items()})
            meta["stem_cases"][name] = {"blob_seed": seed, "base": base, "stem": stem, "coverage": cov,
                                        "input_seed": iseed, "N": N, "H": H, "W": W,
                                        "blob_sha256": hashlib.sha256(data).hexdigest(),
                                        "input_sha256": sha(x), "stages": stages}
            arrays[f"{name}__logits"] = logits
        for name, seed, base, stem, cov, H, W in STEM_CLI_CASES:
            b = synth.make_blob_v2(seed=seed, base=base, stem=stem, coverage=cov)
            path = os.path.join(td, name + "_cli.blob")
            open(path, "wb").write(B.to_bytes(b))
            out = os.path.join(td, name + "_cli.bin")
            subprocess.run([REF_CLI_STEM, path, "rand", out, str(H), str(W)], check=True,
                           capture_output=True)
            o = np.fromfile(out, np.float32).reshape(-1, H, W)
            meta["stem_cli"][name] = {"blob_seed": seed, "base": base, "stem": stem, "coverage": cov,
                                      "H": H, "W": W, "sha256": sha(o)}
            arrays[f"{name}__cli"] = o
        rref = RefReact()
        meta["react_cases"], meta["react_cli"] = {}, {}
        for name, seed, base, cov, iseed, N, H, W in REACT_CASES:
            b = synth.make_blob_react(seed=seed, base=base, coverage=cov)
            data = R.to_bytes(b)
            path = os.path.join(td, name + ".blob")
            open(path, "wb").write(data)
            x = synth.make_input(iseed, N, 120, H, W)
            h, _, ncls = rref.load(path)
            logits = np.stack([rref.forward(h, x[n], ncls) for n in range(N)])
            rref.free(h)
            stages = []
            for n in range(N):
                st = react_chain(rref, b, x[n])
                assert np.array_equal(st["logits"].view(np.uint32), logits[n].view(np.uint32)), \
                    f"{name}: chained reference kernels differ from reference bnn_forward_react"
                stages.append({k: sha(v) for k, v in st.items()})
            meta["react_cases"][name] = {"blob_seed": seed, "base": base, "coverage": cov, "input_seed": iseed,
                                         "N": N, "H": H, "W": W, "blob_sha256": hashlib.sha256(data).hexdigest(),
                                         "input_sha256": sha(x), "stages": stages}
            arrays[f"{name}__logits"] = logits
        for name, seed, base, iseed, H, W, P in REACT_CLI_CASES:
            b = synth.make_blob_react(seed=seed, base=base)
            path = os.path.join(td, name + "_cli.blob")
            open(path, "wb").write(R.to_bytes(b))
            xin = os.path.join(td, name + "_in.bin")
            if iseed >= 0:
                synth.make_input(iseed, 1, 120, H, W)[0].tofile(xin)
            else:
                xin = "rand"
            out = os.path.join(td, name + "_cli.bin")
            spec = f"patch{P}:{xin}" if P else xin
            subprocess.run([REACT_REF_CLI, path, spec, out, str(H), str(W)], check=True, capture_output=True)
            o = np.fromfile(out, np.float32).reshape(-1, H, W)
            meta["react_cli"][name] = {"blob_seed": seed, "base": base, "input_seed": iseed, "H": H, "W": W,
                                       "patch": P, "sha256": sha(o)}
            arrays[f"{name}__cli"] = o
    with open(os.path.join(OUT, "golden.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    np.savez_compressed(os.path.join(OUT, "golden_logits.npz"), **arrays)
    print("wrote", os.path.join(OUT, "golden.json"), "and golden_logits.npz")


if __name__ == "__main__":
    main()
