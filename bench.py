"""Benchmark: full v1 Bi-Real binary UNet forward, 32x32x120 patches, batch 1024.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch 1024] [--no-cpu]
                    [--headline-only | --cfg4-only]

One step = one batched forward of `--batch` synthetic patches (seeded blob at
base 16, x ~ N(0,1)) with the input already resident in HBM; K steps are
timed back to back between device synchronisations and one pair of
timing-only HIP events (no cache fence of their own); a second pass with an
event between consecutive steps gives the spread of single steps.  The
GPU's clocks ramp under sustained load over about 25 ms (per-step time
falls from ~0.58 to ~0.50 ms over the first ~40 forwards, then holds), so
every measurement first runs its workload untimed, back to back
with its warmup and timed runs: --settle forwards (default 120, reported as
settle_steps) before the headline's W warmup and K timed steps, about 40 ms
before each other configuration.  Prints ONE JSON line on stdout:

  value         patches/s: N / ms_per_step, the mean of the K back-to-back
                steps (wall_ms_per_step: the host clock over the same
                steps; evented_step_ms: median, min and max of single steps
                from the second pass)
  with_copies   the same batch from and to pinned host memory, the PCIe
                copies in and out included
  cpu_configs   configs 1-4 on the reference's own code on this host:
                its kernels (cfg1, cfg2), its CLI per patch (cfg3 from the
                config-0 number, cfg4 on one 256x256 patch), with speed-ups
  roofline      the dominant kernel, enc1.conv1.  By default the certified
                first conv (fp16 matrix-core digit sums with a rigorous
                error bound, reference-order recompute of the outputs the
                bound leaves open): its algorithmic bytes (the input once,
                the output bits once) / its median hipEvent-measured
                duration against the 8 TB/s HBM peak, the binding floor of
                that formulation (its matrix-core work takes about half as
                long at the fp16 peak); the FP32 FMA work of the same conv
                per second is reported beside it as fp32_equivalent.  With
                BNN_CERT=0 the order-exact kernel runs instead, and the
                roofline is its FP32 FMA work against the dense FP32 matrix
                peak
  first_conv_exact  the order-exact first conv (a model loaded with
                BNN_CERT=0): its time and FP32 rate against the matrix peak
  bconv         the 17 binary convs: binary-op/s (2 per bit-MAC, border taps
                counted) against the VALU-popcount roofline
  cfg1          benchmark config 1: the isolated binary conv 64->64 at
                64x64, batch 256, int32 P out: binary-op/s against the
                VALU-popcount roofline and the HBM rate of its bytes
  fused_pool    the isolated fused bconv+fold+maxpool kernel at 128->128,
                32x32, batch 1024 (the benchmark's fused-kernel config):
                the kernel the default rule takes (the int8 matrix cores)
                against the int8 peak, and the bit-packed popcount kernel
                (BNN_BCONV_MFMA=0) against the VALU-popcount peak
  cfg4          benchmark config 4: 256x256x120 patches, batch 64, base 32;
                per-kernel times, the int8 matrix-core convs against the
                dense int8 peak
  scene         benchmark config 3: a 956x684x120 scene by 32x32 patches,
                device-resident and from host memory (PCIe included)
  v2_stem       the v2 spectral-stem model (16-channel 1x1 stem, then the
                binary body) at the same batch: patches/s, and its stem
                kernel's HBM rate against the 8 TB/s peak
  v3_react      the v3 ReActNet real-highway model at the same batch:
                patches/s, per-kernel times, and the enc1 conv + projection
                kernel's FP32 rate against the matrix peak
  cpu_baseline  the reference C CLI (oracle/_ref/bnn_infer, built from the
                reference sources) timed on this host: median of reps of one
                patch, like csrc/main.c:55-61; falls back to the checker
                (kind "port") where the reference build is absent
"""
from __future__ import annotations

import argparse
import json
import os
import re
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# MI355X published peaks
PEAK_FP32_FLOPS = 157.3e12          # dense FP32 matrix (MFMA); also the packed-vector figure
PEAK_HBM = 8.0e12
PEAK_INT8_MACS = 2.5e15             # dense int8 matrix: 5.0 POP/s = 2.5e15 MAC/s


def valu_binop_peak() -> float:
    # 256 CU x 64 lanes x 2.4 GHz 32-bit lane-ops; v_bitop3 + v_bcnt per 32
    # bit-MACs = 16 bit-MACs per lane-op = 32 binary ops per lane-op
    return 256 * 64 * 2.4e9 * 16 * 2


def settle(fn, torch, target_s: float = 0.04) -> None:
    """Run fn (which enqueues GPU work) untimed until about target_s seconds
    of it have run back to back: the GPU clocks ramp under sustained load
    over about 25 ms, so each measurement starts at the steady clock."""
    t0 = time.perf_counter()
    fn()
    torch.cuda.synchronize()
    one = max(time.perf_counter() - t0, 1e-5)
    for _ in range(min(2000, int(target_s / one) + 1)):
        fn()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def measured_traffic():
    """HBM bytes per launch of the real first conv from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (calibrated there against a
    device copy of known size), or None if the summary is absent."""
    p = os.path.join(ROOT, "profiles", "unet_b1024_hbm_traffic.md")
    try:
        txt = open(p).read()
    except OSError:
        return None
    m = re.search(r"`k_real_[^`]*`[^\n]*?moves ([\d.]+) MB in and ([\d.]+) MB out", txt)
    return round((float(m.group(1)) + float(m.group(2))) * 1e6) if m else None


def cpu_baseline(blob_path: str, budget_s: float) -> dict:
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    from oracle.oracle import REF_CLI
    env = dict(os.environ, OMP_NUM_THREADS=str(cores))
    if os.path.exists(REF_CLI):
        # calibrate with a short run, then size the sample to the budget
        def run(reps):
            with tempfile.TemporaryDirectory() as td:
                r = subprocess.run([REF_CLI, blob_path, "rand", os.path.join(td, "o.bin"), "32", "32", str(reps)],
                                   capture_output=True, text=True, env=env, timeout=600)
            if r.returncode != 0:
                raise RuntimeError(r.stderr)
            m = re.search(r"# forward\s*:\s*([\d.]+) ms", r.stderr)
            return float(m.group(1))
        t1 = run(3)
        reps = max(5, min(2000, int(budget_s * 1000.0 / max(t1, 1e-3))))
        med = run(reps)
        return {"value": round(1000.0 / med, 2), "unit": "patches/s", "cores": cores, "kind": "reference",
                "sample": f"reference bnn_infer (csrc/main.c) built from its sources, one 32x32x120 patch, "
                          f"median of {reps} reps = {med:.3f} ms/patch, OMP_NUM_THREADS={cores}"}
    import numpy as np
    from bnns_to_c_amd import synth
    from oracle.oracle import Oracle
    model = Oracle().parse(open(blob_path, "rb").read())
    x = synth.make_input(7, 1)
    t0 = time.perf_counter()
    model.forward_batch(x, parallel=False)
    t1 = time.perf_counter() - t0
    n = max(4, min(4096, int(budget_s / max(t1, 1e-4))))
    x = synth.make_input(7, n)
    t0 = time.perf_counter()
    model.forward_batch(x, parallel=False)
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 2), "unit": "patches/s", "cores": cores, "kind": "port",
            "sample": f"CPU restatement (oracle/), {n} patches of 32x32x120 in sequence, "
                      f"OMP_NUM_THREADS={cores}"}


def _median_time(fn, budget_s: float, max_reps: int = 50):
    """fn() run repeatedly for about budget_s seconds (at least 3 times):
    the median wall time in seconds and the number of runs."""
    ts = []
    t_end = time.perf_counter() + budget_s
    while len(ts) < 3 or (time.perf_counter() < t_end and len(ts) < max_reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    import numpy as np
    return float(np.median(ts)), len(ts)


def cpu_layer_baselines(budget_s: float):
    """Benchmark configs 1 and 2 on the reference's own kernels
    (oracle/_ref/libbnnref.so, built from its sources): one patch per call,
    as the reference runs them (batch 1), median over repeated calls;
    None where that build is absent.
      cfg1: bconv_dispatch, 64 -> 64 at 64x64 (csrc/bnn_conv.c:216-223)
      cfg2: bconv_dispatch 128 -> 128 at 32x32, apply_fold_int (skip),
            maxpool_P, apply_fold_int (down) (csrc/bnn_model.c:174-186)"""
    from oracle.oracle import RefC, ref_available
    if not ref_available():
        return None
    import numpy as np
    from bnns_to_c_amd import synth
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    ref = RefC()
    out = {}
    rng = np.random.default_rng(50)

    def signs(*shape):
        return np.where(rng.random(shape) < 0.5, -1, 1).astype(np.int8)
    # cfg1
    a1 = signs(64, 64, 64)
    w1 = ref.pack_weights(signs(64, 64, 3, 3))
    t1, n1 = _median_time(lambda: ref.bconv(a1, w1, 64), budget_s / 2)
    out["cfg1"] = {"patch_s": round(1.0 / t1, 2), "ms_per_patch": round(t1 * 1e3, 3), "cores": cores,
                   "binary_op_s": round(2 * 64 * 64 * 64 * 64 * 9 / t1, 1), "kind": "reference",
                   "sample": f"bconv_dispatch of the reference build, one 64x64 patch per call, median of {n1}"}
    # cfg2
    a2 = signs(128, 32, 32)
    w2 = ref.pack_weights(signs(128, 128, 3, 3))
    r1, r2 = synth.make_thresholds(32, 128, 288), synth.make_thresholds(33, 128, 288)

    def fused():
        P = ref.bconv(a2, w2, 128)
        ref.fold_int(P, *r1)
        ref.fold_int(ref.maxpool(P), *r2)
    t2, n2 = _median_time(fused, budget_s / 2)
    out["cfg2"] = {"patch_s": round(1.0 / t2, 2), "ms_per_patch": round(t2 * 1e3, 3), "cores": cores,
                   "binary_op_s": round(2 * 128 * 32 * 32 * 128 * 9 / t2, 1), "kind": "reference",
                   "sample": f"bconv_dispatch + apply_fold_int + maxpool_P + apply_fold_int of the reference "
                             f"build, one 32x32 patch per call, median of {n2}"}
    return out


def cpu_cli_patch(blob_path: str, H: int, W: int, reps: int):
    """The reference CLI (csrc/main.c) on one H x W "rand" patch of the
    blob: its median forward time in ms (None where it is not built)."""
    from oracle.oracle import REF_CLI
    if not os.path.exists(REF_CLI):
        return None
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    env = dict(os.environ, OMP_NUM_THREADS=str(cores))
    with tempfile.TemporaryDirectory() as td:
        r = subprocess.run([REF_CLI, blob_path, "rand", os.path.join(td, "o.bin"), str(H), str(W), str(reps)],
                           capture_output=True, text=True, env=env, timeout=600)
    if r.returncode != 0:
        raise RuntimeError(r.stderr)
    return float(re.search(r"# forward\s*:\s*([\d.]+) ms", r.stderr).group(1))


def cpu_baseline_react(blob_path: str, budget_s: float):
    """The reference v3 CLI (oracle/_ref/bnn_infer_react, built from its
    sources) on one 32x32x120 "rand" patch, median of reps
    (csrc/main_react.c:85-109); None where that build is absent."""
    from oracle.oracle import REACT_REF_CLI
    if not os.path.exists(REACT_REF_CLI):
        return None
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    env = dict(os.environ, OMP_NUM_THREADS=str(cores))

    def run(reps):
        with tempfile.TemporaryDirectory() as td:
            r = subprocess.run([REACT_REF_CLI, blob_path, "rand", os.path.join(td, "o.bin"), "32", "32", str(reps)],
                               capture_output=True, text=True, env=env, timeout=600)
        if r.returncode != 0:
            raise RuntimeError(r.stderr)
        return float(re.search(r"# forward \S+ reps=\d+\s+median ([\d.]+) ms", r.stdout).group(1))
    t1 = run(3)
    reps = max(5, min(2000, int(budget_s * 1000.0 / max(t1, 1e-3))))
    med = run(reps)
    return {"value": round(1000.0 / max(med, 1e-3), 2), "unit": "patches/s", "cores": cores, "kind": "reference",
            "sample": f"reference bnn_infer_react (csrc/main_react.c) built from its sources, one 32x32x120 "
                      f"patch, median of {reps} reps = {med:.1f} ms/patch (printed to 0.1 ms), "
                      f"OMP_NUM_THREADS={cores}"}


class StepEvents:
    """hipEvents that record a timestamp with no system-scope fence
    (hipEventDisableSystemFence, the HIP flag for events used only to
    measure time): a torch timing event makes its own cache writeback and
    signal between the steps it separates, about 6 us on the stream here,
    which back-to-back forwards do not pay.  Through the process's one HIP
    runtime (torch's and the library's share its soname)."""

    FLAG = 0x20000000  # hipEventDisableSystemFence

    def __init__(self, n: int):
        import ctypes
        self.C = ctypes
        self.hip = None
        for name in ("libamdhip64.so.7", "libamdhip64.so", "libamdhip64.so.6"):
            try:
                self.hip = ctypes.CDLL(name)
                break
            except OSError:
                continue
        assert self.hip is not None, "the HIP runtime (libamdhip64) is not loadable"
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.ev = []
        for _ in range(n):
            e = ctypes.c_void_p()
            rc = self.hip.hipEventCreateWithFlags(ctypes.byref(e), ctypes.c_uint(self.FLAG))
            assert rc == 0, f"hipEventCreateWithFlags: {rc}"
            self.ev.append(e)

    def record(self, k: int, stream_ptr: int) -> None:
        rc = self.hip.hipEventRecord(self.ev[k], self.C.c_void_p(stream_ptr))
        assert rc == 0, f"hipEventRecord: {rc}"

    def ms(self, a: int, b: int) -> float:
        t = self.C.c_float()
        rc = self.hip.hipEventElapsedTime(self.C.byref(t), self.ev[a], self.ev[b])
        assert rc == 0, f"hipEventElapsedTime: {rc}"
        return t.value

    def close(self) -> None:
        for e in self.ev:
            self.hip.hipEventDestroy(e)
        self.ev = []


def conv_time(engine, torch, fn, reps: int = 5):
    """Median first-conv time (ms) and median step time (ms) over reps
    profiled calls of fn, after an untimed settle."""
    import numpy as np
    settle(fn, torch, 0.02)
    torch.cuda.synchronize()
    steps = []
    engine.prof_reset()
    engine.prof_enable(True)
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        steps.append((time.perf_counter() - t0) * 1e3)
    engine.prof_enable(False)
    ms = [m for lab, op, m, w in engine.prof_records() if op == "conv_real"]
    return float(np.median(ms)), float(np.median(steps))


def cert_adversarial(torch, np, engine, blob, synth, td, sp, N, H, W):
    """The certified first conv on inputs built to leave outputs to its
    reference-order recompute (csrc/bnn_conv_realin.c:98-111), each against
    the same batch of N(0,1) patches:
      ties  every band +-1 (integer tap sums) and each channel's fold placed
            exactly on one integer sum, so csrc/bnn_fold.c:62-77 sits on
            z = 0 for about one output in a hundred;
      nan   a quarter of the patches all NaN, the others with a NaN block in
            every band (NaN windows are decided without a recompute);
      inf   one +inf per patch (band 7, pixel (16, 16)): its wave-row's bound
            is infinite, so every output of those rows is recomputed."""
    res = {}

    def run(tag, b, x):
        path = os.path.join(td, f"adv_{tag}.blob")
        blob.write(b, path)
        e = engine.Engine(path)
        dx = torch.from_numpy(x).cuda()
        dy = torch.empty((N, b.n_classes, H, W), dtype=torch.float32, device="cuda")
        fn = lambda: e.forward_device(dx.data_ptr(), N, H, W, dy.data_ptr(), sp)
        conv_ms, step_ms = conv_time(engine, torch, fn)
        e.cert_stats()
        fn()
        und, outs = e.cert_stats()
        e.close()
        res[tag] = {"first_conv_us": round(conv_ms * 1e3, 1), "forward_ms": round(step_ms, 3),
                    "recomputed_outputs": und, "outputs": outs}
        log(f"certified conv, {tag} input: {conv_ms * 1e3:.1f} us, {und} of {outs} outputs recomputed")

    b = synth.make_blob(seed=0, base=16)
    run("normal", b, synth.make_input(1, N, 120, H, W))
    xn = synth.make_input(1, N, 120, H, W)
    xn[: N // 4] = np.nan
    xn[N // 4:, :, 8:16, 10:22] = np.nan
    run("nan", b, xn)
    xi = synth.make_input(1, N, 120, H, W)
    xi[:, 7, H // 2, W // 2] = np.inf
    run("inf", b, xi)
    # ties: the fold's B from one of patch 0's own conv outputs per channel
    bt = synth.make_blob(seed=41)
    xt = np.random.default_rng(42).choice(np.array([-1.0, 1.0], np.float32), size=(N, 120, H, W))
    p0 = os.path.join(td, "adv_ties0.blob")
    blob.write(bt, p0)
    e0 = engine.Engine(p0)
    _, st = e0.forward_debug(xt[:1])
    e0.close()
    conv = st["enc1.conv1"][0]
    act = bt.enc_act1[0]
    A = act.A.astype(np.float32)
    Bv, rs = act.B.copy(), act.rsign.copy()
    for c in range(conv.shape[0]):
        Bv[c] = np.float32(-(A[c] * conv[c, 5 + c, 3 + c]))
        rs[c] = np.float32(0.0) if c % 2 == 0 else np.float32(1e-30)
    act.B, act.rsign = Bv.astype(np.float32), rs.astype(np.float32)
    run("ties", bt, xt)
    return res


def bench_cfg4(sp, stream, td, reps4=5):
    """Benchmark config 4: large tiles, 256 x 256 x 120, batch 64, base 32
    (wide layers, 512 channels at the bottleneck): the forward's time per
    step and every kernel's time by events."""
    import torch

    from bnns_to_c_amd import blob, engine, synth

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # the int8 matrix-core conv takes the fold convs of 32-wide rows with at
    # least 4 chunks of 64 input channels, the popcount kernel the rest
    b4 = synth.make_blob(seed=0, base=32)
    p4 = os.path.join(td, "bench_cfg4.blob")
    blob.write(b4, p4)
    eng4 = engine.Engine(p4)
    N4, S4 = 64, 256
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    x4 = torch.randn((N4, b4.n_bands, S4, S4), generator=gen, device="cuda", dtype=torch.float32)
    y4 = torch.empty((N4, b4.n_classes, S4, S4), dtype=torch.float32, device="cuda")
    settle(lambda: eng4.forward_device(x4.data_ptr(), N4, S4, S4, y4.data_ptr(), sp), torch)
    for _ in range(2):
        eng4.forward_device(x4.data_ptr(), N4, S4, S4, y4.data_ptr(), sp)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(reps4):
        eng4.forward_device(x4.data_ptr(), N4, S4, S4, y4.data_ptr(), sp)
    e1.record(stream)
    torch.cuda.synchronize()
    cfg4_ms = e0.elapsed_time(e1) / reps4
    engine.prof_reset()
    engine.prof_enable(True)
    for _ in range(reps4):
        eng4.forward_device(x4.data_ptr(), N4, S4, S4, y4.data_ptr(), sp)
    torch.cuda.synchronize()
    engine.prof_enable(False)
    agg4 = {}
    for lab, op, ms, work in engine.prof_records():
        a4 = agg4.setdefault(lab, [op, 0.0, 0, work])
        a4[1] += ms
        a4[2] += 1
    cfg4_kern = []
    for lab, (op, tot, cnt, work) in agg4.items():
        us = tot / cnt * 1e3
        k4 = {"label": lab, "op": op, "us": round(us, 2)}
        if op.endswith("_mfma"):
            k4["mac_s"] = round(work / (us / 1e6), 1)  # bit-MACs = int8 MACs
            k4["frac_int8_peak"] = round(work / (us / 1e6) / PEAK_INT8_MACS, 4)
        cfg4_kern.append(k4)
    log(f"cfg4 256x256x120 b{N4} base 32: {cfg4_ms:.3f} ms/step, {N4 / cfg4_ms * 1e3:,.0f} patches/s")
    for k4 in cfg4_kern:
        extra = f"  {k4['frac_int8_peak']:.3f} of int8 peak" if "mac_s" in k4 else ""
        log(f"  {k4['label']:10s} {k4['op']:16s} {k4['us']:9.1f} us{extra}")
    eng4.close()
    del x4, y4

    return cfg4_ms, cfg4_kern, N4, p4, S4


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=1024)
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline work")
    ap.add_argument("--settle", type=int, default=120,
                    help="untimed forwards before the warmup steps, for the GPU clocks to settle")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--headline-only", action="store_true",
                    help="the headline forward and its per-kernel pass only (for profiler runs)")
    ap.add_argument("--cfg4-only", action="store_true",
                    help="benchmark config 4 only, --steps timed forwards and as many with per-kernel events "
                         "(for profiler runs); prints its own JSON line")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the patch batch would shard across GPUs with no exchange "
              "between them, and this build runs on one GPU; use --gpus 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from bnns_to_c_amd import blob, engine, synth

    if args.cfg4_only:
        stream = torch.cuda.Stream()
        torch.cuda.set_stream(stream)
        cfg4_ms, cfg4_kern, N4, _, _ = bench_cfg4(stream.cuda_stream, stream, tempfile.mkdtemp(), reps4=args.steps)
        print(json.dumps({"config": "benchmark config 4: 256x256x120, batch 64, base 32", "ms_per_step": round(cfg4_ms, 4),
                          "patches_s": round(N4 / cfg4_ms * 1e3, 1), "steps": args.steps, "kernels": cfg4_kern}),
              flush=True)
        return 0

    N, H, W = args.batch, 32, 32
    b = synth.make_blob(seed=0, base=16)
    td = tempfile.mkdtemp()
    blob_path = os.path.join(td, "bench.blob")
    blob.write(b, blob_path)
    eng = engine.Engine(blob_path)
    x = torch.from_numpy(synth.make_input(1, N)).cuda()
    y = torch.empty((N, b.n_classes, H, W), dtype=torch.float32, device="cuda")
    # every engine enqueues on this stream and the timing events are recorded
    # on it
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    sp = stream.cuda_stream
    assert sp, "the timing stream must not be the default stream"
    torch.cuda.synchronize()

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


    if not args.headline_only:
        # benchmark config 1: the isolated binary conv, 64->64 at 64x64, batch
        # 256, int32 P out (268 MB, the accumulator the reference's bconv
        # returns)
        N1, S1, C1 = 256, 64, 64
        a1 = synth.make_bits(20, N1, S1, S1, C1)
        L1 = engine.ConvLayer(blob.pack_kidx(synth.make_signs(21, C1, C1)), C1, C1)
        da1 = torch.from_numpy(a1).cuda()
        act1 = torch.empty((N1, S1, S1, C1 // 32), dtype=torch.int32, device="cuda")
        engine.pack_act_device(da1.data_ptr(), act1.data_ptr(), N1, C1, S1, S1, sp)
        del da1
        P1 = torch.empty((N1, C1, S1, S1), dtype=torch.int32, device="cuda")
        settle(lambda: L1.P_device(act1.data_ptr(), N1, S1, S1, P1.data_ptr(), sp), torch)
        for _ in range(3):
            L1.P_device(act1.data_ptr(), N1, S1, S1, P1.data_ptr(), sp)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(20):
            L1.P_device(act1.data_ptr(), N1, S1, S1, P1.data_ptr(), sp)
        e1.record(stream)
        torch.cuda.synchronize()
        c1_ms = e0.elapsed_time(e1) / 20
        c1_bitmacs = N1 * C1 * S1 * S1 * C1 * 9
        c1_rate = 2 * c1_bitmacs / (c1_ms / 1e3)
        c1_bytes = N1 * S1 * S1 * (C1 // 8) + P1.numel() * 4  # packed bits in, int32 P out
        log(f"cfg1 bconv 64->64 64x64 b{N1}, int32 P out: {c1_ms * 1e3:.1f} us, frac {c1_rate / valu_binop_peak():.3f} "
            f"of VALU popcount peak, {c1_bytes / (c1_ms / 1e3) / 1e9:.0f} GB/s of algorithmic HBM bytes")
        L1.close()
        del act1, P1

        # fused bconv + fold + 2x2 max-pool, 128->128 at 32x32, batch 1024
        C = 128
        a = synth.make_bits(30, N, H, W, C)
        w = synth.make_signs(31, C, C)
        L = engine.ConvLayer(blob.pack_kidx(w), C, C, synth.make_thresholds(32, C, 288),
                             synth.make_thresholds(33, C, 288))
        da = torch.from_numpy(a).cuda()
        act = torch.empty((N, H, W, C // 32), dtype=torch.int32, device="cuda")
        engine.pack_act_device(da.data_ptr(), act.data_ptr(), N, C, H, W, sp)
        del da
        skip = torch.empty((N, H, W, C // 32), dtype=torch.int32, device="cuda")
        down = torch.empty((N, H // 2, W // 2, C // 32), dtype=torch.int32, device="cuda")
        reps = 20
        settle(lambda: L.fold_pool_device(act.data_ptr(), N, H, W, skip.data_ptr(), down.data_ptr(), sp), torch)
        for _ in range(3):
            L.fold_pool_device(act.data_ptr(), N, H, W, skip.data_ptr(), down.data_ptr(), sp)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(reps):
            L.fold_pool_device(act.data_ptr(), N, H, W, skip.data_ptr(), down.data_ptr(), sp)
        e1.record(stream)
        torch.cuda.synchronize()
        pool_ms = e0.elapsed_time(e1) / reps
        pool_bitmacs = N * C * H * W * C * 9
        pool_rate = 2 * pool_bitmacs / (pool_ms / 1e3)
        # this shape (cout 128, 32-wide rows) is inside the int8 matrix-core
        # rule unless BNN_BCONV_MFMA=0 keeps the popcount kernel; the
        # fraction is of the path's own peak
        pool_mfma = os.environ.get("BNN_BCONV_MFMA") != "0"
        pool_frac = pool_bitmacs / (pool_ms / 1e3) / PEAK_INT8_MACS if pool_mfma else pool_rate / valu_binop_peak()
        pool_peak = "int8 matrix peak" if pool_mfma else "VALU popcount peak"
        log(f"fused bconv+fold+pool 128->128 32x32 b{N}: {pool_ms * 1e3:.1f} us, frac {pool_frac:.3f} of {pool_peak}")
        L.close()
        pool_pc = None
        if pool_mfma:
            # the same layer on the bit-packed popcount kernel (the mode is
            # read when a layer is made), against the VALU-popcount peak
            old = os.environ.get("BNN_BCONV_MFMA")
            os.environ["BNN_BCONV_MFMA"] = "0"
            try:
                Lp = engine.ConvLayer(blob.pack_kidx(w), C, C, synth.make_thresholds(32, C, 288),
                                      synth.make_thresholds(33, C, 288))
            finally:
                if old is None:
                    os.environ.pop("BNN_BCONV_MFMA", None)
                else:
                    os.environ["BNN_BCONV_MFMA"] = old
            settle(lambda: Lp.fold_pool_device(act.data_ptr(), N, H, W, skip.data_ptr(), down.data_ptr(), sp), torch)
            torch.cuda.synchronize()
            e0.record(stream)
            for _ in range(reps):
                Lp.fold_pool_device(act.data_ptr(), N, H, W, skip.data_ptr(), down.data_ptr(), sp)
            e1.record(stream)
            torch.cuda.synchronize()
            pc_ms = e0.elapsed_time(e1) / reps
            pc_rate = 2 * pool_bitmacs / (pc_ms / 1e3)
            pool_pc = {"kernel": "k_bconv (VALU popcount, BNN_BCONV_MFMA=0)", "us": round(pc_ms * 1e3, 2),
                       "binary_op_s": round(pc_rate, 1), "frac": round(pc_rate / valu_binop_peak(), 4),
                       "frac_of": "VALU popcount peak"}
            log(f"  the same on the popcount kernel: {pc_ms * 1e3:.1f} us, frac {pc_rate / valu_binop_peak():.3f} "
                f"of the VALU popcount peak")
            Lp.close()

        cfg4_ms, cfg4_kern, N4, p4, S4 = bench_cfg4(sp, stream, td)

        # benchmark config 3: a 956 x 684 x 120 scene (N(0,1) plus a per-band
        # offset U(-0.5, 0.5)) cut into 32 x 32 patches, 30 x 22 = 660 with the
        # edge patches zero past the scene; the device call reads the patches
        # straight out of the cube, the host call adds the strip-wise PCIe copy
        SH, SW, PS = 956, 684, 32
        rng = np.random.default_rng(40)
        cube = rng.standard_normal((b.n_bands, SH, SW), dtype=np.float32)
        cube += rng.uniform(-0.5, 0.5, (b.n_bands, 1, 1)).astype(np.float32)
        npatch = ((SH + PS - 1) // PS) * ((SW + PS - 1) // PS)
        d_cube = torch.from_numpy(cube).cuda()
        d_map = torch.empty((b.n_classes, SH, SW), dtype=torch.float32, device="cuda")
        settle(lambda: eng.forward_patched_device(d_cube.data_ptr(), SH, SW, d_map.data_ptr(), PS, sp), torch)
        for _ in range(3):
            eng.forward_patched_device(d_cube.data_ptr(), SH, SW, d_map.data_ptr(), PS, sp)
        torch.cuda.synchronize()
        reps = 10
        e0.record(stream)
        for _ in range(reps):
            eng.forward_patched_device(d_cube.data_ptr(), SH, SW, d_map.data_ptr(), PS, sp)
        e1.record(stream)
        torch.cuda.synchronize()
        scene_dev_ms = e0.elapsed_time(e1) / reps
        host_map = eng.forward_patched(cube, PS)
        assert np.array_equal(host_map.view(np.uint32), d_map.cpu().numpy().view(np.uint32))
        t0 = time.perf_counter()
        for _ in range(3):
            eng.forward_patched(cube, PS)
        scene_host_ms = (time.perf_counter() - t0) / 3 * 1e3
        log(f"scene {SH}x{SW}x{b.n_bands} ({npatch} patches): device {scene_dev_ms:.3f} ms "
            f"({npatch / scene_dev_ms * 1e3:,.0f} patches/s), host pointers {scene_host_ms:.2f} ms "
            f"({cube.nbytes / scene_host_ms / 1e6:.1f} GB/s of input)")
        # per-kernel times of the device scene call (one launch of 660 patches
        # per kernel: the batch is not split across streams here)
        engine.prof_reset()
        engine.prof_enable(True)
        for _ in range(reps):
            eng.forward_patched_device(d_cube.data_ptr(), SH, SW, d_map.data_ptr(), PS, sp)
        torch.cuda.synchronize()
        engine.prof_enable(False)
        agg3 = {}
        for lab, op, ms, work in engine.prof_records():
            agg3.setdefault(lab, [op, []])[1].append(ms)
        scene_kern = [{"label": lab, "op": op, "us": round(float(np.median(v)) * 1e3, 2)}
                      for lab, (op, v) in agg3.items()]
        for k3 in scene_kern:
            log(f"  scene {k3['label']:10s} {k3['op']:12s} {k3['us']:9.1f} us")
        del d_cube, d_map

        adversarial = cert_adversarial(torch, np, engine, blob, synth, td, sp, N, H, W)

        # the v2 spectral-stem model (csrc/bnn_model_stem.c): 16-channel stem
        # (the reference exporter's default), base 16, same batch and input
        bs = synth.make_blob_v2(seed=0, base=16, stem=16)
        stem_path = os.path.join(td, "bench_stem.blob")
        blob.write(bs, stem_path)
        seng = engine.StemEngine(stem_path)

        def sstep():
            seng.forward_device(x.data_ptr(), N, H, W, y.data_ptr(), sp)

        settle(sstep, torch)
        for _ in range(args.warmup):
            sstep()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(args.steps):
            sstep()
        e1.record(stream)
        torch.cuda.synchronize()
        v2_ms = e0.elapsed_time(e1) / args.steps
        engine.prof_reset()
        engine.prof_enable(True)
        for _ in range(args.steps):
            sstep()
        torch.cuda.synchronize()
        engine.prof_enable(False)
        stem_ms = [ms for lab, op, ms, work in engine.prof_records() if lab == "stem.conv"]
        stem_ms = sum(stem_ms) / len(stem_ms)
        # algorithmic bytes: every input float once, one 32-bit word of stem bits per pixel out
        stem_bytes = N * bs.n_bands * H * W * 4 + N * H * W * 4
        stem_rate = stem_bytes / (stem_ms / 1e3)
        log(f"v2 stem model: {v2_ms:.4f} ms/step, {N / v2_ms * 1e3:,.0f} patches/s; stem kernel "
            f"{stem_ms * 1e3:.1f} us, {stem_rate / 1e9:.0f} GB/s ({stem_rate / PEAK_HBM:.3f} of HBM peak)")
        seng.close()

        # the v3 ReActNet model (csrc/bnn_model_react.c): float highway, taps,
        # 1x1 projections, RPReLU epilogues; base 16, same batch and input
        from bnns_to_c_amd import blob_react
        br = synth.make_blob_react(seed=0, base=16)
        react_path = os.path.join(td, "bench_react.blob")
        blob_react.write(br, react_path)
        reng = engine.ReactEngine(react_path)

        def rstep():
            reng.forward_device(x.data_ptr(), N, H, W, y.data_ptr(), sp)

        settle(rstep, torch)
        for _ in range(args.warmup):
            rstep()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(args.steps):
            rstep()
        e1.record(stream)
        torch.cuda.synchronize()
        v3_ms = e0.elapsed_time(e1) / args.steps
        engine.prof_reset()
        engine.prof_enable(True)
        for _ in range(args.steps):
            rstep()
        torch.cuda.synchronize()
        engine.prof_enable(False)
        ragg = {}
        for lab, op, ms, work in engine.prof_records():
            a = ragg.setdefault(lab, [op, 0.0, 0, work])
            a[1] += ms
            a[2] += 1
        rkern = [{"label": lab, "op": op, "us": round(tot / cnt * 1e3, 2)} for lab, (op, tot, cnt, _) in ragg.items()]
        in_us = ragg["enc1.u1"][1] / ragg["enc1.u1"][2] * 1e3
        # enc1 unit 1: the 3x3 conv (1,080 FMAs per output) and the projection
        # (120 per output), 16 channels x 32 x 32 per patch
        in_flops = 2.0 * N * br.enc[0].conv1.cout * H * W * br.n_bands * 10
        in_rate = in_flops / (in_us / 1e6)
        v3_cpu = None if args.no_cpu else cpu_baseline_react(react_path, args.cpu_budget / 2)
        log(f"v3 ReActNet model: {v3_ms:.4f} ms/step, {N / v3_ms * 1e3:,.0f} patches/s; enc1 unit-1 kernel "
            f"{in_us:.1f} us, {in_rate / 1e12:.1f} TFLOP/s ({in_rate / PEAK_FP32_FLOPS:.3f} of peak)")
        for k in rkern:
            log(f"  {k['label']:10s} {k['op']:10s} {k['us']:9.1f} us")
        reng.close()

    # the headline, measured last: the configurations above have kept the
    # GPU busy for several seconds by now, so its clocks have settled
    def step():
        eng.forward_device(x.data_ptr(), N, H, W, y.data_ptr(), sp)

    # Settle: the GPU's clocks ramp under sustained load (measured on the
    # box: per-step time falls from ~0.58 to ~0.50 ms over the first ~40
    # forwards, about 25 ms, then holds; after half a second idle it ramps
    # again).  args.settle untimed forwards go first, queued back to back
    # with the W warmup steps and the timed ones, so the timed steps run at
    # the steady clock; the count is reported as "settle_steps".
    for _ in range(args.settle):
        step()
    for _ in range(args.warmup):
        step()
    # The K timed steps run back to back between one pair of timing-only
    # events (StepEvents) and device synchronisations: ms_per_step is their
    # mean (the reference's figure: N / wall time of one batched forward;
    # csrc/main.c:55-61).  An event between consecutive steps is a packet of
    # its own on the stream that the next step's first kernel waits for
    # (about 3 us a step here even without a cache fence), so the spread
    # comes from a second pass of K steps with an event between each pair:
    # its median, min and max are reported beside the mean.
    evs = StepEvents(2)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    evs.record(0, sp)
    for k in range(args.steps):
        step()
    evs.record(1, sp)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = evs.ms(0, 1) / args.steps
    evs.close()
    evs = StepEvents(args.steps + 1)
    evs.record(0, sp)
    for k in range(args.steps):
        step()
        evs.record(k + 1, sp)
    torch.cuda.synchronize()
    step_ms = [evs.ms(k, k + 1) for k in range(args.steps)]
    evs.close()
    med_ms = float(np.median(step_ms))
    value = N / (ms_per_step / 1e3)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log("  step times with an event between steps (ms): " + " ".join(f"{t:.3f}" for t in step_ms))
    log(f"forward: {ms_per_step:.4f} ms/step (mean of {args.steps} back-to-back steps; with an event between steps "
        f"median {med_ms:.4f}, min {min(step_ms):.4f}, max {max(step_ms):.4f}), {value:,.0f} patches/s")


    # per-kernel times: the same forward with an event pair around every kernel
    engine.prof_reset()
    engine.prof_enable(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    engine.prof_enable(False)
    recs = engine.prof_records()
    agg = {}
    for lab, op, ms, work in recs:
        a = agg.setdefault(lab, [op, [], 0, work])
        a[1].append(ms)
        a[2] += 1
    # which first-conv kernel ran: the certified one unless BNN_CERT=0 (its
    # shape condition, 4 <= cin <= 128 and W in multiples of 4, holds here)
    cert = os.environ.get("BNN_CERT") != "0"
    real_bytes = N * 120 * H * W * 4 + N * H * W * 4  # input floats once, output words once
    kernels = []
    for lab, (op, mss, cnt, work) in agg.items():
        mean = float(np.median(mss))  # median over the profiled forwards
        if op == "conv_real":
            rate = 2 * work / (mean / 1e3)
            if cert:
                # bound by HBM: frac is the fraction of the 8 TB/s peak
                kernels.append({"label": lab, "op": op, "ms": round(mean, 5), "bound": "hbm",
                                "gb_s": round(real_bytes / (mean / 1e3) / 1e9, 1),
                                "frac": round(real_bytes / (mean / 1e3) / PEAK_HBM, 4),
                                "fp32_equivalent_tflops": round(rate / 1e12, 3)})
            else:
                kernels.append({"label": lab, "op": op, "ms": round(mean, 5), "bound": "mfma",
                                "tflops": round(rate / 1e12, 3), "frac": round(rate / PEAK_FP32_FLOPS, 4)})
        else:
            rate = 2 * work / (mean / 1e3)
            kernels.append({"label": lab, "op": op, "ms": round(mean, 5), "tbinops": round(rate / 1e12, 2),
                            "frac": round(rate / valu_binop_peak(), 4)})
    for k in kernels:
        log(f"  {k['label']:10s} {k['op']:10s} {k['ms']*1e3:9.1f} us  frac {k['frac']:.3f}")
    real = next(k for k in kernels if k["op"] == "conv_real")
    real_work = agg[real["label"]][3]
    real_flops = 2 * real_work
    achieved = real_flops / (real["ms"] / 1e3)
    if cert:
        rate_b = real_bytes / (real["ms"] / 1e3)
        # outputs the bound left open and the kernel recomputed in the
        # reference's order, in one headline forward
        eng.cert_stats()
        step()
        und, outs = eng.cert_stats()
        roofline = {"bound": "hbm",
                    "kernel": "enc1.conv1 certified first conv + real fold (fp16 matrix-core integer-digit sums, "
                              "rigorous error bound, reference-order recompute of undecided outputs)",
                    "achieved": round(rate_b / 1e9, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                    "frac": round(rate_b / PEAK_HBM, 4), "traffic": measured_traffic(),
                    "traffic_source": "profiles/unet_b1024_hbm_traffic.md (rocprofv3 FETCH_SIZE+WRITE_SIZE, "
                                      "calibrated)",
                    "algorithmic": f"{real_bytes} B/launch = {N} patches x (120 x 32 x 32 x 4 B in + 32 x 32 x 4 B "
                                   "out)",
                    "fp32_equivalent": {"tflops": round(achieved / 1e12, 3),
                                        "of_fp32_matrix_peak": round(achieved / PEAK_FP32_FLOPS, 4),
                                        "note": f"{real_flops:.4g} FLOP of the FP32 conv per launch / the same time"},
                    "recomputed_outputs": und, "outputs": outs}
    else:
        roofline = {"bound": "mfma", "kernel": "enc1.conv1 real-input conv + real fold (order-exact FP32, K=1 MFMA)",
                    "achieved": round(achieved / 1e12, 3), "peak": PEAK_FP32_FLOPS / 1e12, "unit": "TFLOP/s",
                    "frac": round(achieved / PEAK_FP32_FLOPS, 4), "traffic": measured_traffic(),
                    "traffic_source": "profiles/unet_b1024_hbm_traffic.md (rocprofv3 FETCH_SIZE+WRITE_SIZE, "
                                      "calibrated)",
                    "algorithmic": f"{real_flops:.4g} FLOP/launch = 2 x 17,694,720 MAC x {N} patches"}
    log(f"roofline: {roofline['kernel']}: {roofline['achieved']} {roofline['unit']}, frac {roofline['frac']}")

    exact = None
    if cert and not args.headline_only:
        # the order-exact first conv on the same batch, from a model loaded
        # with BNN_CERT=0 (the variable is read when a model is loaded)
        os.environ["BNN_CERT"] = "0"
        try:
            xeng = engine.Engine(blob_path)
        finally:
            os.environ.pop("BNN_CERT", None)
        settle(lambda: xeng.forward_device(x.data_ptr(), N, H, W, y.data_ptr(), sp), torch)
        engine.prof_reset()
        engine.prof_enable(True)
        for _ in range(10):
            xeng.forward_device(x.data_ptr(), N, H, W, y.data_ptr(), sp)
        torch.cuda.synchronize()
        engine.prof_enable(False)
        xms = float(np.median([ms for lab, op, ms, work in engine.prof_records() if op == "conv_real"]))
        xrate = real_flops / (xms / 1e3)
        exact = {"kernel": "order-exact FP32 first conv (K=1 MFMA chains in the reference's order), BNN_CERT=0",
                 "us": round(xms * 1e3, 2), "tflops": round(xrate / 1e12, 3),
                 "frac": round(xrate / PEAK_FP32_FLOPS, 4), "peak": PEAK_FP32_FLOPS / 1e12}
        log(f"order-exact first conv (BNN_CERT=0): {xms * 1e3:.1f} us, {xrate / 1e12:.1f} TFLOP/s, "
            f"frac {xrate / PEAK_FP32_FLOPS:.3f} of the FP32 matrix peak")
        xeng.close()
    bin_ms = sum(k["ms"] for k in kernels if k["op"] != "conv_real")
    bin_work = sum(agg[k["label"]][3] for k in kernels if k["op"] != "conv_real")
    bin_rate = 2 * bin_work / (bin_ms / 1e3)

    if not args.headline_only:
        # the same batch from and to host memory (pinned buffers): the copies in
        # and out over PCIe are part of each call (bnn_forward_batch)
        xh = torch.from_numpy(synth.make_input(1, N)).pin_memory()
        yh = torch.empty((N, b.n_classes, H, W), dtype=torch.float32).pin_memory()
        for _ in range(2):
            eng.forward_batch_ptr(xh.data_ptr(), N, H, W, yh.data_ptr())
        host_ms = []
        for _ in range(max(3, min(args.steps, 10))):
            h0 = time.perf_counter()
            eng.forward_batch_ptr(xh.data_ptr(), N, H, W, yh.data_ptr())
            host_ms.append((time.perf_counter() - h0) * 1e3)
        pcie_ms = float(np.median(host_ms))
        assert np.array_equal(yh.numpy().view(np.uint32), y.cpu().numpy().view(np.uint32))
        log(f"forward with host buffers (pinned, copies in and out included): {pcie_ms:.3f} ms, "
            f"{N / pcie_ms * 1e3:,.0f} patches/s ({xh.numel() * 4 / pcie_ms / 1e6:.1f} GB/s of input)")
        del xh, yh

    cpu = None
    cpu_cfg = {}
    if not args.no_cpu and not args.headline_only:
        log("cpu baseline ...")
        cpu = cpu_baseline(blob_path, args.cpu_budget)
        log(f"cpu baseline: {cpu}")
        # the other configs on the reference's own code, same host, same run
        lay = cpu_layer_baselines(args.cpu_budget / 4) or {}
        gpu_ps = {"cfg1": N1 / (c1_ms / 1e3), "cfg2": N / (pool_ms / 1e3)}
        for k, v in lay.items():
            v["speedup"] = round(gpu_ps[k] / v["patch_s"], 1)
            cpu_cfg[k] = v
        if cpu:
            # cfg3: the scene is the reference's per-patch forward, patch after patch
            cpu_cfg["cfg3"] = {"scene_ms": round(npatch / cpu["value"] * 1e3, 1), "patches_s": cpu["value"],
                               "cores": cpu["cores"], "kind": cpu["kind"],
                               "speedup": round(scene_dev_ms and (npatch / scene_dev_ms * 1e3) / cpu["value"], 1),
                               "sample": "the config-0 measurement (reference bnn_infer per 32x32 patch) times "
                                         f"{npatch} patches"}
        t4 = cpu_cli_patch(p4, S4, S4, 1)
        if t4:
            cpu_cfg["cfg4"] = {"ms_per_patch": round(t4, 1), "patch_s": round(1e3 / t4, 3), "cores": cpu["cores"]
                               if cpu else None, "kind": "reference",
                               "speedup": round((N4 / cfg4_ms * 1e3) / (1e3 / t4), 1),
                               "sample": "reference bnn_infer (csrc/main.c) on one 256x256 rand patch of the base-32 "
                                         "blob, one rep"}
        for k, v in cpu_cfg.items():
            log(f"cpu {k}: {v}")
    eng.close()

    out = {
        "metric": "patches/s full UNet @32x32x120 b1024; bconv binary-op/s as % of roofline",
        "value": round(value, 1),
        "unit": "patches/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "wall_ms_per_step": round(wall / args.steps * 1e3, 5),
        "settle_steps": args.settle,
        "evented_step_ms": {"median": round(med_ms, 5), "min": round(min(step_ms), 5),
                            "max": round(max(step_ms), 5),
                            "note": "a second pass of the same K steps with a timing event between "
                                    "consecutive steps (each event a packet the next step waits for)"},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 first conv (certified: fp16 matrix-core digit sums, exact fp32 recompute where undecided) "
                 "+ xnor-popcount (u32) binary convs",
        "data": "synthetic: seeded random blob (base 16, Bernoulli sign weights, U[-fan_in/4,fan_in/4] "
                "ge/lt thresholds) and x ~ N(0,1) patches, resident in HBM",
        "config": {"workload": "v1 Bi-Real binary UNet forward (nearest upsampler), 32x32x120 patches",
                   "batch": N, "H": H, "W": W, "n_bands": 120, "n_classes": 3, "base_channels": 16},
        "roofline": roofline,
        "bconv": {"layers": 17, "kernels": sum(1 for k in kernels if k["op"] != "conv_real"),
                  "binary_op_s": round(bin_rate, 1), "peak": valu_binop_peak(),
                  "frac": round(bin_rate / valu_binop_peak(), 4), "ms": round(bin_ms, 5),
                  "unit": "binary-op/s (2 per bit-MAC, border taps counted)"},
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    if not args.headline_only:
        out.update({
            "with_copies": {"config": "the same batch from and to pinned host memory (bnn_forward_batch: copies "
                                      "in and out over PCIe included)",
                            "ms_per_step": round(pcie_ms, 4), "patches_s": round(N / pcie_ms * 1e3, 1)},
            "cpu_configs": cpu_cfg,
            "first_conv_exact": exact,
            "cfg1": {"config": "isolated bconv 64->64, 64x64, batch 256, int32 P out (benchmark config 1)",
                     "us": round(c1_ms * 1e3, 2), "binary_op_s": round(c1_rate, 1),
                     "frac": round(c1_rate / valu_binop_peak(), 4),
                     "hbm_GB_s": round(c1_bytes / (c1_ms / 1e3) / 1e9, 1),
                     "hbm_frac": round(c1_bytes / (c1_ms / 1e3) / PEAK_HBM, 4)},
            "fused_pool": {"config": "bconv 128->128 + fold + 2x2 maxpool + fold, 32x32, batch 1024",
                           "us": round(pool_ms * 1e3, 2), "binary_op_s": round(pool_rate, 1),
                           "kernel": "k_bconv_mfma (int8 matrix cores)" if pool_mfma else "k_bconv (VALU popcount)",
                           "frac": round(pool_frac, 4), "frac_of": pool_peak,
                           **({"popcount": pool_pc} if pool_pc else {})},
            "cfg4": {"config": "large tiles: 256x256x120, batch 64, base 32 (512 channels at the bottleneck)",
                     "ms_per_step": round(cfg4_ms, 4), "patches_s": round(N4 / cfg4_ms * 1e3, 1),
                     "kernels": cfg4_kern,
                     "int8_mfma_rule": "fold and pool convs with cout % 64 == 0, rows at least 16 wide and "
                                       "64+ input channels (enc2.c2 .. dec2.c2 here)"},
            "scene": {"config": f"{SH}x{SW}x{b.n_bands} cube, {PS}x{PS} patches ({npatch}, edge patches zero "
                                "past the scene), benchmark config 3",
                      "device_ms": round(scene_dev_ms, 4), "device_patches_s": round(npatch / scene_dev_ms * 1e3, 1),
                      "host_ms": round(scene_host_ms, 3),
                      "host_note": "host cube in, host map out: strips through pinned buffers over PCIe",
                      "kernels": scene_kern},
            "cert_adversarial": {"config": f"the headline batch ({N} patches 32x32x120): the certified first conv "
                                           "on N(0,1) patches, on patches with NaNs, on patches with one +inf "
                                           "each, and on +-1 bands with each channel's fold placed on an integer "
                                           "tap sum (about 1% of outputs on the fold's switch point)",
                                 **adversarial},
            "v2_stem": {"config": "v2 spectral-stem model, 16-channel 1x1 stem, base 16, 32x32x120, batch 1024",
                        "ms_per_step": round(v2_ms, 5), "patches_s": round(N / v2_ms * 1e3, 1),
                        "stem_kernel_us": round(stem_ms * 1e3, 2), "stem_bytes": stem_bytes,
                        "stem_hbm_GB_s": round(stem_rate / 1e9, 1), "stem_frac": round(stem_rate / PEAK_HBM, 4)},
            "v3_react": {"config": "v3 ReActNet real-highway model, base 16, 32x32x120, batch 1024",
                         "ms_per_step": round(v3_ms, 5), "patches_s": round(N / v3_ms * 1e3, 1),
                         "enc1_kernel_us": round(in_us, 2), "enc1_tflops": round(in_rate / 1e12, 3),
                         "enc1_frac": round(in_rate / PEAK_FP32_FLOPS, 4),
                         "enc1_algorithmic": f"{in_flops:.4g} FLOP/launch = 2 x 16 x 1024 px x 120 x (9 + 1) "
                                             f"x {N} patches",
                         "kernels": rkern, "cpu_baseline": v3_cpu},
        })
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
