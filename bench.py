#!/usr/bin/env python3
"""Benchmark of the FP8 hot path on one MI355X.

Step (timed): config 3 of the baseline -- block_scaled_matmul forward + FP8
backward on x [8192, 2048], W [2048, 8192], dY [8192, 8192] (bf16, synthetic,
seeded), the kernel sequence of fp8.block_scaled_matmul's autograd path:
quantize x along K and x.T along M (one read of x), W.T along K and W along N
(one read of W) -> GEMM Y; quantize dY along N and dY.T along M (one read of
dY) -> GEMM dX, GEMM dW.  Every kernel is a C-ABI call into libtg_fp8.so on
torch's current stream (the *_km entry points: scales kept K-block-major, as
the autograd path keeps them); the step allocates nothing.

value        = 3 * 2*8192*2048*8192 FLOP / step time (TFLOP/s, quantization included),
               timed over exactly --steps steps after an untimed 150 ms clock-settle
               phase of the same step (reported as clock_settle) and --warmup steps
roofline     = the GEMM kernel: 2*M*N*K FLOP per launch / its mean launch time
               (HIP events around each GEMM launch, in a second pass of the
               same steps right after the timed region: an event record on
               the stream leaves it idle for ~4.5 us, so the region that
               gives `value` has events only at its two ends) vs MI355X
               dense FP8 MFMA peak 5.0 PFLOP/s
sustained_clock = after the timed region, the step and then its dX GEMM alone
               back to back for 3 s each, with amdsmi polled for the engine
               clock (median) and socket energy (average power) against the cap;
               the GEMM's rate is also given against the FP8 peak scaled from
               its 2400 MHz to the clock it sustains (not run under rocprofv3)
norm_quant   = config 2 fused RMSNorm -> FP8 quantize, bytes per launch
               84,414,464 (x read + y/q/scales written + gamma) / mean launch
               time vs 8 TB/s HBM; input/output sets rotate over > 256 MB so
               the Infinity Cache cannot serve them
norm_bwd     = rms_norm's backward (kernels.py:104-118) at config 2's shape:
               x, dy read + dx written + gamma / dgamma = 100,671,488 B per call
               (row kernel + column reduce) vs 8 TB/s HBM
gemv         = config 5 decode GEMV on a pre-quantized W [4096, 14336] (e4m3,
               128x128 scales) for M in {1, 8, 32}: algorithmic bytes of the
               GEMV launch (W bytes + W scales + x bytes + x scales + bf16 out)
               / mean launch time vs 8 TB/s; 5 weight copies rotate (> 256 MB)
bwd_bf16     = the reference's straight-through bf16 backward (fp8.py:85-98)
               at config 3: 2 bf16 GEMMs (+ operand packing) per call vs the
               2.5 PFLOP/s dense bf16 MFMA peak
block_step   = config 4: one decoder block training step (block.py), FP8 linears
               vs bf16 linears, wall time per step
xent         = config 4's head: fused logit cap + cross entropy (losses.py) on
               bf16 logits [8192, 50304]; forward reads the logits once
               (+ targets, per-row loss / lse), backward reads them again and
               writes bf16 dlogits; bytes / mean launch time vs 8 TB/s
decode       = KV-cached decode (decode.py) of the reference model config:
               ms per decode step at batch 1 and 8, and the kept FP8 weights +
               KV cache read per step against 8 TB/s
block_k_sizes = config 3's forward (tg_block_scaled_matmul) at block_k 128,
               64 (zero-filled 128-byte slots) and 256 (repeated scales):
               mean time per call, quantization included
io_floor     = (--only) config 2's bytes moved by csrc/probe/io_floor.hip with
               the fused norm kernel's access pattern and no arithmetic: the
               attainable rate of that read / write mix, beside the real kernel
quant_floor  = (--only) config 3's dual quantizers beside the same kernel with
               its arithmetic taken out (csrc/probe/quant_floor.hip): the I/O
               floor of their access pattern, with and without the scales
gemv_floor   = (--only) the reference decode weights at 8 rows: the direct
               GEMV's loads moved by csrc/probe/gemv_stream.hip with no
               arithmetic (with and without the x rows, cached and
               non-temporal), beside tg_gemv_fp8 on the same weights
cpu_baseline = the CPU oracle (numpy + C) on a row sample of the same step

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                      [--only step|norm_quant|norm_bwd|gemv|bwd_bf16|block_step|xent|decode|
                              vendor_gemm|c1|block_k|io_floor|quant_floor|gemv_floor]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "train-gpt_amd"))
sys.path.insert(0, ROOT)

FP8_PEAK_TFLOPS = 5000.0       # MI355X dense FP8 MFMA
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
HBM_PEAK_GBPS = 8000.0         # MI355X HBM3E
M3, K3, N3 = 8192, 2048, 8192
GEMM_FLOP = 2.0 * M3 * N3 * K3
STEP_FLOP = 3 * GEMM_FLOP
C2_ROWS, C2_D = 8 * 1024, 2048
C2_BYTES = C2_ROWS * C2_D * (2 + 2 + 1) + C2_ROWS * (C2_D // 128) * 4 + C2_D * 2
C2_BWD_BYTES = C2_ROWS * C2_D * (2 + 2 + 2) + 2 * C2_D * 2
C5_K, C5_N = 4096, 14336
CLOCK_SETTLE_MS = 150.0        # untimed steps before the warm-up (the clock ramps ~30 ms after idle)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "bench_hbm_traffic_counters.md")


def under_counter_collection() -> bool:
    """True inside `rocprofv3 --pmc` (its launcher exports ROCPROF_COUNTER_COLLECTION=1).
    A full bench run under counter collection once died with SIGSEGV in a
    profiler host thread; the only part of that run no single-workload counter
    pass had covered besides the C4 block step was the decode workload's
    captured-graph replay, so the decode workload is left out in that mode."""
    return os.environ.get("ROCPROF_COUNTER_COLLECTION", "") == "1"


def under_profiler() -> bool:
    """True inside any rocprofv3 run (its launcher always exports ROCPROF_OUTPUT_PATH)."""
    return "ROCPROF_OUTPUT_PATH" in os.environ


FP8_PEAK_CLOCK_MHZ = 2400.0    # the engine clock the 5.0 PFLOP/s dense FP8 peak is quoted at
POWER_SECONDS = 3.0            # wall time of each sustained-clock phase


class PowerSampler:
    """Sustained engine clock and socket power while a workload runs back to
    back.  amdsmi (read-only queries) serves the SMU's metrics, which it
    refreshes about once a second: a host thread polls every 10 ms and keeps
    each refresh (a new energy-counter timestamp) with its engine clock and
    accumulated socket energy.  Refreshes that land inside the phase give the
    clock (median) and, between the first and the last of them, the average
    power (energy delta / SMU time delta).  The amdsmi device is the one whose
    PCI bus matches torch's cuda:0."""

    def __init__(self):
        self.error = None
        try:
            import amdsmi
            import torch
            amdsmi.amdsmi_init()
            props = torch.cuda.get_device_properties(0)
            handles = amdsmi.amdsmi_get_processor_handles()
            mine = [h for h in handles
                    if int(amdsmi.amdsmi_get_gpu_device_bdf(h).split(":")[1], 16) == props.pci_bus_id]
            if len(mine) != 1:
                raise RuntimeError(f"{len(mine)} amdsmi devices on PCI bus {props.pci_bus_id}")
            self.amdsmi, self.h = amdsmi, mine[0]
            self.cap_w = amdsmi.amdsmi_get_power_cap_info(self.h)["power_cap"] / 1e6
        except Exception as e:          # no amdsmi, or no access to the metrics table
            self.error = f"{type(e).__name__}: {e}"

    def run(self, fn, seconds=POWER_SECONDS, sync_every=10):
        """Calls fn() repeatedly for `seconds` (at least 2.5 s, so that two
        metrics refreshes fall inside); returns the median clock, the average
        socket power and the mean wall time per call."""
        if self.error:
            return {"unavailable": self.error}
        import statistics
        import threading
        import torch
        refreshes, stop = [], threading.Event()

        def poll():
            last = None
            while not stop.is_set():
                try:
                    e = self.amdsmi.amdsmi_get_energy_count(self.h)
                    if e["timestamp"] != last:
                        m = self.amdsmi.amdsmi_get_gpu_metrics_info(self.h)
                        refreshes.append((time.perf_counter(), m["current_gfxclk"],
                                          e["energy_accumulator"] * e["counter_resolution"] * 1e-6,
                                          e["timestamp"] * 1e-9))
                        last = e["timestamp"]
                except Exception:
                    pass
                time.sleep(0.01)

        th = threading.Thread(target=poll, daemon=True)
        torch.cuda.synchronize()
        th.start()
        time.sleep(0.05)                # the thread has seen the current refresh
        t0, calls = time.perf_counter(), 0
        while time.perf_counter() - t0 < seconds:
            for _ in range(sync_every):
                fn()
            torch.cuda.synchronize()
            calls += sync_every
        wall = time.perf_counter() - t0
        stop.set()
        th.join(timeout=2.0)            # a metrics query that never returns must not hold the bench line
        refreshes = list(refreshes)
        # refreshes seen after the phase began and before it ended (a refresh
        # is seen within ~10 ms of happening)
        inside = [r for r in refreshes if t0 + 0.02 <= r[0] <= t0 + wall and isinstance(r[1], int)]
        if len(inside) < 2:
            return {"unavailable": f"{len(inside)} metrics refreshes inside the phase"}
        a, b = inside[0], inside[-1]
        return {"gfxclk_mhz": statistics.median(r[1] for r in inside),
                "socket_power_w": round((b[2] - a[2]) / (b[3] - a[3]), 1),
                "power_cap_w": round(self.cap_w, 1), "refreshes": len(inside),
                "seconds": round(wall, 3), "us_per_call": round(wall / calls * 1e6, 2)}


def sustained_clock(step, seconds=POWER_SECONDS):
    """The C3 step and its dX GEMM alone, each back to back for `seconds`: the
    engine clock and socket power they sustain, and the GEMM's rate against the
    dense FP8 peak scaled to that clock."""
    ps = PowerSampler()
    out = {"step": ps.run(step.run, seconds)}
    gemm = ps.run(lambda: step._gemm(step.qdy, step.sdy, step.qw, step.sw, step.dx, M3, K3, N3, None),
                  seconds, sync_every=20)
    if "us_per_call" in gemm:
        tflops = GEMM_FLOP / (gemm["us_per_call"] * 1e-6) / 1e12
        peak = FP8_PEAK_TFLOPS * gemm["gfxclk_mhz"] / FP8_PEAK_CLOCK_MHZ
        gemm.update({"tflops": round(tflops, 1), "peak_at_clock_tflops": round(peak, 1),
                     "frac_at_clock": round(tflops / peak, 4)})
    out["gemm_dx"] = gemm
    return out


def measured_traffic():
    """HBM bytes per dispatch from the committed, copy-calibrated
    FETCH_SIZE + WRITE_SIZE counter passes (lines "traffic <kernel> <bytes>")."""
    out = {}
    if os.path.exists(TRAFFIC_FILE):
        for line in open(TRAFFIC_FILE):
            f = line.split()
            if len(f) == 3 and f[0] == "traffic":
                out[f[1]] = int(f[2])
    return out


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    # the clock ramp after idle is covered by the CLOCK_SETTLE_MS phase in
    # main(), ahead of these warm-up steps
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--norm-iters", type=int, default=200)
    p.add_argument("--only", choices=["step", "norm_quant", "norm_bwd", "gemv", "bwd_bf16",
                                      "block_step", "xent", "decode", "vendor_gemm", "c1", "block_k", "io_floor", "quant_floor",
                                      "gemv_floor"],
                   help="run one secondary workload alone and print its JSON object")
    p.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                   help="only run a plain device copy of MIB MiB (calibrates the FETCH_SIZE / "
                        "WRITE_SIZE counters for the roofline traffic figure) and exit")
    return p.parse_args()


def copy_probe(mib: int) -> None:
    """A plain copy of known size: FETCH_SIZE / WRITE_SIZE of this dispatch
    divided by mib MiB is the counter's scale factor on this GPU."""
    import torch
    src = torch.ones(mib * (1 << 20) // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": mib * (1 << 20)}))


def c3_inputs():
    """Config 3's bf16 inputs (seed 2): x [8192, 2048] ~N(0,1), W [2048, 8192]
    ~N(0, 0.02^2), dY [8192, 8192] ~N(0, 1e-3^2), as bf16 bit patterns from
    numpy's default_rng (RNE from f32)."""
    import numpy as np
    from oracle import bf16 as ob
    rng = np.random.default_rng(2)
    return (ob.randn_bf16(rng, (M3, K3)), ob.randn_bf16(rng, (K3, N3), std=0.02),
            ob.randn_bf16(rng, (M3, N3), std=1e-3))


def host_cpu():
    """(usable host cores, CPU model name)."""
    import os
    cores = len(os.sched_getaffinity(0))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return cores, model


class Step:
    """Config-3 forward + FP8 backward through the C ABI with preallocated buffers."""

    def __init__(self, dev):
        import torch
        import _tglib as L
        self.L, self.lib, self.torch = L, L.lib(), torch
        bf = torch.bfloat16
        # config 3's inputs (seed 2), drawn once on the host; the CPU baseline
        # runs on these same arrays
        self.host = c3_inputs()
        to_dev = lambda u16: torch.from_numpy(u16.view("int16")).view(bf).to(dev)
        self.x, self.w, self.dy = (to_dev(a) for a in self.host)
        u8, f32 = torch.uint8, torch.float32
        e = lambda *s: torch.empty(s, dtype=u8, device=dev)
        f = lambda *s: torch.empty(s, dtype=f32, device=dev)
        # scales K-block-major, (K/128, rows): the layout fp8.block_scaled_matmul's
        # autograd path and the composites keep (tg_quantize_dual*_km, tg_gemm_fp8_nt_km)
        self.qx, self.sx = e(M3, K3), f(K3 // 128, M3)          # x along K
        self.qwt, self.swt = e(N3, K3), f(K3 // 128, N3)        # W.T along K
        self.qdy, self.sdy = e(M3, N3), f(N3 // 128, M3)        # dY along N
        self.qw, self.sw = e(K3, N3), f(N3 // 128, K3)          # W along N
        self.qxt, self.sxt = e(K3, M3), f(M3 // 128, K3)        # X.T along M
        self.qdyt, self.sdyt = e(N3, M3), f(M3 // 128, N3)      # dY.T along M
        self.y = torch.empty((M3, N3), dtype=bf, device=dev)
        self.dx = torch.empty((M3, K3), dtype=bf, device=dev)
        self.dw = torch.empty((K3, N3), dtype=bf, device=dev)
        self.stream = L.stream_of(self.x)
        self.events = []

    def _gemm(self, qa, sa, qb, sb, c, M, N, K, ev):
        L = self.L
        if ev is not None:
            s, e = self.torch.cuda.Event(enable_timing=True), self.torch.cuda.Event(enable_timing=True)
            s.record()
        L.check(self.lib.tg_gemm_fp8_nt_km(L.ptr(qa), L.ptr(sa), L.ptr(qb), L.ptr(sb), 1, L.ptr(c),
                                           L.TG_DTYPE_BF16, M, N, K, 128, self.stream))
        if ev is not None:
            e.record()
            ev.append((s, e))

    def run(self, ev=None):
        L, lib, st, p = self.L, self.lib, self.stream, self.L.ptr
        # forward (fp8.py:66,68,70-78); x.T along M and W along N are the
        # backward's operands, kept from the same reads
        L.check(lib.tg_quantize_dual_pair_km(p(self.x), M3, K3, p(self.qx), p(self.sx), p(self.qxt),
                                             p(self.sxt), p(self.w), K3, N3, p(self.qw), p(self.sw),
                                             p(self.qwt), p(self.swt), 128, st))
        self._gemm(self.qx, self.sx, self.qwt, self.swt, self.y, M3, N3, K3, ev)
        # dY along N (for dX) and dY.T along M (for dW) from one read of dY
        L.check(lib.tg_quantize_dual_km(p(self.dy), M3, N3, 128, p(self.qdy), p(self.sdy), p(self.qdyt),
                                        p(self.sdyt), st))
        # dX = dY . W.T
        self._gemm(self.qdy, self.sdy, self.qw, self.sw, self.dx, M3, K3, N3, ev)
        # dW = X.T . dY
        self._gemm(self.qxt, self.sxt, self.qdyt, self.sdyt, self.dw, K3, N3, M3, ev)


def bench_norm(dev, iters):
    """Config 2 fused RMSNorm -> quantize; mean kernel time over rotating buffer sets."""
    import torch
    import _tglib as L
    lib = L.lib()
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    nsets = 5                                    # 5 x 84 MB > 256 MB Infinity Cache
    xs, ys, qs, ss = [], [], [], []
    for _ in range(nsets):
        x = torch.randn((C2_ROWS, C2_D), generator=g, device=dev)
        mask = torch.rand((C2_ROWS, C2_D), generator=g, device=dev) < 1e-3
        xs.append(torch.where(mask, x * 50, x).to(torch.bfloat16))
        ys.append(torch.empty((C2_ROWS, C2_D), dtype=torch.bfloat16, device=dev))
        qs.append(torch.empty((C2_ROWS, C2_D), dtype=torch.uint8, device=dev))
        ss.append(torch.empty((C2_ROWS, C2_D // 128), dtype=torch.float32, device=dev))
    gamma = (1 + 0.1 * torch.randn((C2_D,), generator=g, device=dev)).to(torch.bfloat16)
    st = L.stream_of(gamma)

    def launch(i):
        k = i % nsets
        L.check(lib.tg_rms_norm_fp8(L.ptr(xs[k]), L.ptr(gamma), L.ptr(ys[k]), L.ptr(qs[k]), L.ptr(ss[k]),
                                    C2_ROWS, C2_D, 1e-6, 128, st))

    for i in range(10):
        launch(i)
    torch.cuda.synchronize()
    # back-to-back launches between one pair of events on the launch stream:
    # the mean launch duration (what the rocprofv3 kernel trace averages)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(iters):
        launch(i)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / iters
    gbps = C2_BYTES / (ms * 1e-3) / 1e9
    return {"workload": "C2 fused RMSNorm+FP8 quant, x bf16 [8,1024,2048], eps 1e-6",
            "us_per_launch": round(ms * 1e3, 3), "bytes_per_launch": C2_BYTES,
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                         "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                         "traffic": measured_traffic().get("rmsnorm_fp8")}}


def bench_io_floor(dev, iters):
    """The I/O floor of config 2's fused norm -> FP8 kernel: libtg_probe.so's
    io_floor_kernel moves the same bytes on the same launch shape with no
    arithmetic (read-only, bf16 copy, config 2's read / write mix, writes only),
    for 1, 2, 4 and 8 rows per wave, timed like `norm_quant` beside the real
    kernel over the same rotating buffer sets."""
    import ctypes
    import torch
    import _tglib as L
    import build as tg_build
    lib = L.lib()
    if not os.path.exists(tg_build.PROBE_LIB):
        raise RuntimeError(f"{tg_build.PROBE_LIB} is missing: run python train-gpt_amd/build.py")
    probe = ctypes.CDLL(tg_build.PROBE_LIB)
    probe.tg_probe_io_floor.restype = ctypes.c_int
    probe.tg_probe_io_floor.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    nsets = 5
    xs = [torch.randn((C2_ROWS, C2_D), generator=g, device=dev).to(torch.bfloat16) for _ in range(nsets)]
    ys = [torch.empty((C2_ROWS, C2_D), dtype=torch.bfloat16, device=dev) for _ in range(nsets)]
    qs = [torch.empty((C2_ROWS, C2_D), dtype=torch.uint8, device=dev) for _ in range(nsets)]
    ss = [torch.empty((C2_ROWS, C2_D // 128), dtype=torch.float32, device=dev) for _ in range(nsets)]
    gamma = torch.ones((C2_D,), dtype=torch.bfloat16, device=dev)
    st = L.stream_of(gamma)
    xb, qb, sb = C2_ROWS * C2_D * 2, C2_ROWS * C2_D, C2_ROWS * (C2_D // 128) * 4
    modes = {0: ("read x", xb), 1: ("read x, write y (bf16 copy)", 2 * xb),
             2: ("read x, write y, q, scales (config 2's mix)", 2 * xb + qb + sb),
             3: ("write y, q, scales", xb + qb + sb)}

    def rate(us, byts):
        gbps = byts / (us * 1e-6) / 1e9
        return {"us_per_launch": round(us, 3), "bytes_per_launch": byts, "GB/s": round(gbps, 1),
                "frac_of_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4)}

    out = {"workload": "I/O floor of C2: rows 8192 x 2048 bf16, the fused norm kernel's access pattern "
                       "without arithmetic (csrc/probe/io_floor.hip)", "modes": []}
    for mode, (what, byts) in modes.items():
        row = {"mode": mode, "traffic": what}
        for rpw in (1, 2, 4, 8):
            def launch(i, mode=mode, rpw=rpw):
                k = i % nsets
                L.check(probe.tg_probe_io_floor(mode, L.ptr(xs[k]), L.ptr(ys[k]), L.ptr(qs[k]), L.ptr(ss[k]),
                                                C2_ROWS, rpw, st))
            row[f"rows_per_wave_{rpw}"] = rate(_mean_launch_us(launch, iters), byts)
        out["modes"].append(row)

    # the same rows pipelined (io_pipe_kernel): two rows' loads in flight per
    # wave, each row's stores one row later, no branches around any access
    probe.tg_probe_io_pipe.restype = ctypes.c_int
    probe.tg_probe_io_pipe.argtypes = probe.tg_probe_io_floor.argtypes
    out["modes_pipelined"] = []
    for mode, (what, byts) in modes.items():
        row = {"mode": mode, "traffic": what}
        for rpw in (2, 4, 8):
            def launch(i, mode=mode, rpw=rpw):
                k = i % nsets
                L.check(probe.tg_probe_io_pipe(mode, L.ptr(xs[k]), L.ptr(ys[k]), L.ptr(qs[k]), L.ptr(ss[k]),
                                               C2_ROWS, rpw, st))
            row[f"rows_per_wave_{rpw}"] = rate(_mean_launch_us(launch, iters), byts)
        out["modes_pipelined"].append(row)

    def norm(i):
        k = i % nsets
        L.check(lib.tg_rms_norm_fp8(L.ptr(xs[k]), L.ptr(gamma), L.ptr(ys[k]), L.ptr(qs[k]), L.ptr(ss[k]),
                                    C2_ROWS, C2_D, 1e-6, 128, st))
    out["rms_norm_fp8_same_run"] = rate(_mean_launch_us(norm, iters), C2_BYTES)
    # the same bf16 copy by torch's own copy kernel, and the mix at 4x the rows
    # (a longer transfer: the launch's fixed ramp-up and drain weigh less)
    out["torch_copy_same_bytes"] = rate(_mean_launch_us(lambda i: ys[i % nsets].copy_(xs[i % nsets]), iters),
                                        2 * xb)
    big = [torch.empty((4 * C2_ROWS, C2_D), dtype=torch.bfloat16, device=dev) for _ in range(2)]
    bigy = [torch.empty_like(b) for b in big]
    bigq = [torch.empty((4 * C2_ROWS, C2_D), dtype=torch.uint8, device=dev) for _ in range(2)]
    bigs = [torch.empty((4 * C2_ROWS, C2_D // 128), dtype=torch.float32, device=dev) for _ in range(2)]
    for b in big:
        b.normal_()

    def mix4(i):
        k = i % 2
        L.check(probe.tg_probe_io_floor(2, L.ptr(big[k]), L.ptr(bigy[k]), L.ptr(bigq[k]), L.ptr(bigs[k]),
                                        4 * C2_ROWS, 2, st))
    out["mix_at_4x_rows"] = rate(_mean_launch_us(mix4, max(iters // 4, 10)), 4 * (2 * xb + qb + sb))
    mix = [r for r in out["modes"] + out["modes_pipelined"] if r["mode"] == 2]
    best = max(m[k]["GB/s"] for m in mix for k in m if k.startswith("rows_per_wave"))
    out["norm_vs_best_mix_floor"] = round(out["rms_norm_fp8_same_run"]["GB/s"] / best, 4)
    # A different access pattern for the same bytes (csrc/probe/io_floor.hip's
    # io_stream_kernel): x as a plain stream of 16-byte units in address order,
    # y / q / scale stores per unit, no rows; grid and loads in flight swept.
    probe.tg_probe_io_stream.restype = ctypes.c_int
    probe.tg_probe_io_stream.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    units = C2_ROWS * C2_D // 8
    stream_rows = []
    for grid in (256, 512, 1024, 2048, 4096, 8192):
        for unroll in (2, 4, 8):
            def launch(i, grid=grid, unroll=unroll):
                k = i % nsets
                L.check(probe.tg_probe_io_stream(L.ptr(xs[k]), L.ptr(ys[k]), L.ptr(qs[k]), L.ptr(ss[k]), units,
                                                 grid, unroll, st))
            r = rate(_mean_launch_us(launch, iters), 2 * xb + qb + sb)
            r.update({"grid": grid, "units_in_flight_per_lane": unroll})
            stream_rows.append(r)
    out["stream_pattern_same_bytes"] = stream_rows
    best_stream = max(r["GB/s"] for r in stream_rows)
    out["best_stream_vs_best_row_pattern"] = round(best_stream / best, 4)
    out["norm_vs_best_of_both_patterns"] = round(out["rms_norm_fp8_same_run"]["GB/s"] / max(best, best_stream), 4)
    return out


def bench_quant_floor(dev, iters):
    """The I/O floor of config 3's dual quantizers: libtg_probe.so's
    quant_floor (csrc/probe/quant_floor.hip) runs the product's
    quant_dual_kernel with its arithmetic taken out -- the same loads, LDS
    traffic and stores on the same grid and tile order -- with and without the
    K-block-major scale stores, timed beside tg_quantize_dual_km (dY 8192 x
    8192) and tg_quantize_dual_pair_km (x 8192 x 2048 + W 2048 x 8192) on the
    step's buffers (three rotating input sets, one output set, as the step
    rewrites its quantized operands), interleaved, median of 7 rounds."""
    import ctypes
    import statistics
    import torch
    import _tglib as L
    import build as tg_build
    lib = L.lib()
    if not os.path.exists(tg_build.PROBE_LIB):
        raise RuntimeError(f"{tg_build.PROBE_LIB} is missing: run python train-gpt_amd/build.py")
    probe = ctypes.CDLL(tg_build.PROBE_LIB)
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    probe.tg_probe_quant_floor.restype = ctypes.c_int
    probe.tg_probe_quant_floor.argtypes = [ctypes.c_int, vp, i64, i64, vp, vp, vp, vp, vp, i64, i64, vp, vp,
                                           vp, vp, vp]
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    nsets = 3                                    # 3 x 134 MB of dY > 256 MB Infinity Cache

    def outs(r, c):
        return (torch.empty((r, c), dtype=torch.uint8, device=dev),
                torch.empty((c // 128, r), dtype=torch.float32, device=dev),
                torch.empty((c, r), dtype=torch.uint8, device=dev),
                torch.empty((r // 128, c), dtype=torch.float32, device=dev))
    dys = [(torch.randn((M3, N3), generator=g, device=dev) * 1e-3).to(torch.bfloat16) for _ in range(nsets)]
    xs = [torch.randn((M3, K3), generator=g, device=dev).to(torch.bfloat16) for _ in range(nsets)]
    ws = [(torch.randn((K3, N3), generator=g, device=dev) * 0.02).to(torch.bfloat16) for _ in range(nsets)]
    # one output set, as in the C3 step (the step rewrites the same quantized
    # operands every step; only the inputs are new)
    ody, ox, ow = [outs(M3, N3)] * nsets, [outs(M3, K3)] * nsets, [outs(K3, N3)] * nsets
    st = L.stream_of(dys[0])
    P = L.ptr

    def per_elem(r, c):          # 2 B read + (1 + 4/128) B written twice
        return r * c * 2 + 2 * (r * c + r * c // 128 * 4)
    dy_bytes, pair_bytes = per_elem(M3, N3), per_elem(M3, K3) + per_elem(K3, N3)

    def dy_prod(i):
        k = i % nsets
        L.check(lib.tg_quantize_dual_km(P(dys[k]), M3, N3, 128, *[P(t) for t in ody[k]], st))

    def dy_probe(mode):
        def f(i):
            k = i % nsets
            L.check(probe.tg_probe_quant_floor(mode, P(dys[k]), M3, N3, *[P(t) for t in ody[k]],
                                               None, 0, 0, None, None, None, None, st))
        return f

    def pair_prod(i):
        k = i % nsets
        L.check(lib.tg_quantize_dual_pair_km(P(xs[k]), M3, K3, *[P(t) for t in ox[k]], P(ws[k]), K3, N3,
                                             *[P(t) for t in ow[k]], 128, st))

    def pair_probe(mode):
        def f(i):
            k = i % nsets
            L.check(probe.tg_probe_quant_floor(mode, P(xs[k]), M3, K3, *[P(t) for t in ox[k]], P(ws[k]), K3, N3,
                                               *[P(t) for t in ow[k]], st))
        return f
    cases = {"dY 8192 x 8192": (dy_bytes, {"product tg_quantize_dual_km": dy_prod, "io_floor_with_scales":
                                           dy_probe(0), "io_floor_no_scales": dy_probe(1)}),
             "x 8192 x 2048 + W 2048 x 8192": (pair_bytes, {"product tg_quantize_dual_pair_km": pair_prod,
                                                            "io_floor_with_scales": pair_probe(0),
                                                            "io_floor_no_scales": pair_probe(1)})}
    res = {}
    for rnd in range(7):
        for cname, (byts, fns) in cases.items():
            for name, f in fns.items():
                res.setdefault((cname, name), []).append(_mean_launch_us(f, iters, warm=3))
    out = {"workload": "config 3's dual quantizers (dY; x + W pair) beside the same kernel without arithmetic "
                       "(csrc/probe/quant_floor.hip), 3 rotating input sets and one output set (as in the "
                       "C3 step), median of 7 interleaved rounds", "cases": []}
    for cname, (byts, fns) in cases.items():
        row = {"case": cname, "bytes_per_launch": byts}
        for name in fns:
            us = statistics.median(res[(cname, name)])
            gbps = byts / (us * 1e-6) / 1e9
            row[name] = {"us_per_launch": round(us, 2), "GB/s": round(gbps, 1),
                         "frac_of_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4)}
        prod = [v for k, v in row.items() if k.startswith("product")][0]
        row["product_vs_floor_with_scales"] = round(row["io_floor_with_scales"]["us_per_launch"] /
                                                    prod["us_per_launch"], 4)
        out["cases"].append(row)
    return out


def bench_gemv_floor(dev, iters):
    """The streaming floor of the direct decode GEMV at the reference decode
    weights (8 activation rows): libtg_probe.so's gemv_stream_kernel issues
    the same weight loads on the same grid with no arithmetic, with and
    without every workgroup's read of the x rows, with cached and with
    non-temporal loads; tg_gemv_fp8 runs beside it on the same weights.
    Weight copies rotate over > 800 MB, so HBM serves them."""
    import ctypes
    import torch
    import _tglib as L
    import build as tg_build
    lib = L.lib()
    if not os.path.exists(tg_build.PROBE_LIB):
        raise RuntimeError(f"{tg_build.PROBE_LIB} is missing: run python train-gpt_amd/build.py")
    probe = ctypes.CDLL(tg_build.PROBE_LIB)
    probe.tg_probe_gemv_stream.restype = ctypes.c_int
    probe.tg_probe_gemv_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                           ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_void_p]
    M = 8
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    out = {"workload": "reference decode weights (d 2304, d_ff 9216) at 8 rows: the direct GEMV's loads without "
                       "arithmetic (csrc/probe/gemv_stream.hip) beside tg_gemv_fp8", "cus": cus, "shapes": []}
    # clock settle: ~50 ms of launches before the first timed one
    wz = torch.zeros((6912, 2304), dtype=torch.uint8, device=dev)
    sz = torch.empty(432 * 512, dtype=torch.int32, device=dev)
    t_settle = time.perf_counter()
    while (time.perf_counter() - t_settle) < 0.05:
        for _ in range(20):
            L.check(probe.tg_probe_gemv_stream(L.ptr(wz), 6912, 2304, None, 0, L.ptr(sz), 432, 1,
                                               L.stream_of(wz)))
        torch.cuda.synchronize()
    del wz, sz
    for name, N, K in (("wo", 2304, 2304), ("qkv", 6912, 2304), ("w_up", 9216, 2304), ("w_down", 2304, 9216)):
        nset = int(800e6 // (N * K)) + 1
        ws = [torch.randint(0, 126, (N, K), generator=g, device=dev, dtype=torch.uint8) for _ in range(nset)]
        wsc = [torch.rand((N + 127) // 128, K // 128, generator=g, device=dev) * 1e-2 for _ in range(nset)]
        xq = torch.randint(0, 126, (M, K), generator=g, device=dev, dtype=torch.uint8)
        xs = torch.rand(M, K // 128, generator=g, device=dev)
        o = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        nrb = (N + 15) // 16
        grid = min(nrb, 2 * cus)
        sink = torch.empty(grid * 512, dtype=torch.int32, device=dev)
        st = L.stream_of(o)
        wbytes = N * K
        row = {"weight": name, "N": N, "K": K, "weight_bytes": wbytes, "grid": grid}

        def rate(us):
            return {"us_per_launch": round(us, 3), "weight_GB/s": round(wbytes / (us * 1e-6) / 1e9, 1)}

        def gemv(i):
            L.check(lib.tg_gemv_fp8(L.ptr(xq), L.ptr(xs), L.ptr(ws[i % nset]), L.ptr(wsc[i % nset]), 128, L.ptr(o),
                                    M, N, K, 128, st))
        # two passes over the four launches; the second pass is reported (the
        # first pass over freshly allocated copies runs slower)
        for _ in range(2):
            for label, xb, cached in (("loads_cached", 0, 1), ("loads_cached_with_x", M * K, 1),
                                      ("loads_nontemporal_with_x", M * K, 0)):
                def launch(i, xb=xb, cached=cached):
                    L.check(probe.tg_probe_gemv_stream(L.ptr(ws[i % nset]), N, K, L.ptr(xq), xb, L.ptr(sink),
                                                       grid, cached, st))
                row[label] = rate(_mean_launch_us(launch, iters))
            row["tg_gemv_fp8"] = rate(_mean_launch_us(gemv, iters))
        out["shapes"].append(row)
        del ws, wsc
        torch.cuda.empty_cache()
    # C5 (14336 x 4096, 128 x 128 scales) on the staged GEMV: the product at 8
    # and 32 rows beside gemv_staged_kernel, its weight stream with no MFMAs,
    # x fragments or reduction (weight only, and with the 8-row x copy)
    probe.tg_probe_gemv_staged.restype = ctypes.c_int
    probe.tg_probe_gemv_staged.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int64,
                                           ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                           ctypes.c_int, ctypes.c_void_p]
    N, K = C5_N, C5_K
    nset = int(800e6 // (N * K)) + 1
    ws = [torch.randint(0, 126, (N, K), generator=g, device=dev, dtype=torch.uint8) for _ in range(nset)]
    wsc = [torch.rand((N + 127) // 128, K // 128, generator=g, device=dev) * 1e-2 for _ in range(nset)]
    groups = (N + 7) // 8
    grid = max(min(cus, groups), (groups + 7) // 8)
    sink = torch.empty(grid * 512, dtype=torch.int32, device=dev)
    st = L.stream_of(sink)
    wbytes = N * K
    c5 = {"weight": "C5", "N": N, "K": K, "weight_bytes": wbytes, "grid": grid}

    def rate5(us):
        return {"us_per_launch": round(us, 3), "weight_GB/s": round(wbytes / (us * 1e-6) / 1e9, 1)}
    xq8 = torch.randint(0, 126, (8, K), generator=g, device=dev, dtype=torch.uint8)
    for _ in range(2):   # the second pass is reported (first touches of the copies run slower)
        for label, xb in (("staged_loads", 0), ("staged_loads_with_x_copy_8_rows", 8 * K)):
            def launch(i, xb=xb):
                L.check(probe.tg_probe_gemv_staged(L.ptr(ws[i % nset]), L.ptr(wsc[i % nset]), 128, N, K,
                                                   L.ptr(xq8), xb, L.ptr(sink), grid, st))
            c5[label] = rate5(_mean_launch_us(launch, iters))
        for M in (8, 32):
            xq = torch.randint(0, 126, (M, K), generator=g, device=dev, dtype=torch.uint8)
            xs = torch.rand(M, K // 128, generator=g, device=dev)
            o = torch.empty(M, N, dtype=torch.bfloat16, device=dev)

            def gemv(i, xq=xq, xs=xs, o=o, M=M):
                L.check(lib.tg_gemv_fp8(L.ptr(xq), L.ptr(xs), L.ptr(ws[i % nset]), L.ptr(wsc[i % nset]), 128,
                                        L.ptr(o), M, N, K, 128, st))
            c5[f"tg_gemv_fp8_M{M}"] = rate5(_mean_launch_us(gemv, iters))
    out["c5_staged"] = c5
    del ws, wsc
    torch.cuda.empty_cache()
    return out


def _mean_launch_us(launch, iters, warm=5):
    """Mean duration of back-to-back launches between one pair of events on
    the launch stream (what the rocprofv3 kernel trace averages)."""
    import torch
    for i in range(warm):
        launch(i)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(iters):
        launch(i)
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / iters * 1e3


def bench_norm_bwd(dev, iters):
    """rms_norm backward at config 2's shape (row kernel + column reduce)."""
    import torch
    import _tglib as L
    lib = L.lib()
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    nsets = 3                                    # 3 x 100 MB > 256 MB Infinity Cache
    bf = torch.bfloat16
    xs = [torch.randn((C2_ROWS, C2_D), generator=g, device=dev).to(bf) for _ in range(nsets)]
    dys = [(torch.randn((C2_ROWS, C2_D), generator=g, device=dev) * 1e-2).to(bf) for _ in range(nsets)]
    dxs = [torch.empty((C2_ROWS, C2_D), dtype=bf, device=dev) for _ in range(nsets)]
    gamma = (1 + 0.1 * torch.randn((C2_D,), generator=g, device=dev)).to(bf)
    dgamma = torch.empty((C2_D,), dtype=bf, device=dev)
    wsb = lib.tg_rms_norm_bwd_workspace(C2_ROWS, C2_D)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    st = L.stream_of(gamma)

    def launch(i):
        k = i % nsets
        L.check(lib.tg_rms_norm_bwd(L.ptr(xs[k]), L.ptr(gamma), L.ptr(dys[k]), L.ptr(dxs[k]),
                                    L.ptr(dgamma), C2_ROWS, C2_D, 1e-6, L.ptr(ws), wsb, st))
    us = _mean_launch_us(launch, iters)
    gbps = C2_BWD_BYTES / (us * 1e-6) / 1e9
    out = {"workload": "rms_norm backward (kernels.py:104-118), x/dy bf16 [8,1024,2048]",
           "us_per_call": round(us, 3), "bytes_per_call": C2_BWD_BYTES,
           "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                        "traffic": measured_traffic().get("rmsnorm_bwd")}}
    # the row kernel's I/O with no arithmetic (libtg_probe.so's io_bwd_kernel,
    # same row walk), on the product's grid (256) and larger ones
    import ctypes
    import build as tg_build
    if os.path.exists(tg_build.PROBE_LIB):
        probe = ctypes.CDLL(tg_build.PROBE_LIB)
        probe.tg_probe_io_bwd.restype = ctypes.c_int
        probe.tg_probe_io_bwd.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                                                  ctypes.c_void_p]
        part = torch.empty(4096 * C2_D, dtype=torch.float32, device=dev)
        floor = {}
        for grid, depth in ((256, 2), (512, 2), (1024, 2), (2048, 2), (256, 3), (256, 4), (512, 3)):
            def pl(i, grid=grid, depth=depth):
                k = i % nsets
                L.check(probe.tg_probe_io_bwd(L.ptr(xs[k]), L.ptr(dys[k]), L.ptr(dxs[k]), L.ptr(part), C2_ROWS,
                                              grid, depth, st))
            pus = _mean_launch_us(pl, iters)
            byts = 3 * C2_ROWS * C2_D * 2 + grid * C2_D * 4
            floor[f"grid_{grid}_rows_in_flight_{depth}"] = {"us_per_launch": round(pus, 3), "bytes_per_launch": byts,
                                                            "GB/s": round(byts / (pus * 1e-6) / 1e9, 1)}
        out["row_kernel_io_floor"] = floor
    return out


def bench_gemv(dev, iters):
    """Config 5: decode GEMV on a pre-quantized W (128x128 scales), M in {1, 8, 32};
    M = 1 on the VALU kernel (tg_gemv_fp8_rowdot, what fp8_gemv picks), with the
    MFMA kernel's time beside it."""
    import torch
    import _tglib as L
    lib = L.lib()
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    nsets = 5                                    # 5 x 58.7 MB > 256 MB Infinity Cache
    wq, ws = [], []
    for _ in range(nsets):
        w = (torch.randn((C5_K, C5_N), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        q = torch.empty((C5_N, C5_K), dtype=torch.uint8, device=dev)
        s = torch.empty(((C5_N + 127) // 128, C5_K // 128), dtype=torch.float32, device=dev)
        L.check(lib.tg_quantize_weight_128x128(L.ptr(w), C5_K, C5_N, L.ptr(q), L.ptr(s), L.stream_of(w)))
        wq.append(q)
        ws.append(s)
        del w
    out = []
    for M in (1, 8, 32):
        x = torch.randn((M, C5_K), generator=g, device=dev).to(torch.bfloat16)
        xq = torch.empty((M, C5_K), dtype=torch.uint8, device=dev)
        xs = torch.empty((M, C5_K // 128), dtype=torch.float32, device=dev)
        y = torch.empty((M, C5_N), dtype=torch.bfloat16, device=dev)
        st = L.stream_of(x)
        L.check(lib.tg_quantize_rows(L.ptr(x), L.TG_DTYPE_BF16, M, C5_K, 128, L.ptr(xq), L.ptr(xs), st))

        def launcher(fn):
            def launch(i):
                k = i % nsets
                L.check(fn(L.ptr(xq), L.ptr(xs), L.ptr(wq[k]), L.ptr(ws[k]), 128, L.ptr(y),
                           M, C5_N, C5_K, 128, st))
            return launch
        # what fp8.fp8_gemv picks: the VALU kernel for 1-2 rows, the MFMA one above
        rowdot = M <= 2
        fn = lib.tg_gemv_fp8_rowdot if rowdot else lib.tg_gemv_fp8
        us = _mean_launch_us(launcher(fn), iters)
        us_mfma = _mean_launch_us(launcher(lib.tg_gemv_fp8), iters) if rowdot else us

        def step(i):          # x quantization + GEMV, the decode step's FP8 matmul
            L.check(lib.tg_quantize_rows(L.ptr(x), L.TG_DTYPE_BF16, M, C5_K, 128, L.ptr(xq), L.ptr(xs), st))
            launcher(fn)(i)
        us_step = _mean_launch_us(step, iters)
        byts = C5_N * C5_K + ws[0].numel() * 4 + M * C5_K + M * (C5_K // 128) * 4 + 2 * M * C5_N
        gbps = byts / (us * 1e-6) / 1e9
        tkey = "gemv_rowdot_m1" if rowdot else ("gemv_fp8_m16" if M <= 16 else "gemv_fp8_m32")
        out.append({"M": M, "kernel": "gemv_rowdot_kernel" if rowdot else "gemv_fp8_kernel",
                    "us_per_launch": round(us, 3), "us_mfma_gemv": round(us_mfma, 3),
                    "us_quant_plus_gemv": round(us_step, 3), "bytes_per_launch": byts,
                    "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                                 "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                                 "traffic": measured_traffic().get(tkey)}})
    return {"workload": "C5 decode GEMV, W e4m3 [14336, 4096] + 128x128 scales (pre-quantized), "
                        "x quantized 1x128", "by_M": out}


def bench_bwd_bf16(dev, iters):
    """The reference's straight-through bf16 backward at config 3 (2 GEMMs per call)."""
    import torch
    import _tglib as L
    lib = L.lib()
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    bf = torch.bfloat16
    x = torch.randn((M3, K3), generator=g, device=dev).to(bf)
    w = (torch.randn((K3, N3), generator=g, device=dev) * 0.02).to(bf)
    dy = (torch.randn((M3, N3), generator=g, device=dev) * 1e-3).to(bf)
    dx = torch.empty((M3, K3), dtype=bf, device=dev)
    dw = torch.empty((K3, N3), dtype=bf, device=dev)
    wsb = lib.tg_block_scaled_matmul_bwd_bf16_workspace(M3, N3, K3)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    st = L.stream_of(x)
    B = L.TG_DTYPE_BF16

    def launch(i):
        L.check(lib.tg_block_scaled_matmul_bwd_bf16(L.ptr(x), B, L.ptr(w), B, L.ptr(dy), B, L.ptr(dx),
                                                     L.ptr(dw), M3, N3, K3, L.ptr(ws), wsb, st))
    us = _mean_launch_us(launch, iters, warm=3)
    tf = 2 * GEMM_FLOP / (us * 1e-6) / 1e12
    return {"workload": "C3 straight-through bf16 backward (fp8.py:85-98): dX = dY . W.T, "
                        "dW = X.T . dY (read in place by the contraction-major kernel)",
            "us_per_call": round(us, 2), "tflops": round(tf, 1),
            "frac_of_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)}


def bench_block(dev, steps=5, warm=3):
    """Config 4: one decoder block training step (block.py), FP8 path vs the
    same block with bf16 linears; wall time per step after a synchronize."""
    import torch
    import block
    cfg = block.C4
    params = block.init_params(cfg, dev)
    ids, tgt = block.random_batch(cfg, dev)
    out = {"workload": "C4 decoder block fwd+bwd: d 2048, 16x128 heads, MLP 8192 GELU, 4 x 2048 tokens, "
                       "vocab 50304 (bf16 logits), CE loss; FP8 linears + HIP norms",
           "flop_per_step": block.flops_per_step(cfg)}
    for impl in ("fp8", "bf16"):
        for _ in range(warm):
            block.step_grads(params, ids, tgt, cfg, impl)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            loss, _ = block.step_grads(params, ids, tgt, cfg, impl)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        out[impl] = {"ms_per_step": round(dt * 1e3, 3),
                     "tokens_per_s": round(cfg.batch * cfg.seq_len / dt, 1),
                     "loss": round(float(loss), 6)}
    return out


def bench_vendor_gemm(dev, iters):
    """Context for the GEMM roofline: this library's block-scaled FP8 GEMM and
    bf16 GEMM beside the vendor library's (hipBLASLt through torch) plain FP8
    GEMM (one scale per tensor, no block promotion) and bf16 GEMM at the three
    C3 shapes, each timed alone (20 launches after 5 warm-ups)."""
    import torch
    import _tglib as L
    lib = L.lib()
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    bf = torch.bfloat16

    def timed(f):
        for _ in range(5):
            f()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(iters):
            f()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / iters * 1e3

    out = {}
    for name, (M, N, K) in (("Y", (M3, N3, K3)), ("dX", (M3, K3, N3)), ("dW", (K3, N3, M3))):
        a = torch.randn((M, K), generator=g, device=dev).to(bf)
        b = torch.randn((N, K), generator=g, device=dev).to(bf)
        st = L.stream_of(a)
        qa = torch.empty((M, K), dtype=torch.uint8, device=dev)
        sa = torch.empty((M, K // 128), dtype=torch.float32, device=dev)
        qb = torch.empty((N, K), dtype=torch.uint8, device=dev)
        sb = torch.empty((N, K // 128), dtype=torch.float32, device=dev)
        L.check(lib.tg_quantize_rows(L.ptr(a), L.TG_DTYPE_BF16, M, K, 128, L.ptr(qa), L.ptr(sa), st))
        L.check(lib.tg_quantize_rows(L.ptr(b), L.TG_DTYPE_BF16, N, K, 128, L.ptr(qb), L.ptr(sb), st))
        c = torch.empty((M, N), dtype=bf, device=dev)
        flop = 2.0 * M * N * K
        # the K-block-major scale layout the C3 step and the autograd path run on
        sa_km, sb_km = sa.t().contiguous(), sb.t().contiguous()
        t_ours = timed(lambda: L.check(lib.tg_gemm_fp8_nt_km(L.ptr(qa), L.ptr(sa_km), L.ptr(qb), L.ptr(sb_km), 1,
                                                             L.ptr(c), L.TG_DTYPE_BF16, M, N, K, 128, st)))
        t_ours_bf16 = timed(lambda: L.check(lib.tg_gemm_bf16_nt(L.ptr(a), L.ptr(b), L.ptr(c), M, N, K, st)))
        a8, b8 = a.to(torch.float8_e4m3fn), b.to(torch.float8_e4m3fn)
        one = torch.tensor(1.0, device=dev)
        t_vendor = timed(lambda: torch._scaled_mm(a8, b8.t(), scale_a=one, scale_b=one, out_dtype=bf))
        t_vendor_bf16 = timed(lambda: a @ b.t())
        out[name] = {"M": M, "N": N, "K": K,
                     "block_scaled_fp8_tflops": round(flop / t_ours / 1e6, 1),
                     "vendor_plain_fp8_tflops": round(flop / t_vendor / 1e6, 1),
                     "bf16_tflops": round(flop / t_ours_bf16 / 1e6, 1),
                     "vendor_bf16_tflops": round(flop / t_vendor_bf16 / 1e6, 1)}
    return {"workload": "C3 GEMM shapes: tg_gemm_fp8_nt_km (1x128 block scales, K-block-major) and tg_gemm_bf16_nt "
                        "against "
                        "torch._scaled_mm (per-tensor scales) and torch bf16 matmul (hipBLASLt)",
            "by_gemm": out}


def _dequant(q, s):
    """e4m3 bytes (R, C) uint8 and 1x128 scales (R, C/128) f32 -> f32 (R, C)."""
    import torch
    return q.view(torch.float8_e4m3fn).float() * s.repeat_interleave(128, dim=1)


def _dequant_tiles(q, s, n):
    """f32 values of a weight quantized with one scale per 128x128 tile:
    q (N, K) e4m3 bytes, s (ceil(N/128), K/128)."""
    import torch
    full = s.repeat_interleave(128, dim=0)[:n].repeat_interleave(128, dim=1)
    return q.view(torch.float8_e4m3fn).float() * full


def _maxrel(a, b):
    d = (a.float() - b.float()).abs().max()
    return round(float(d / b.float().abs().max().clamp_min(1e-30)), 6)


def step_accuracy(step, rows=256):
    """Error of the step's three FP8 GEMM outputs on their first `rows` rows,
    max-abs-normalised, against the f32 product of the same dequantized bytes
    (the parity bar) and against a bf16 matmul of the unquantized operands
    (f32 accumulation: the error FP8 adds), both computed by torch on the GPU
    outside the timed region."""
    import torch
    r = rows
    xf, wf, dyf = step.x.float(), step.w.float(), step.dy.float()
    out = {"rows_checked": r}
    ref = _dequant(step.qx[:r], step.sx.t()[:r]) @ _dequant(step.qwt, step.swt.t()).t()
    out["y_vs_dequant_f32"] = _maxrel(step.y[:r], ref)
    out["y_vs_bf16_matmul"] = _maxrel(step.y[:r], xf[:r] @ wf)
    ref = _dequant(step.qdy[:r], step.sdy.t()[:r]) @ _dequant(step.qw, step.sw.t()).t()
    out["dx_vs_dequant_f32"] = _maxrel(step.dx[:r], ref)
    out["dx_vs_bf16_matmul"] = _maxrel(step.dx[:r], dyf[:r] @ wf.t())
    ref = _dequant(step.qxt[:r], step.sxt.t()[:r]) @ _dequant(step.qdyt, step.sdyt.t()).t()
    out["dw_vs_dequant_f32"] = _maxrel(step.dw[:r], ref)
    out["dw_vs_bf16_matmul"] = _maxrel(step.dw[:r], xf.t()[:r] @ dyf)
    del xf, wf, dyf, ref
    torch.cuda.empty_cache()
    return out


def bench_block_k(dev, iters):
    """The C3 forward (tg_block_scaled_matmul, x[8192,2048] . W[2048,8192]
    with both quantizations) at block sizes other than 128 (fp8.py:30-36 takes
    any block_k dividing K): 256 runs the tuned GEMM on repeated scales, 64 on
    zero-filled 128-byte slots (twice the MFMA work)."""
    import torch
    import _tglib as L
    lib = L.lib()
    M, K, N = 8192, 2048, 8192
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    x = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn((K, N), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    st = L.stream_of(x)
    out = {"workload": "C3 block_scaled_matmul forward, x[8192,2048] W[2048,8192] bf16, quantization included"}
    for bk in (128, 64, 256):
        ws_bytes = lib.tg_block_scaled_matmul_workspace(M, N, K, bk)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)

        def fwd(i, bk=bk, ws=ws, ws_bytes=ws_bytes):
            L.check(lib.tg_block_scaled_matmul(L.ptr(x), L.ptr(w), L.ptr(y), M, N, K, bk, L.ptr(ws),
                                               ws_bytes, st))
        us = _mean_launch_us(fwd, iters)
        out[f"block_k_{bk}"] = {"us_per_call": round(us, 2), "tflops": round(2.0 * M * N * K / (us * 1e-6) / 1e12, 1)}
        del ws
    return out


def bench_c1(dev, iters):
    """Config 1: the forward block_scaled_matmul at x[2048,768] . W[768,3072]
    (tg_block_scaled_matmul: both quantizations + the GEMM), and the GEMM alone
    on the quantized operands; launch-bound at this size (1.9 us at peak)."""
    import torch
    import _tglib as L
    lib = L.lib()
    M, K, N = 2048, 768, 3072
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    x = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn((K, N), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    st = L.stream_of(x)
    ws_bytes = lib.tg_block_scaled_matmul_workspace(M, N, K, 128)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)

    def fwd(i):
        L.check(lib.tg_block_scaled_matmul(L.ptr(x), L.ptr(w), L.ptr(y), M, N, K, 128, L.ptr(ws),
                                           ws_bytes, st))
    us = _mean_launch_us(fwd, iters)
    qx = torch.empty((M, K), dtype=torch.uint8, device=dev)
    sx = torch.empty((M, K // 128), dtype=torch.float32, device=dev)
    qwt = torch.empty((N, K), dtype=torch.uint8, device=dev)
    swt = torch.empty((N, K // 128), dtype=torch.float32, device=dev)
    L.check(lib.tg_quantize_rows(L.ptr(x), L.TG_DTYPE_BF16, M, K, 128, L.ptr(qx), L.ptr(sx), st))
    L.check(lib.tg_quantize_cols(L.ptr(w), L.TG_DTYPE_BF16, K, N, 128, L.ptr(qwt), L.ptr(swt), st))
    y2 = torch.empty_like(y)

    def gemm(i):
        L.check(lib.tg_gemm_fp8_nt(L.ptr(qx), L.ptr(sx), L.ptr(qwt), L.ptr(swt), 1, L.ptr(y2),
                                   L.TG_DTYPE_BF16, M, N, K, 128, st))
    us_gemm = _mean_launch_us(gemm, iters)
    flop = 2.0 * M * N * K
    ref = _dequant(qx, sx) @ _dequant(qwt, swt).t()
    # the config's literal wording: one scale per 128x128 tile of W
    qw8 = torch.empty((N, K), dtype=torch.uint8, device=dev)
    sw8 = torch.empty(((N + 127) // 128, K // 128), dtype=torch.float32, device=dev)
    y8 = torch.empty_like(y)

    def fwd_128x128(i):
        L.check(lib.tg_quantize_rows(L.ptr(x), L.TG_DTYPE_BF16, M, K, 128, L.ptr(qx), L.ptr(sx), st))
        L.check(lib.tg_quantize_weight_128x128(L.ptr(w), K, N, L.ptr(qw8), L.ptr(sw8), st))
        L.check(lib.tg_gemm_fp8_nt(L.ptr(qx), L.ptr(sx), L.ptr(qw8), L.ptr(sw8), 128, L.ptr(y8),
                                   L.TG_DTYPE_BF16, M, N, K, 128, st))

    def gemm_128x128(i):
        L.check(lib.tg_gemm_fp8_nt(L.ptr(qx), L.ptr(sx), L.ptr(qw8), L.ptr(sw8), 128, L.ptr(y8),
                                   L.TG_DTYPE_BF16, M, N, K, 128, st))
    us8 = _mean_launch_us(fwd_128x128, iters)
    us8_gemm = _mean_launch_us(gemm_128x128, iters)
    ref8 = _dequant(qx, sx) @ (_dequant_tiles(qw8, sw8, N)).t()
    return {"workload": "C1 block_scaled_matmul forward, x[2048,768] bf16, W[768,3072] bf16, 1x128 scales",
            "us_per_call": round(us, 3), "tflops_with_quantization": round(flop / us / 1e6, 1),
            "us_gemm": round(us_gemm, 3), "tflops_gemm": round(flop / us_gemm / 1e6, 1),
            "y_vs_dequant_f32": _maxrel(y, ref),
            "y_vs_bf16_matmul": _maxrel(y, x.float() @ w.float()),
            "same_bits_composite_vs_gemm": bool(torch.equal(y.view(torch.int16), y2.view(torch.int16))),
            "w_scales_128x128": {
                "us_per_call": round(us8, 3), "tflops_with_quantization": round(flop / us8 / 1e6, 1),
                "us_gemm": round(us8_gemm, 3), "tflops_gemm": round(flop / us8_gemm / 1e6, 1),
                "y_vs_dequant_f32": _maxrel(y8, ref8),
                "y_vs_bf16_matmul": _maxrel(y8, x.float() @ w.float())}}


def bench_xent(dev, iters):
    """Config 4's head: tg_logit_cap_xent_fwd / _bwd on bf16 logits [8192, 50304]
    (824 MB, larger than the Infinity Cache, so one buffer set)."""
    import torch
    import _tglib as L
    lib = L.lib()
    R, V, cap = 4 * 2048, 50304, 15.0
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    logits = (torch.randn((R, V), generator=g, device=dev) * 3).to(torch.bfloat16)
    tgt = torch.randint(0, V, (R,), generator=g, device=dev)
    loss = torch.empty(R, dtype=torch.float32, device=dev)
    lse = torch.empty(R, dtype=torch.float32, device=dev)
    one = torch.ones(1, dtype=torch.float32, device=dev)
    dl = torch.empty_like(logits)
    st = L.stream_of(logits)

    def fwd(i):
        L.check(lib.tg_logit_cap_xent_fwd(L.ptr(logits), L.ptr(tgt), R, V, cap, L.ptr(loss), L.ptr(lse), st))

    def bwd(i):
        L.check(lib.tg_logit_cap_xent_bwd(L.ptr(logits), L.ptr(tgt), L.ptr(lse), L.ptr(one), 1.0 / R,
                                          None, R, V, cap, L.ptr(dl), st))
    n = max(iters // 10, 5)
    out = {"workload": "C4 head: logit cap 15 + cross entropy, bf16 logits [8192, 50304], f32 loss, "
                       "bf16 dlogits"}
    for name, fn, byts in (("fwd", fwd, R * V * 2 + R * 16), ("bwd", bwd, 2 * R * V * 2 + R * 12)):
        us = _mean_launch_us(fn, n, warm=2)
        gbps = byts / (us * 1e-6) / 1e9
        out[name] = {"us_per_launch": round(us, 2), "bytes_per_launch": byts,
                     "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                                  "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                                  "traffic": measured_traffic().get("xent_" + name)}}
    return out


def decode_weight_bytes(cfg):
    """HBM bytes of the kept FP8 weights one decode step reads: e4m3 bytes plus
    128x128 fp32 scales of the six linears per layer and of the unembedding."""
    d, h, f, V, L = cfg.d_model, cfg.n_heads * cfg.head_dim, cfg.d_ff, cfg.vocab_size, cfg.n_layers
    wb = lambda K, N: K * N + ((N + 127) // 128) * (K // 128) * 4
    return L * (3 * wb(d, h) + wb(h, d) + wb(d, f) + wb(f, d)) + wb(d, V)


def bench_decode(dev, steps=32, prompt=128):
    """KV-cached decode (decode.py) of the reference Config (d 2304, 24 layers,
    18 x 128 heads, d_ff 9216, vocab 50257): prefill `prompt` tokens, then
    `steps` decode steps, each one replay of the captured step graph; ms per
    step and the weight-read rate per step (kept FP8 weights + scales + the KV
    cache positions <= t; the captured attention reads the whole cache under a
    mask, which the figure does not count)."""
    import torch
    import decode
    cfg = decode.Config()
    params = decode.init_params(cfg, dev, seed=0)
    out = {"workload": "KV-cached decode, reference Config (24 layers, d 2304, 18x128 heads, d_ff 9216, "
                       f"vocab 50257), FP8 weights 128x128 scales, prompt {prompt}, {steps} steps"}
    for B in (1, 8):
        model = decode.FP8Decoder(params, cfg, max_batch=B)
        model.capture_step(B)
        g = torch.Generator(device=dev).manual_seed(1)
        ids = torch.randint(0, cfg.vocab_size, (B, prompt), generator=g, device=dev)
        toks = torch.randint(0, cfg.vocab_size, (steps + 4, B), generator=g, device=dev)
        model.prefill(ids)
        for i in range(4):
            model.step(toks[i])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            model.step(toks[4 + i])
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        ctx = prompt + 4 + steps / 2
        kv = 2 * cfg.n_layers * B * cfg.n_heads * ctx * cfg.head_dim * 2
        byts = decode_weight_bytes(cfg) + kv
        gbps = byts / dt / 1e9
        out[f"batch_{B}"] = {"ms_per_step": round(dt * 1e3, 3), "tokens_per_s": round(B / dt, 1),
                             "bytes_per_step": int(byts),
                             "roofline": {"bound": "hbm", "achieved": round(gbps, 1),
                                          "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                                          "frac": round(gbps / HBM_PEAK_GBPS, 4)}}
        del model
        torch.cuda.empty_cache()
    return out


def cpu_baseline(inputs, repeats=5):
    """The CPU oracle on the step: quantize (C oracle) and the dequantized f32
    GEMMs (numpy/BLAS) of fwd + FP8 bwd on the GPU step's own input arrays,
    best of `repeats` after one warm-up (the reference's own timing method,
    bench.py:118-135).  FLOP counted = 3 * 2 * 8192 * 2048 * 8192."""
    import numpy as np
    from threadpoolctl import threadpool_info
    from oracle import cbind, fp8_ref
    x, w, dy = inputs
    rows = x.shape[0]
    dec = lambda q, s: (fp8_ref.E4M3FN_VALUES[q].reshape(q.shape[0], -1, 128)
                        * s[:, :, None]).reshape(q.shape[0], -1)
    def one_step():
        qx, sx = cbind.quantize_rows_bf16(x)
        qwt, swt = cbind.quantize_cols_bf16(w)
        y = dec(qx, sx) @ dec(qwt, swt).T
        qdy, sdy = cbind.quantize_rows_bf16(dy)
        qw, sw = cbind.quantize_rows_bf16(w)
        dx = dec(qdy, sdy) @ dec(qw, sw).T
        qxt, sxt = cbind.quantize_cols_bf16(x)
        qdyt, sdyt = cbind.quantize_cols_bf16(dy)
        dw = dec(qxt, sxt) @ dec(qdyt, sdyt).T
        assert y.shape == (rows, N3) and dx.shape == (rows, K3) and dw.shape == (K3, N3)

    one_step()
    times = []
    t_all = time.perf_counter()
    for _ in range(repeats):
        t0 = time.perf_counter()
        one_step()
        times.append(time.perf_counter() - t0)
    total = time.perf_counter() - t_all
    dt = min(times)
    flop = 3 * 2.0 * rows * K3 * N3
    threads = max([i.get("num_threads", 1) for i in threadpool_info()] + [1])
    host_cores, model = host_cpu()
    return {"value": round(flop / dt / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "host_cores": host_cores, "cpu_model": model,
            "threads": {"quantizers": 1, "blas_gemm": threads},
            "sample": f"C3 fwd+FP8 bwd on all {rows} token rows of the GPU step's own input arrays "
                      f"(numpy default_rng(2)), best of {repeats} ({total:.1f} s of CPU time): C oracle "
                      f"quantizers single-thread, numpy f32 dequant GEMMs on {threads} BLAS threads"}


def main():
    args = parse()
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    dev = torch.device("cuda:0")
    if args.only == "decode" and under_counter_collection():
        print(json.dumps({"error": "the decode workload replays a captured HIP graph and is not run "
                                   "under rocprofv3 counter collection"}))
        sys.exit(2)
    if args.only and args.only != "step":
        fn = {"norm_quant": bench_norm, "norm_bwd": bench_norm_bwd, "gemv": bench_gemv,
              "bwd_bf16": lambda d, _: bench_bwd_bf16(d, 10),
              "block_step": lambda d, _: bench_block(d), "xent": bench_xent,
              "decode": lambda d, _: bench_decode(d),
              "vendor_gemm": lambda d, _: bench_vendor_gemm(d, 20),
              "c1": bench_c1, "block_k": bench_block_k, "io_floor": bench_io_floor, "gemv_floor": bench_gemv_floor,
              "quant_floor": bench_quant_floor}[args.only]
        print(json.dumps({args.only: fn(dev, args.norm_iters)}))
        return
    step = Step(dev)
    # Clock settle: after idle the GPU clock ramps for ~30 ms (the first ~40
    # C3 steps run 5-25% slower than the steady state a training loop runs
    # at), so untimed steps run for CLOCK_SETTLE_MS of wall time before the
    # requested warm-up steps; both are reported, and the timed region below
    # is exactly --steps full steps.
    settle_steps, t_settle = 0, time.perf_counter()
    while (time.perf_counter() - t_settle) * 1e3 < CLOCK_SETTLE_MS:
        for _ in range(10):
            step.run()
        torch.cuda.synchronize()
        settle_steps += 10
    settle_ms = (time.perf_counter() - t_settle) * 1e3
    for _ in range(args.warmup):
        step.run()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        step.run()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = max(wall * 1e3, start.elapsed_time(stop)) / args.steps
    # the GEMMs' launch times: the same steps again, HIP events around each GEMM
    # launch on its stream (kept out of the region above: every event record
    # leaves the stream idle for a few microseconds)
    ev = []
    for _ in range(args.steps):
        step.run(ev)
    torch.cuda.synchronize()
    gemm_ms = sum(s.elapsed_time(e) for s, e in ev) / len(ev)
    gemm_tflops = GEMM_FLOP / (gemm_ms * 1e-3) / 1e12
    value = STEP_FLOP / (ms_step * 1e-3) / 1e12
    accuracy = step_accuracy(step)
    power = (sustained_clock(step) if not under_profiler() else
             {"skipped": "not run under rocprofv3 (it would add ~2 s of launches to the trace)"})
    if args.only == "step":
        norm = norm_bwd = gemv = bwd_bf16 = block_step = xent = dec = c1 = bks = None
    else:
        c1 = bench_c1(dev, args.norm_iters)
        bks = bench_block_k(dev, args.norm_iters)
        norm = bench_norm(dev, args.norm_iters)
        norm_bwd = bench_norm_bwd(dev, args.norm_iters)
        gemv = bench_gemv(dev, args.norm_iters)
        bwd_bf16 = bench_bwd_bf16(dev, 10)
        block_step = bench_block(dev)
        xent = bench_xent(dev, args.norm_iters)
        dec = (bench_decode(dev) if not under_counter_collection() else
               {"skipped": "captured-graph replay is not run under rocprofv3 counter collection"})
    out = {
        "metric": "FP8 block-scaled GEMM TFLOP/s (% fp8 MFMA peak); RMSNorm+quant HBM GB/s",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "clock_settle": {"steps": settle_steps, "ms": round(settle_ms, 1)},
        "ms_per_step": round(ms_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp8e4m3 (f32 accumulate, bf16 io)",
        "data": "synthetic (numpy default_rng(2), the same arrays as cpu_baseline)",
        "config": {"workload": "C3 block_scaled_matmul fwd + FP8 bwd, x[8192,2048] W[2048,8192] "
                               "dY[8192,8192] bf16, 1x128 scales (quantization included)",
                   "M": M3, "K": K3, "N": N3, "block_k": 128},
        "gemm_us_per_launch": round(gemm_ms * 1e3, 2),
        "roofline": {"bound": "mfma", "achieved": round(gemm_tflops, 1), "peak": FP8_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(gemm_tflops / FP8_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic().get("gemm_fp8_nt_256")},
        "accuracy": accuracy,
        "sustained_clock": power,
        "c1": c1,
        "block_k_sizes": bks,
        "norm_quant": norm,
        "norm_bwd": norm_bwd,
        "gemv": gemv,
        "bwd_bf16": bwd_bf16,
        "block_step": block_step,
        "xent": xent,
        "decode": dec,
    }
    if args.only == "step":                      # the headline step alone (no secondary workloads)
        out = {k: out[k] for k in ("metric", "value", "unit", "steps", "warmup", "clock_settle", "ms_per_step",
                                   "gemm_us_per_launch", "roofline", "accuracy", "sustained_clock")}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(step.host)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
