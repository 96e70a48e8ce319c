"""Benchmark of the gfx950 N-d convolution hot path (BASELINE.json metric).

Workload ("C2"): Conv4d bf16 with fp32 accumulation, in=32 out=64,
kernel 3, padding 'same', stride 1, bias; x[2,32,16,16,16,16] ~ N(0,1) (seed 0), weight and
bias ~ U(+-1/sqrt(32*81)). A step is one forward plus the full backward (dx, dW, db) through
``torch_convnd.conv_nd(..., backend="native")`` for a synthetic upstream gradient dY (the
layer inside a network receives dY; the reference's benchmark differentiates
y.square().mean() instead, src/torch_convnd/benchmark.py:36-70, whose elementwise loss
kernels are not convolution work). Inputs and dY are resident in HBM before the timed
region; the correctness gate runs first (check, then time).

Prints ONE JSON line. ``value`` is forward+backward TFLOP/s (algorithmic FLOPs: 3x the
forward's 2*N*P*Co*(C/g)*taps; db and the loss are not counted) over wall-clock time
between synchronisations. ``roofline`` is the dominant kernel's algorithmic FLOPs per launch
over its average launch time, measured with HIP events around every launch in the timed
region. ``cpu_baseline`` times this repo's restatement of the reference's backend="torch"
CPU path (oracle/torch_path.py) on the host cores.
"""

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "torch-convnd_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "Conv4d fwd & fwd+bwd TFLOP/s at 1 GPU (bf16) + % of MFMA/HBM roofline"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (AMD published)
PEAK_HBM_GBS = 8000.0

PEAK_FP32_TFLOPS = 157.3  # MI355X fp32 MFMA (AMD published)

X_SHAPE = (2, 32, 16, 16, 16, 16)
W_SHAPE = (64, 32, 3, 3, 3, 3)
STRIDE, PADDING, DILATION, GROUPS = (1,) * 4, (1,) * 4, (1,) * 4, 1

# x shape, w shape, stride, padding, dilation, groups, bias, dtype name,
# and the rooflines reported for it (the first is the bound).
CONFIGS = {
    "C1": ((4, 2, 8, 8, 8, 16), (8, 2, 3, 3, 3, 3), (1,) * 4, (1,) * 4, (1,) * 4, 1, True, "float32",
           ("fp32_mfma", "hbm")),
    "C2": (X_SHAPE, W_SHAPE, STRIDE, PADDING, DILATION, GROUPS, True, "bfloat16", ("bf16_mfma",)),
    "C3": ((1, 16, 12, 12, 12, 12, 12), (32, 16, 3, 3, 3, 3, 3), (1,) * 5, (1,) * 5, (1,) * 5, 1, True,
           "bfloat16", ("bf16_mfma",)),
    "C4_fp32": ((1, 8, 8, 8, 8, 8, 8, 8), (16, 8, 3, 3, 3, 3, 3, 3), (1,) * 6, (1,) * 6, (1,) * 6, 1, True,
                "float32", ("fp32_mfma",)),
    "C4_bf16": ((1, 8, 8, 8, 8, 8, 8, 8), (16, 8, 3, 3, 3, 3, 3, 3), (1,) * 6, (1,) * 6, (1,) * 6, 1, True,
                "bfloat16", ("bf16_mfma",)),
    "C5": ((2, 64, 24, 24, 24, 12), (128, 16, 3, 3, 3, 5), (2, 2, 2, 1), (1, 1, 1, 4), (1, 1, 1, 2), 4, False,
           "bfloat16", ("bf16_mfma", "hbm")),
}
PEAKS = {"bf16_mfma": (PEAK_BF16_TFLOPS, "TFLOP/s"), "fp32_mfma": (PEAK_FP32_TFLOPS, "TFLOP/s"),
         "hbm": (PEAK_HBM_GBS, "GB/s")}


CL_CONFIGS = ("C2", "C5")


def to_channels_last(t):
    """Same values, stored [N, *spatial, C]."""
    order = (0, *range(2, t.dim()), 1)
    return t.permute(order).contiguous().permute(0, t.dim() - 1, *range(1, t.dim() - 1))


def config_work(name):
    """(forward FLOP, forward bytes, forward+backward bytes) of a config: FLOP = 2 N P Co
    (C/g) taps; bytes = |x| + |W| + |y| (+|b|) forward and |dY| + |x| + |W| + |dx| + |dW|
    backward, in the config's element size."""
    xs, ws, stride, padding, dilation, groups, bias, dtype, _ = CONFIGS[name]
    out = [(n + 2 * p - d * (k - 1) - 1) // s + 1
           for n, k, s, p, d in zip(xs[2:], ws[2:], stride, padding, dilation)]
    el = 4 if dtype == "float32" else 2
    nx, nw, ny = math.prod(xs), math.prod(ws), xs[0] * ws[0] * math.prod(out)
    flops = 2 * xs[0] * math.prod(out) * ws[0] * ws[1] * math.prod(ws[2:])
    fwd_bytes = el * (nx + nw + ny + (ws[0] if bias else 0))
    bwd_bytes = el * (ny + nx + nw + nx + nw)
    return flops, fwd_bytes, fwd_bytes + bwd_bytes


def forward_flops(x_shape=X_SHAPE, w_shape=W_SHAPE):
    positions = math.prod(x_shape[2:])  # 'same' padding, stride 1
    return 2 * x_shape[0] * positions * w_shape[0] * w_shape[1] * math.prod(w_shape[2:])


def make_inputs(torch, dtype, device, x_shape=X_SHAPE, w_shape=W_SHAPE, seed=0):
    g = torch.Generator().manual_seed(seed)
    bound = 1.0 / math.sqrt(w_shape[1] * math.prod(w_shape[2:]))
    x = torch.randn(x_shape, generator=g)
    w = (torch.rand(w_shape, generator=g) * 2 - 1) * bound
    b = (torch.rand((w_shape[0],), generator=g) * 2 - 1) * bound
    return [t.to(dtype).to(device) for t in (x, w, b)]


def correctness_gate(torch, np, conv, x, w, b):
    """Check sampled outputs and gradients of the full-size problem against float64 sums
    computed directly from the definition (check, then time)."""
    xs, ws, bs = (t.detach().requires_grad_() for t in (x, w, b))
    y = conv(xs, ws, bs)
    dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(7)).to(y.dtype).to(y.device)
    gx, gw, gb = torch.autograd.grad(y, (xs, ws, bs), dy)
    torch.cuda.synchronize()
    X = x.double().cpu().numpy()
    W = w.double().cpu().numpy()
    B = b.double().cpu().numpy()
    DY = dy.double().cpu().numpy()
    Xp = np.pad(X, ((0, 0), (0, 0)) + ((1, 1),) * 4)
    DYp = np.pad(DY, ((0, 0), (0, 0)) + ((1, 1),) * 4)
    rng = np.random.default_rng(3)
    Y, GX, GW = (t.detach().double().cpu().numpy() for t in (y, gx, gw))
    worst = 0.0
    for _ in range(64):
        n, co = rng.integers(2), rng.integers(64)
        o = rng.integers(16, size=4)
        ref = B[co] + np.sum(W[co] * Xp[n, :, o[0]:o[0] + 3, o[1]:o[1] + 3, o[2]:o[2] + 3, o[3]:o[3] + 3])
        worst = max(worst, abs(Y[n, co, o[0], o[1], o[2], o[3]] - ref) / (2e-2 * (abs(ref) + 0.05)))
        ci = rng.integers(32)
        # dX[x] = sum_{co,t} W[co,ci,t] * dY[x + 1 - t] (stride 1, pad 1): flipped window.
        win = DYp[n, :, o[0]:o[0] + 3, o[1]:o[1] + 3, o[2]:o[2] + 3, o[3]:o[3] + 3]
        ref = np.sum(W[:, ci, ::-1, ::-1, ::-1, ::-1] * win)
        worst = max(worst, abs(GX[n, ci, o[0], o[1], o[2], o[3]] - ref) / (2e-2 * (abs(ref) + 0.5)))
    for _ in range(8):
        co, ci = rng.integers(64), rng.integers(32)
        t = rng.integers(3, size=4)
        patch = Xp[:, ci, t[0]:t[0] + 16, t[1]:t[1] + 16, t[2]:t[2] + 16, t[3]:t[3] + 16]
        ref = np.sum(DY[:, co] * patch)
        worst = max(worst, abs(GW[co, ci, t[0], t[1], t[2], t[3]] - ref) / (2e-2 * (abs(ref) + 20.0)))
    ref_db = DY.sum(axis=(0, 2, 3, 4, 5))
    worst = max(worst, float(np.max(np.abs(gb.detach().double().cpu().numpy() - ref_db) / (2e-2 * (np.abs(ref_db) + 20.0)))))
    if worst > 1.0:
        raise SystemExit(f"correctness gate failed (worst normalised error {worst:.3f})")
    return worst


def profiled_traffic():
    """HBM-side bytes per launch of each MFMA kernel, measured by two rocprofv3 PMC runs
    (FETCH_SIZE, WRITE_SIZE) scaled by a copy of known size; recorded in
    profiles/c2_hbm_traffic.md (None when that file is absent)."""
    path = ROOT / "profiles" / "c2_hbm_traffic.md"
    try:
        for line in path.read_text(encoding="utf-8").splitlines():
            if line.strip().startswith("traffic_bytes_per_launch:"):
                return json.loads(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return {}


def cpu_baseline(torch):
    """The reference's backend="torch" CPU path (restated in oracle/torch_path.py) on the
    same C2 problem, bf16 with fp32 partial accumulation; median of timed fwd+bwd runs."""
    from oracle import torch_path

    cores = cpu_threads()
    previous = torch.get_num_threads()
    torch.set_num_threads(cores)
    try:
        x, w, b = make_inputs(torch, torch.bfloat16, "cpu")
        x, w, b = (t.requires_grad_() for t in (x, w, b))
        out_shape = (X_SHAPE[0], W_SHAPE[0], *X_SHAPE[2:])
        dy = torch.randn(out_shape, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)

        def run():
            y = torch_path.torch_backend_conv(x, w, b, STRIDE, PADDING, DILATION, GROUPS)
            torch.autograd.grad(y, (x, w, b), dy)

        def forward():
            with torch.no_grad():
                torch_path.torch_backend_conv(x, w, b, STRIDE, PADDING, DILATION, GROUPS)

        def median_s(fn, budget_s):
            fn()  # warmup (first-call allocations)
            start = time.perf_counter()
            fn()  # one run to size the sample to the time budget
            first = time.perf_counter() - start
            iterations = max(3, min(1000, int(budget_s / max(first, 1e-3))))
            times = []
            for _ in range(iterations):
                t0 = time.perf_counter()
                fn()
                times.append(time.perf_counter() - t0)
            return statistics.median(times), iterations

        median, iterations = median_s(run, 10.0)
        fwd_median, fwd_iterations = median_s(forward, 3.0)
        return {
            "value": round(3 * forward_flops() / median / 1e12, 6),
            "unit": "TFLOP/s",
            "cores": cores,
            "kind": "port",
            "fwd_bwd_ms": round(median * 1e3, 2),
            "fwd_ms": round(fwd_median * 1e3, 2),
            "fwd_tflops": round(forward_flops() / fwd_median / 1e12, 6),
            "affinity_cores": len(os.sched_getaffinity(0)),
            "sample": (
                f"full C2 problem, fwd + full bwd (dx, dW, db) for a fixed dY, bf16, median of "
                f"{iterations} runs after a warmup and a sizing run ({median * 1e3:.0f} ms each); forward alone "
                f"median of {fwd_iterations} runs; {cores} threads; torch {torch.__version__}, "
                f"{_cpu_model()}"
            ),
        }
    finally:
        torch.set_num_threads(previous)


def cpu_threads():
    """Host threads for the CPU baseline: the cores this process may run on, capped by the
    host's per-job thread allowance when OMP_NUM_THREADS sets one (a shared GPU box gives each
    GPU's job a CPU share and exports it there)."""
    cores = len(os.sched_getaffinity(0))
    try:
        share = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        share = 0
    return min(cores, share) if share > 0 else cores


def measure_configs(torch, device, iterations=30, warmup=5, only=None):
    """Every BASELINE config at full size through conv_nd(backend="native"): forward alone
    and forward + full backward (dx, dW, db) for a resident synthetic dY; each the median of
    `iterations` calls timed with their own HIP event pair after `warmup` calls (warm caches:
    every working set is below the 256 MB Infinity Cache and nothing is flushed)."""
    import torch_convnd
    from torch_convnd import _build, _capi

    lib = _build.hip_library()
    out = {}
    # Channels-last runs of C2 and C5, x stored [N, *spatial, C]: "_channels_last" with
    # memory_format=torch.preserve_format (dY, output and grad_input in that layout too; the
    # forward makes no layout copy), "_channels_last_input" with the default contract
    # (contiguous output, grad_input and dY, as the reference operators return).
    runs = [(name, name, None) for name in CONFIGS]
    for name in CL_CONFIGS:
        runs += [(f"{name}_channels_last", name, torch.preserve_format),
                 (f"{name}_channels_last_input", name, torch.contiguous_format)]
    for name, base, cl_format in runs:
        channels_last = cl_format is not None
        memory_format = cl_format if channels_last else torch.contiguous_format
        xs, ws, stride, padding, dilation, groups, bias, dtype_name, roofs = CONFIGS[base]
        if only is not None and name not in only:
            continue
        dtype = getattr(torch, dtype_name)
        x, w, b = make_inputs(torch, dtype, device, xs, ws)
        if channels_last:
            x = to_channels_last(x)
        if not bias:
            b = None
        leaves = [t.detach().requires_grad_() for t in (x, w, b) if t is not None]

        def conv(*ts):
            return torch_convnd.conv_nd(ts[0], ts[1], ts[2] if len(ts) > 2 else None, stride, padding,
                                        dilation, groups, backend="native", memory_format=memory_format)

        y = conv(*leaves)
        dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(5)).to(dtype).to(device)
        if memory_format is torch.preserve_format:
            dy = to_channels_last(dy)
        del y

        def fwd():
            with torch.no_grad():
                conv(*(x, w, b)[: len(leaves)])

        def step():
            torch.autograd.grad(conv(*leaves), leaves, dy)

        times = {}
        for label, fn in (("fwd", fwd), ("fwd_bwd", step)):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            pairs = []
            for _ in range(iterations):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                fn()
                e1.record()
                pairs.append((e0, e1))
            torch.cuda.synchronize()
            times[label] = statistics.median(a.elapsed_time(b_) for a, b_ in pairs)
        flops, fwd_bytes, step_bytes = config_work(base)
        entry = {"dtype": dtype_name,
                 "plans": list(_capi.plan_names(lib, xs, ws, stride, padding, dilation, groups, dtype))}
        for label, work_flops, work_bytes in (("fwd", flops, fwd_bytes), ("fwd_bwd", 3 * flops, step_bytes)):
            ms = times[label]
            tflops = work_flops / (ms * 1e-3) / 1e12
            entry[f"{label}_ms"] = round(ms, 4)
            entry[f"{label}_tflops"] = round(tflops, 2)
            for roof in roofs:
                peak, unit = PEAKS[roof]
                achieved = tflops if unit == "TFLOP/s" else work_bytes / (ms * 1e-3) / 1e9
                entry[f"{label}_frac_{roof}"] = round(achieved / peak, 4)
        entry["bound"] = roofs[0]
        out[name] = entry
        del x, w, b, leaves, dy
    return out


def _cpu_model():
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.partition(":")[2].strip()
    except OSError:
        pass
    return "unknown CPU"


def measure_peaks(torch, device):
    """Achieved bf16 GEMM rate (torch.matmul, square n^3) and device copy bandwidth."""
    res = {}
    for n, it in ((8192, 20), (16384, 5)):
        a = torch.randn(n, n, device=device, dtype=torch.bfloat16)
        b = torch.randn(n, n, device=device, dtype=torch.bfloat16)
        for _ in range(3):
            torch.matmul(a, b)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(it):
            torch.matmul(a, b)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / it
        res[f"bf16_matmul_{n}"] = {"ms": round(ms, 3), "tflops": round(2 * n**3 / (ms * 1e-3) / 1e12, 1)}
        del a, b
    src = torch.empty(1 << 30, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 10
    res["copy_1GiB"] = {"ms": round(ms, 3), "tb_s_read_plus_write": round(2 * (1 << 30) / (ms * 1e-3) / 1e12, 2)}
    return res


def _timed_ms(torch, fn, steps, warmup):
    """Mean milliseconds of fn() over `steps` calls (HIP events on torch's current stream)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def measure_partial(torch, device, steps, warmup):
    """Partial convolution on C2 (bf16, bias, single-channel mask with 30 % holes)."""
    import torch_convnd

    x, w, b = make_inputs(torch, torch.bfloat16, device)
    g = torch.Generator().manual_seed(9)
    mask = (torch.rand((X_SHAPE[0], 1, *X_SHAPE[2:]), generator=g) > 0.3).to(torch.bfloat16).to(device)

    def partial():
        return torch_convnd.partial_conv_nd(x, w, b, STRIDE, "same", DILATION, GROUPS, mask=mask, backend="native")

    out, update = partial()
    out_shape = tuple(out.shape)
    n, co = out_shape[:2]
    positions = math.prod(out_shape[2:])
    # The rescale alone, on resident raw output and counts of the same shapes.
    raw = torch.randn(out_shape, generator=g).to(torch.bfloat16).to(device)
    counts = torch.randint(0, 82, (n, 1, *out_shape[2:]), generator=g).float().to(device)
    window = float(math.prod(W_SHAPE[2:]))
    op = torch.ops.torch_convnd.partial_rescale.default
    fused_ms = _timed_ms(torch, lambda: op(raw, counts, b, window), steps, warmup)

    def unfused():
        # The same rescale as separate PyTorch elementwise launches (the reference's form).
        upd = counts.clamp(0, 1)
        ratio = (upd * window / counts.clamp_min(torch.finfo(torch.float32).tiny)).to(raw.dtype)
        return torch.addcmul(b.reshape(1, -1, 1, 1, 1, 1), raw, ratio) * upd.to(raw.dtype)

    unfused_ms = _timed_ms(torch, unfused, steps, warmup)
    fwd_ms = _timed_ms(torch, partial, steps, warmup)
    xs, ws, bs = (t.detach().requires_grad_() for t in (x, w, b))
    cot = torch.randn(out_shape, generator=g).to(torch.bfloat16).to(device)

    def step():
        y, _ = torch_convnd.partial_conv_nd(xs, ws, bs, STRIDE, "same", DILATION, GROUPS, mask=mask, backend="native")
        torch.autograd.grad(y, (xs, ws, bs), cot)

    step_ms = _timed_ms(torch, step, steps, warmup)
    # Algorithmic HBM bytes of one rescale launch: read raw, write out (2 B each per
    # element), read the counts once (4 B per count position), read the bias.
    rescale_bytes = 2 * 2 * n * co * positions + 4 * n * positions + 2 * co
    achieved = rescale_bytes / (fused_ms * 1e-3) / 1e9
    return {
        "metric": "partial convolution on C2 (bf16, bias, 30% hole mask)",
        "config": {"workload": "C2 partial_conv_nd x[2,32,16,16,16,16] w[64,32,3,3,3,3] same padding",
                   "mask": "[2,1,16,16,16,16], 30% holes"},
        "steps": steps, "warmup": warmup,
        "rescale_fused_us": round(fused_ms * 1e3, 2),
        "rescale_unfused_torch_us": round(unfused_ms * 1e3, 2),
        "partial_fwd_us": round(fwd_ms * 1e3, 2),
        "partial_fwd_bwd_us": round(step_ms * 1e3, 2),
        "roofline": {"bound": "hbm", "kernel": "partial_rescale_runs", "achieved": round(achieved, 1),
                     "peak": 8000.0, "unit": "GB/s", "frac": round(achieved / 8000.0, 4),
                     "bytes_per_launch": rescale_bytes},
    }


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=100)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-configs", action="store_true",
                        help="skip the per-config fwd / fwd+bwd timings of C1-C5")
    parser.add_argument("--configs", default="",
                        help="comma-separated subset of C1,C2,C3,C4_fp32,C4_bf16,C5,C2_channels_last,"
                        "C5_channels_last,C2_channels_last_input,C5_channels_last_input for the per-config "
                        "timings (default: all)")
    parser.add_argument(
        "--calibration-copy-mib", type=int, default=0,
        help="first run a plain elementwise copy of this many MiB three times (the known-size "
        "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes)")
    parser.add_argument(
        "--peaks", action="store_true",
        help="only measure the on-box achieved peaks (a large bf16 GEMM through torch.matmul, "
        "i.e. hipBLASLt, and a 1 GiB device copy) and print them as one JSON line")
    parser.add_argument(
        "--partial", action="store_true",
        help="measure partial convolution on the C2 shape instead (bf16, bias, a 30%% hole "
        "mask): the fused gfx950 rescale kernel against its HBM roofline, the same rescale as "
        "PyTorch elementwise ops, and partial_conv_nd forward and forward+backward")
    parser.add_argument(
        "--epilogue", action="store_true",
        help="measure the C2 bf16 forward followed by GELU (inference, no autograd): "
        "conv_nd then torch.nn.functional.gelu against conv_nd(activation='gelu') with the "
        "activation fused into the epilogue")
    args = parser.parse_args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU: this build's hot path is a single-GPU kernel set "
            f"(requested --gpus {args.gpus}); run with --gpus 1",
            file=sys.stderr,
        )
        sys.exit(2)

    import numpy as np
    import torch

    import torch_convnd
    from torch_convnd import _build, _capi

    if not (torch.cuda.is_available() and torch.version.hip is not None):
        raise SystemExit("bench.py needs a ROCm GPU")
    torch.backends.cuda.matmul.allow_tf32 = False
    torch_convnd.load_native()
    lib = _build.hip_library()
    device = torch.device("cuda", 0)
    if args.peaks:
        print(json.dumps(measure_peaks(torch, device)), flush=True)
        return
    if args.partial:
        print(json.dumps(measure_partial(torch, device, args.steps, args.warmup)), flush=True)
        return
    if args.epilogue:
        x, w, b = make_inputs(torch, torch.bfloat16, device)

        def unfused():
            y = torch_convnd.conv_nd(x, w, b, STRIDE, "same", DILATION, GROUPS, backend="native")
            return torch.nn.functional.gelu(y)

        def fused():
            return torch_convnd.conv_nd(x, w, b, STRIDE, "same", DILATION, GROUPS, backend="native",
                                        activation="gelu")

        with torch.no_grad():
            diff = (fused().float() - unfused().float()).abs().max().item()
            unfused_ms = _timed_ms(torch, unfused, args.steps, args.warmup)
            fused_ms = _timed_ms(torch, fused, args.steps, args.warmup)
        print(json.dumps({
            "metric": "C2 bf16 forward + GELU (inference)", "steps": args.steps, "warmup": args.warmup,
            "unfused_us": round(unfused_ms * 1e3, 2), "fused_us": round(fused_ms * 1e3, 2),
            "fused_tflops": round(forward_flops() / (fused_ms * 1e-3) / 1e12, 1),
            "max_abs_diff_vs_unfused": diff,
        }), flush=True)
        return
    if args.calibration_copy_mib > 0:
        src = torch.ones(args.calibration_copy_mib << 18, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)  # reads and writes exactly the tensor's bytes
        torch.cuda.synchronize()
        del src, dst
    x, w, b = make_inputs(torch, torch.bfloat16, device)

    def conv(xx, ww, bb):
        return torch_convnd.conv_nd(xx, ww, bb, STRIDE, "same", DILATION, GROUPS, backend="native")

    plans = _capi.plan_names(lib, X_SHAPE, W_SHAPE, STRIDE, PADDING, DILATION, GROUPS, torch.bfloat16)
    gate = correctness_gate(torch, np, conv, x, w, b)

    xs, ws, bs = (t.detach().requires_grad_() for t in (x, w, b))
    # Upstream gradient of the layer output: synthetic, resident in HBM before timing.
    out_shape = (X_SHAPE[0], W_SHAPE[0], *X_SHAPE[2:])
    cotangent = torch.randn(out_shape, generator=torch.Generator().manual_seed(5))
    cotangent = cotangent.to(torch.bfloat16).to(device)

    def step():
        y = conv(xs, ws, bs)
        torch.autograd.grad(y, (xs, ws, bs), cotangent)

    def fwd_only():
        with torch.no_grad():
            conv(x, w, b)

    for _ in range(args.warmup):
        step()
        fwd_only()
    torch.cuda.synchronize()

    # Forward alone (the metric's first half).
    _capi.read_kernel_times(lib)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        fwd_only()
    torch.cuda.synchronize()
    fwd_ms = (time.perf_counter() - t0) * 1e3 / args.steps

    # Timed fwd+bwd steps (the headline value), free of any instrumentation.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    step_ms = (time.perf_counter() - t0) * 1e3 / args.steps

    # The same steps again with every main kernel launch bracketed by HIP events recorded on
    # its launch stream (an event record costs a few microseconds of stream time, so this
    # region is kept apart from the headline one).
    lib.convnd_hip_timing_enable(1)
    torch.cuda.synchronize()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    lib.convnd_hip_timing_enable(0)
    kernels = _capi.read_kernel_times(lib)

    flops = forward_flops()
    value = 3 * flops / (step_ms * 1e-3) / 1e12
    fwd_tflops = flops / (fwd_ms * 1e-3) / 1e12
    per_kernel = {}
    for name, (total, count) in kernels.items():
        if count:
            avg_ms = total / count
            per_kernel[name] = {
                "avg_us": round(avg_ms * 1e3, 2),
                "launches": count,
                "tflops": round(flops / (avg_ms * 1e-3) / 1e12, 2),
                "frac_bf16_peak": round(flops / (avg_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            }
    dominant = max(per_kernel, key=lambda k: per_kernel[k]["avg_us"])
    achieved = per_kernel[dominant]["tflops"]
    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) input, U(+-1/sqrt(fan_in)) weight/bias)",
        "config": {
            "workload": "C2: Conv4d bf16 (fp32 accumulate) 32->64 k3 padding=same x[2,32,16,16,16,16], "
            "forward + full backward (dx, dW, db) for a resident synthetic dY",
            "global_batch": X_SHAPE[0],
            "forward_gflop": round(flops / 1e9, 3),
            "parallelism": "single GPU",
            "kernels": {"forward": plans[0], "grad_input": plans[1], "grad_weight": plans[2]},
        },
        "fwd_ms": round(fwd_ms, 4),
        "fwd_tflops": round(fwd_tflops, 3),
        "fwd_frac_bf16_peak": round(fwd_tflops / PEAK_BF16_TFLOPS, 4),
        "fwd_bwd_frac_bf16_peak": round(value / PEAK_BF16_TFLOPS, 4),
        "kernel_times": per_kernel,
        "roofline": {
            "bound": "mfma",
            "kernel": dominant,
            "achieved": achieved,
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": profiled_traffic().get(dominant),
            "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
        },
        "correctness_gate_worst": round(gate, 4),
        "timing": {
            "value": "wall clock between synchronisations over the timed steps, no events",
            "fwd_ms": "wall clock of forward-only calls, no events",
            "roofline": "HIP events recorded around every launch of the kernel on its launch "
            "stream in a separate region, averaged",
            "configs": "median of 30 calls after 5 warmups, one HIP event pair per call",
            "cache": "warm: every working set is below the 256 MB Infinity Cache; no flush",
        },
    }
    if not args.no_configs:
        only = [c for c in args.configs.split(",") if c] or None
        result["configs"] = measure_configs(torch, device, only=only)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(torch)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
