"""Benchmark of the Hyena long-convolution hot path on one MI355X.

Default workload (the BASELINE metric's configuration, config 3): causal 1D
FFT convolution forward + backward at B=1, D=4096, L=262144 (FFT length
2^19), x / upstream gradient bf16 ~ N(0,1), filter fp32 N(0,1)*exp(-a_d t/L)
with a_d ~ U(1,50), shortcut bf16.  A step is one forward and one backward
call on inputs resident in HBM, with outputs and workspace preallocated.

Prints one JSON line with the driver's fields plus:
  roofline     -- algorithmic HBM bytes of the fwd+bwd pair / its measured time,
                  against MI355X's 8 TB/s (the path is HBM-bound by definition
                  of the metric);
  cpu_baseline -- the CPU oracle (float32 torch.fft restatement of the
                  reference path, autograd backward) on a bounded channel
                  sample of the same workload, on this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
       python bench.py --workload cfg1|cfg2|cfg4|cfg5   (the other benchmark
           configurations, for the per-config report; same JSON fields, value =
           algorithmic GB/s of the phase the reference's benchmark quotes for that config)
       python bench.py --workload cfg2-fwd-bwd   (config 2's block with its
           backward, report-only)
       python bench.py --workload cfg4-circular|well-rb   (periodic and
           mixed boundaries, report-only: cfg4's shape with circular padding;
           the rayleigh_benard Well config's layer, x periodic / y zero-padded)
       python bench.py --workload hyena-gated   (report-only: the Hyena gates
           fused into the causal conv, with the unfused composition's time)
       python bench.py --workload siren-conv-1d    (report-only: SIREN filter + causal conv fwd+bwd at config
                                                    3's shape with the filter never formed, and the composition)
       python bench.py --workload hyena-norm       (report-only: the Hyena output gate + RMSNorm over
                                                    channels + channels-last layout, fwd+bwd, cfg4 shape)
       python bench.py --workload hyena-groupnorm  (report-only: the Hyena conv-input gate + GroupNorm(1, C)
                                                    channels-first, fwd+bwd, cfg4 shape)
       python bench.py --workload hyena-gated-2d   (report-only: the gated 2D
           conv at cfg4's shape, with torch gates around the same conv and the
           conv alone)
       python bench.py --copy-calibration   (one plain copy kernel of known size,
                                             for scaling rocprof FETCH/WRITE_SIZE)
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch


ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "FFT-conv fwd+bwd ms & HBM GB/s (% peak), 1D D=4096 L=256K, 1 MI355X"
CFG = dict(B=1, D=4096, L=262144, K=262144, a_lo=1.0, a_hi=50.0)


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def copy_calibration() -> None:
    """One device-to-device copy of exactly 1 GiB (read 1 GiB, write 1 GiB)."""
    n = 1 << 28
    a = torch.ones(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4}))


def cpu_baseline(channels: int, iters: int) -> dict:
    """Oracle fwd+bwd on a channel sample of the config-3 workload, host cores."""
    from nvsubquadratic_amd.workloads import algorithmic_bytes_causal1d, causal1d_case
    from oracle.fftconv_ref import causal_fftconv1d_chunked_torch

    n_threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(n_threads)
    c = causal1d_case(CFG["B"], CFG["D"], CFG["L"], torch.bfloat16, (CFG["a_lo"], CFG["a_hi"]),
                      channels=slice(0, channels))
    times = []
    for it in range(iters + 1):
        x = c.x.clone().requires_grad_(True)
        k = c.k[None].clone().requires_grad_(True)
        s = c.s.clone().requires_grad_(True)
        t0 = time.perf_counter()
        # 128-channel chunks bound host memory (nvsubquadratic/ops/fftconv_chunked.py:285-322 semantics)
        y = causal_fftconv1d_chunked_torch(x, k, s, chunk_size=128)
        y.backward(c.g)
        dt = time.perf_counter() - t0
        if it > 0:
            times.append(dt)
        _log(f"cpu baseline iter {it}: {dt:.2f}s")
    med = statistics.median(times)
    nbytes = algorithmic_bytes_causal1d(CFG["B"], channels, CFG["L"], CFG["K"], 2, "fwd+bwd")
    full_ms = med * 1e3 * CFG["D"] / channels
    return {
        "value": round(nbytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": n_threads,
        "kind": "port",
        "ms_per_step_extrapolated": round(full_ms, 1),
        "sample": (f"{channels} of {CFG['D']} channels (B=1, L=262144, bf16 I/O), fwd+bwd with torch.fft fp32 "
                   f"on CPU + autograd in 128-channel chunks, median of {iters} after 1 warmup; "
                   f"value = algorithmic bytes of the "
                   f"sample / median time; ms_per_step_extrapolated scales to all {CFG['D']} channels"),
    }


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "fftconv1d_causal_cfg3_fwd_bwd_traffic.txt")


def measured_traffic() -> int | None:
    """HBM bytes of one config-3 step from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary, each scaled by its copy-kernel calibration factor."""
    try:
        lines = open(TRAFFIC_PROFILE).read().splitlines()
    except OSError:
        return None
    ff = wf = None
    total = 0.0
    for ln in lines:
        t = ln.split()
        if not t or t[0].startswith("#"):
            continue
        if t[0] == "calibration":
            ff, wf = float(t[1]), float(t[2])
        elif t[0] == "kernel" and ff is not None:
            total += float(t[2]) * 1024 * ff + float(t[3]) * 1024 * wf
    return int(round(total)) if total else None


# ---------------------------------------------------------------------------
# The reference's unfused PyTorch path on the same GPU, timed beside this build's kernels (report-only fields
# "torch_gpu_ms_per_step" and "speedup_vs_torch_gpu"): the reference publishes its fused kernels only as speedups
# over that path (docs/benchmarks.md:47-49, 78-81).  These restate its torch ops: the causal 1D conv of
# ops/fftconv.py:546-600, the 2D / 3D convs of :662-733 / :736-812 at the reference's own FFT sizes, and the B2B
# block (projection conv, gate, mixer conv with skip, gate) as separate depthwise torch convs and products.
# ---------------------------------------------------------------------------
def _torch_causal_fftconv1d(x, k, s):
    L, K = x.shape[-1], k.shape[-1]
    n = min(L + K, 2 * L)
    y = torch.fft.irfft(torch.fft.rfft(x.float(), n=n) * torch.fft.rfft(k.float(), n=n), n=n)[..., :L].to(x.dtype)
    return y if s is None else y + s.to(x.dtype).view(1, -1, 1) * x


def _torch_fftconv_nd(x, k, s):
    nd = x.ndim - 2
    S, Kd = x.shape[2:], k.shape[-nd:]
    fs = [min(Si + (Ki + 1) // 2, 2 * Si) for Si, Ki in zip(S, Kd)]
    dims = tuple(range(2, 2 + nd))
    kdims = tuple(range(k.ndim - nd, k.ndim))
    full = torch.fft.irfftn(torch.fft.rfftn(x.float(), s=fs, dim=dims) * torch.fft.rfftn(k.float(), s=fs, dim=kdims),
                            s=fs, dim=dims)
    y = full[(Ellipsis, *[slice(Ki // 2, Ki // 2 + Si) for Si, Ki in zip(S, Kd)])].to(x.dtype)
    return y + s.view(1, -1, *([1] * nd)).to(x.dtype) * x


def _torch_b2b(x, wp, wm, skip):
    import torch.nn.functional as Fn

    C, L = x.shape[1] // 3, x.shape[-1]
    p = Fn.conv1d(x.float(), wp.unsqueeze(1), padding=wp.shape[-1] - 1, groups=3 * C)[..., :L]
    q, kk, v = p.split(C, dim=1)
    z = kk * v
    h = Fn.conv1d(z, wm.unsqueeze(1), padding=wm.shape[-1] - 1, groups=C)[..., :L]
    if skip is not None:
        h = h + skip.view(1, -1, 1) * z
    return (q * h).to(x.dtype)


def _torch_gpu_ms(step, steps: int = 5, warmup: int = 1) -> float:
    """Mean ms per step of a torch-path step on the current stream (freed afterwards)."""
    t = statistics.mean(_time_steps(step, steps, warmup))
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return round(t, 4)


def cpu_baseline_other(name: str, iters: int = 3) -> dict:
    """The oracle (float32 torch on all the host cores) on the whole of config 1, 2, 4 or 5, the phase the GPU line
    times: at least ``iters`` steps after a warmup, more while under ~10 s; the median step."""
    from nvsubquadratic_amd.workloads import (algorithmic_bytes_b2b, algorithmic_bytes_causal1d,
                                              algorithmic_bytes_nd, causal1d_case_fast, radial_filter)
    from oracle.direct_ref import b2b_causal_conv1d_torch
    from oracle.fftconv_ref import causal_fftconv1d_torch, fftconv_nd_torch

    n_threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(n_threads)
    gen = torch.Generator().manual_seed(0)
    if name == "cfg1":
        B, D, L = 2, 128, 4096
        c = causal1d_case_fast(B, D, L, torch.float32, (1.0, 10.0), "cpu", seed=0)
        run = lambda: causal_fftconv1d_torch(c.x, c.k[None], c.s)  # noqa: E731
        nbytes = algorithmic_bytes_causal1d(B, D, L, L, 4, "fwd")
        what = "whole config (B=2 D=128 L=4096 fp32), forward, torch.fft"
    elif name == "cfg2":
        B, C, L = 4, 4096, 8192
        x = torch.randn(B, 3 * C, L, generator=gen).to(torch.bfloat16)
        wp = torch.randn(3 * C, 3, generator=gen)
        wm = torch.randn(C, 128, generator=gen) / 128 ** 0.5
        run = lambda: b2b_causal_conv1d_torch(x, wp, wm, None)  # noqa: E731
        nbytes = algorithmic_bytes_b2b(B, C, L, 3, 128, 2)
        what = "whole config (B=4 D=4096 L=8192, k=3 then k=128, bf16 I/O), forward, torch conv1d fp32"
    elif name in ("cfg4", "cfg5"):
        nd = 2 if name == "cfg4" else 3
        B, C, size, sig = (16, 384, 128, (4.0, 64.0)) if nd == 2 else (2, 128, 64, (2.0, 32.0))
        x = torch.randn(B, C, *([size] * nd), generator=gen).to(torch.bfloat16)
        k = radial_filter(C, size, sig[0], sig[1], nd, gen)
        sv = torch.randn(C, generator=gen).to(torch.bfloat16)
        if nd == 2:
            run = lambda: fftconv_nd_torch(x, k, sv)  # noqa: E731
            phase = "fwd"
        else:
            g = torch.randn(x.shape, generator=gen).to(torch.bfloat16)

            def run():
                xx, kk, ss = (t.clone().requires_grad_(True) for t in (x, k, sv))
                fftconv_nd_torch(xx, kk, ss).backward(g)
            phase = "fwd+bwd"
        nbytes = algorithmic_bytes_nd(B, C, [size] * nd, [size] * nd, 2, phase)
        what = (f"whole config (B={B} C={C}, {size}^{nd}, bf16 I/O), {phase}, torch.fft fp32 at the reference's "
                f"FFT size")
    else:
        return {}
    times, t_start = [], time.perf_counter()
    for it in range(1000):
        t0 = time.perf_counter()
        with torch.set_grad_enabled(name == "cfg5"):
            run()
        if it > 0:
            times.append(time.perf_counter() - t0)
        if len(times) >= iters and time.perf_counter() - t_start > 10.0:
            break
    med = statistics.median(times)
    return {
        "value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": n_threads, "kind": "port",
        "ms_per_step": round(med * 1e3, 2),
        "sample": f"{what}; median of {len(times)} steps after 1 warmup (at least {iters}, ~10 s); value = algorithmic "
                  f"bytes of the sample / median time",
    }


def counter_traffic(profile: str) -> int | None:
    """HBM bytes of one step from a committed counter summary (its 'step total' read + write GB, already scaled
    by the copy calibration)."""
    try:
        for ln in open(os.path.join(ROOT, "profiles", profile)):
            t = ln.split()
            if len(t) >= 4 and t[0] == "step" and t[1] == "total":
                return int(round((float(t[3]) + float(t[4])) * 1e9))
    except (OSError, ValueError, IndexError):
        return None
    return None


_COUNTER_PROFILES = {"cfg1": "fftconv1d_causal_cfg1_fwd_counters.md", "cfg2": "b2b_cfg2_fwd_counters.md",
                     "cfg4": "fftconv2d_cfg4_fwd_counters.md", "cfg5": "fftconv3d_cfg5_fwd_bwd_counters.md"}


def _time_steps(step, steps: int, warmup: int, min_warm_s: float = 0.25) -> list[float]:
    """Event-timed steps on the current stream (ms each) after untimed warmup.

    The warmup runs ``warmup`` steps (which hold the first-call costs), then more for at least ``min_warm_s``
    seconds: a sub-millisecond step otherwise gets timed while the GPU clock is still ramping (0.31 against 0.27 ms
    for config 2's forward).
    """
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < min_warm_s and n < 10000:
        step()
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()  # count the device's time, not the enqueue rate
    torch.cuda.synchronize()
    _log(f"warmup: {warmup} + {n} steps")
    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record(stream)
    for i in range(steps):
        step()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    return [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]


def other_workload(name: str, steps: int, warmup: int, cpu: bool = True, compare: bool = True) -> None:
    """Configs 1, 2, 4, 5 of the benchmark set (inputs resident in HBM)."""
    from nvsubquadratic_amd import causal_conv1d_hip as CC
    from nvsubquadratic_amd import fftconv_hip as F
    from nvsubquadratic_amd.workloads import (algorithmic_bytes_b2b, algorithmic_bytes_causal1d,
                                              algorithmic_bytes_nd, causal1d_case_fast, radial_filter)

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    extra = {}
    if name == "cfg1":
        B, D, L = 2, 128, 4096
        c = causal1d_case_fast(B, D, L, torch.float32, (1.0, 10.0), dev, seed=0)
        y = torch.empty_like(c.x)
        phase, dtype = "fwd", "f32"
        nbytes = algorithmic_bytes_causal1d(B, D, L, L, 4, "fwd")
        desc = "cfg1: causal FFT long conv fwd, B=2 D=128 L=4096 K=4096, FFT length 8192, fp32 I/O"

        def step():
            F.causal_fftconv1d_fwd_raw(c.x, c.k, c.s, y)

        def step_torch():
            with torch.no_grad():
                _torch_causal_fftconv1d(c.x, c.k, c.s)
    elif name == "cfg2":
        B, C, L, Kp, Km = 4, 4096, 8192, 3, 128
        x = torch.randn(B, 3 * C, L, device=dev, generator=gen).to(torch.bfloat16)
        wp = torch.randn(3 * C, Kp, device=dev, generator=gen)
        wm = torch.randn(C, Km, device=dev, generator=gen) / Km ** 0.5
        # fp32 accumulation; the k=128 mixer's products are three bf16 products of split operands
        phase, dtype = "fwd", "f32 (bf16x3 mixer products)"
        nbytes = algorithmic_bytes_b2b(B, C, L, Kp, Km, 2)
        desc = "cfg2: B2B short-conv block fwd (k=3 proj -> gate -> k=128 mixer -> gate), B=4 L=8192 D=4096, bf16 I/O"

        def step():
            with torch.no_grad():
                CC.b2b_causal_conv1d(x, wp, wm, None)

        def step_torch():
            with torch.no_grad():
                _torch_b2b(x, wp, wm, None)
    elif name == "cfg2-fwd-bwd":
        # report-only: the config-2 block with its backward (autograd), skip = 0 as in config 2
        B, C, L, Kp, Km = 4, 4096, 8192, 3, 128
        x = torch.randn(B, 3 * C, L, device=dev, generator=gen).to(torch.bfloat16).requires_grad_(True)
        wp = torch.randn(3 * C, Kp, device=dev, generator=gen).requires_grad_(True)
        wm = (torch.randn(C, Km, device=dev, generator=gen) / Km ** 0.5).requires_grad_(True)
        sk = torch.zeros(C, device=dev, requires_grad=True)
        g = torch.randn(B, C, L, device=dev, generator=gen).to(torch.bfloat16)
        phase, dtype = "fwd+bwd", "f32"
        nbytes = algorithmic_bytes_b2b(B, C, L, Kp, Km, 2, "fwd+bwd")
        desc = ("cfg2-fwd-bwd: B2B short-conv block fwd+bwd (k=3 proj -> gate -> k=128 mixer -> gate), "
                "B=4 L=8192 D=4096, bf16 I/O")

        def step():
            x.grad = wp.grad = wm.grad = sk.grad = None
            CC.b2b_causal_conv1d(x, wp, wm, sk).backward(g)
    elif name in ("cfg4", "cfg5"):
        nd = 2 if name == "cfg4" else 3
        B, C, size, sig = (16, 384, 128, (4.0, 64.0)) if nd == 2 else (2, 128, 64, (2.0, 32.0))
        x = torch.randn(B, C, *([size] * nd), device=dev, generator=gen).to(torch.bfloat16)
        k = radial_filter(C, size, sig[0], sig[1], nd, gen, dev)
        s = torch.randn(C, device=dev, generator=gen).to(torch.bfloat16)
        fn = F.fftconv2d_bhl if nd == 2 else F.fftconv3d_bhl
        phase, dtype = ("fwd", "f32") if nd == 2 else ("fwd+bwd", "f32")
        nbytes = algorithmic_bytes_nd(B, C, [size] * nd, [size] * nd, 2, phase)
        # FFT sizes: the reference's own F = S + K/2 per axis: config 4's forward keeps no state and runs the
        # one-kernel image forward on 192^2; config 5 the mixed-radix plan on 96^3
        fft = "FFT 192^2 (one-kernel image forward, mixed-radix)" if nd == 2 else "FFT 96^3 per axis (mixed-radix)"
        desc = (f"cfg{4 if nd == 2 else 5}: {nd}D non-causal FFT conv {phase}, B={B} C={C} {size}^{nd}, "
                f"filter {size}^{nd} fp32, {fft}, bf16 I/O")
        if nd == 2:
            def step():
                with torch.no_grad():
                    fn(x, k, s)

            def step_torch():
                with torch.no_grad():
                    _torch_fftconv_nd(x, k, s)
        else:
            xg, kg, sg = (t.detach().requires_grad_(True) for t in (x, k, s))
            g = torch.randn(x.shape, device=dev, generator=gen).to(torch.bfloat16)

            def step():
                xg.grad = kg.grad = sg.grad = None
                fn(xg, kg, sg).backward(g)

            def step_torch():
                xg.grad = kg.grad = sg.grad = None
                _torch_fftconv_nd(xg, kg, sg).backward(g)
    elif name in ("cfg4-circular", "well-rb"):
        # periodic boundaries (report-only): cfg4's shape with fft_padding="circular" (FFT 128^2, no padding),
        # and the rayleigh_benard Hyena layer (examples/well/v2/rayleigh_benard/hyena.py: 512x128 / patch 8 =
        # 64x16 tokens, H=384, batch 64, fft_padding=["circular", "zero"], kernel 64 x 31)
        from nvsubquadratic_amd import circular_fftconv_hip as C
        from nvsubquadratic_amd import mixed_fftconv_hip as M

        if name == "cfg4-circular":
            B, Ch, S, K, phase = 16, 384, (128, 128), (128, 128), "fwd"
            fn = C.circular_fftconv2d_fp32_bhl
            desc = ("cfg4-circular: 2D circular FFT conv fwd, B=16 C=384 128^2, filter 128^2 fp32, FFT 128^2, "
                    "bf16 I/O")
        else:
            B, Ch, S, K, phase = 64, 384, (64, 16), (64, 31), "fwd+bwd"
            fn = lambda x_, k_, s_: M.mixed_fftconv2d_fp32_bhl(x_, k_, (True, False), s_)  # noqa: E731
            desc = ("well-rb: 2D mixed-boundary FFT conv fwd+bwd (x periodic, y zero-padded), B=64 C=384 64x16, "
                    "filter 64x31 fp32, FFT 64x32, bf16 I/O")
        x = torch.randn(B, Ch, *S, device=dev, generator=gen).to(torch.bfloat16)
        k = torch.randn(1, Ch, *K, device=dev, generator=gen) / (K[0] * K[1]) ** 0.5
        s = torch.randn(Ch, device=dev, generator=gen).to(torch.bfloat16)
        dtype = "f32"
        nbytes = algorithmic_bytes_nd(B, Ch, list(S), list(K), 2, phase)
        if phase == "fwd":
            def step():
                with torch.no_grad():
                    fn(x, k, s)
        else:
            xg, kg, sg = (t.detach().requires_grad_(True) for t in (x, k, s))
            g = torch.randn(x.shape, device=dev, generator=gen).to(torch.bfloat16)

            def step():
                xg.grad = kg.grad = sg.grad = None
                fn(xg, kg, sg).backward(g)
    elif name == "hyena-gated":
        # report-only: the Hyena layer's gated long conv, fused, against the same layer composed of torch
        # gates around the HIP conv (hyena_nd.py:546,558,570), fwd+bwd
        import torch.nn.functional as Fn

        from nvsubquadratic_amd.gated_fftconv_hip import hyena_gated_causal_fftconv1d_bhl
        from nvsubquadratic_amd.workloads import algorithmic_bytes_gated

        B, Ch, L = 4, 1024, 8192
        q, kk, v = (torch.randn(B, Ch, L, device=dev, generator=gen).to(torch.bfloat16).requires_grad_(True)
                    for _ in range(3))
        w = (torch.randn(1, Ch, L, device=dev, generator=gen) / L ** 0.5).requires_grad_(True)
        sh = torch.randn(Ch, device=dev, generator=gen).to(torch.bfloat16).requires_grad_(True)
        g = torch.randn(B, Ch, L, device=dev, generator=gen).to(torch.bfloat16)
        phase, dtype = "fwd+bwd", "f32"
        nbytes = algorithmic_bytes_gated(B, Ch, L, L, 2)
        desc = ("hyena-gated: gated causal FFT conv fwd+bwd (z = q silu(k), y = (conv(z) + s z) sigmoid(v)), "
                "B=4 D=1024 L=8192 K=8192, bf16 I/O; gates as elementwise HIP kernels around the fused conv kernels "
                "both ways (at 2^25 elements they beat the gated forward kernel, which the library keeps for calls "
                "below 2^22 elements)")

        def clear():
            for t in (q, kk, v, w, sh):
                t.grad = None

        def step():
            clear()
            hyena_gated_causal_fftconv1d_bhl(q, kk, v, w, sh, "silu", "sigmoid").backward(g)

        def step_unfused():
            clear()
            z = q * Fn.silu(kk)
            (F.causal_fftconv1d_bhl(z, w, sh) * torch.sigmoid(v)).backward(g)

        if compare:
            extra["unfused_ms_per_step"] = round(statistics.mean(_time_steps(step_unfused, steps, warmup)), 4)
    elif name == "hyena-gated-2d":
        # report-only (2D): the gates inside the N-d conv's first and last passes, against torch's gate ops
        # around the same HIP conv (which keeps z for the backward) and the conv alone, fwd+bwd at cfg4's shape
        import torch.nn.functional as Fn

        from nvsubquadratic_amd.gated_fftconv_hip import hyena_gated_fftconv2d_bhl
        from nvsubquadratic_amd.workloads import algorithmic_bytes_gated

        B, Ch, X, K = 16, 384, 128, 128
        q, kk, v = (torch.randn(B, Ch, X, X, device=dev, generator=gen).to(torch.bfloat16).requires_grad_(True)
                    for _ in range(3))
        w = radial_filter(Ch, K, 4.0, 64.0, 2, gen, dev).unsqueeze(0).requires_grad_(True)
        sh = torch.randn(Ch, device=dev, generator=gen).to(torch.bfloat16).requires_grad_(True)
        g = torch.randn(B, Ch, X, X, device=dev, generator=gen).to(torch.bfloat16)
        phase, dtype = "fwd+bwd", "f32"
        nbytes = algorithmic_bytes_gated(B, Ch, X * X, K * K, 2)
        desc = ("hyena-gated-2d: gated 2D FFT conv fwd+bwd (z = q silu(k), y = (conv(z) + s z) silu(v)), "
                "B=16 C=384 128^2, filter 128^2 fp32, FFT 192^2 (mixed-radix), bf16 I/O; gate kernels around the conv")

        def clear():
            for t in (q, kk, v, w, sh):
                t.grad = None

        def step():
            clear()
            hyena_gated_fftconv2d_bhl(q, kk, v, w, sh, "silu").backward(g)

        def step_torch_gates():
            clear()
            (F.fftconv2d_bhl(q * Fn.silu(kk), w, sh) * Fn.silu(v)).backward(g)

        def step_conv_only():
            clear()
            F.fftconv2d_bhl(q, w, sh).backward(g)

        if compare:
            extra["torch_gates_ms_per_step"] = round(statistics.mean(_time_steps(step_torch_gates, steps, warmup)), 4)
            extra["conv_only_ms_per_step"] = round(statistics.mean(_time_steps(step_conv_only, steps, warmup)), 4)
    elif name == "siren-1d":
        # report-only: the SIREN filter of a long-context Hyena layer (kernels_nd.py:876, CKConvND's causal
        # half): HIP hidden stack + one readout GEMM, fwd+bwd, against the reference's torch layers on the same GPU
        import torch.nn.functional as Fn

        from nvsubquadratic_amd.siren_hip import siren_filter, siren_grid

        H, L, E, HD, nh = 4096, 262144, 32, 32, 2
        grid = siren_grid((L,), (1.0,), (L,), dev)[L - 1:].contiguous()  # [L, 1]: the points the causal crop keeps
        gen_c = torch.Generator().manual_seed(0)
        mk = lambda *shape, b: ((torch.rand(*shape, generator=gen_c) * 2 - 1) * b).to(dev).requires_grad_(True)  # noqa
        w0, b0 = mk(E, 1, b=2 * 3.14159 * 10.0), mk(E, b=1.0)
        hw = [mk(HD, E, b=(6 / E) ** 0.5)] + [mk(HD, HD, b=(6 / HD) ** 0.5) for _ in range(nh - 1)]
        hb = [mk(HD, b=1.0) for _ in range(nh)]
        wo, bo = mk(H, HD, b=(6 / HD) ** 0.5 / 512), mk(H, b=0.1)
        g = torch.randn(H, L, device=dev, generator=gen)
        phase, dtype = "fwd+bwd", "f32"
        nbytes = 2 * H * L * 4
        desc = ("siren-1d: SIREN filter synthesis fwd+bwd (pos-emb 32, 2 hidden layers of 32, readout to 4096 "
                "channels) on the 262144 causal points, fp32; writes k [H, L] and reads its gradient")

        def clear():
            for t in (w0, b0, *hw, *hb, wo, bo):
                t.grad = None

        def step():
            clear()
            siren_filter(grid, w0, b0, hw, hb, wo, bo).backward(g)

        def step_torch():
            clear()
            h = torch.sin(Fn.linear(grid, w0, b0))
            for w, b in zip(hw, hb):
                h = torch.sin(Fn.linear(h, w, b))
            Fn.linear(h, wo, bo).t().backward(g)

        if compare:
            extra["torch_layers_ms_per_step"] = round(statistics.mean(_time_steps(step_torch, steps, warmup)), 4)
    elif name == "siren-conv-1d":
        # report-only: a long-context Hyena layer's SIREN filter and causal conv together (CKConvND's causal path,
        # ckconv_nd.py:1149-1164, identity mask) at config 3's shape, the filter never formed
        # (siren_causal_fftconv1d), against the HIP composition that forms it (siren_filter, then the conv)
        from nvsubquadratic_amd.fftconv_hip import causal_fftconv1d_bhl
        from nvsubquadratic_amd.siren_hip import siren_causal_fftconv1d, siren_filter, siren_grid

        B, H, L, E, HD, nh = 1, 4096, 262144, 32, 32, 2
        grid = siren_grid((L,), (1.0,), (L,), dev)[L - 1:].contiguous()
        gen_c = torch.Generator().manual_seed(0)
        mk = lambda *shape, b: ((torch.rand(*shape, generator=gen_c) * 2 - 1) * b).to(dev).requires_grad_(True)  # noqa
        w0, b0 = mk(E, 1, b=2 * 3.14159 * 10.0), mk(E, b=1.0)
        hw = [mk(HD, E, b=(6 / E) ** 0.5)] + [mk(HD, HD, b=(6 / HD) ** 0.5) for _ in range(nh - 1)]
        hb = [mk(HD, b=1.0) for _ in range(nh)]
        wo, bo = mk(H, HD, b=(6 / HD) ** 0.5 / 512), mk(H, b=0.1)
        x = torch.randn(B, H, L, device=dev, generator=gen).to(torch.bfloat16).requires_grad_(True)
        sh = torch.randn(H, device=dev, generator=gen).to(torch.bfloat16).requires_grad_(True)
        g = torch.randn(B, H, L, device=dev, generator=gen).to(torch.bfloat16)
        phase, dtype = "fwd+bwd", "f32"
        nbytes = 5 * B * H * L * 2  # x, y (forward); g, x, gx (backward), bf16; the filter is not an operand
        desc = ("siren-conv-1d: SIREN filter (pos-emb 32, 2 hidden layers of 32) and causal FFT conv fwd+bwd, B=1 "
                "H=4096 L=K=262144, bf16 I/O, fp32 arithmetic; the filter [H, L] and its gradient never formed")

        def clear():
            for t in (w0, b0, *hw, *hb, wo, bo, x, sh):
                t.grad = None

        def step():
            clear()
            siren_causal_fftconv1d(x, grid, w0, b0, hw, hb, wo, bo, sh).backward(g)

        def step_composed():
            clear()
            causal_fftconv1d_bhl(x, siren_filter(grid, w0, b0, hw, hb, wo, bo), sh).backward(g)

        if compare:
            extra["composed_ms_per_step"] = round(statistics.mean(_time_steps(step_composed, steps, warmup)), 4)
    elif name == "hyena-norm":
        # report-only (norms): the Hyena output tail y * sigmoid(v) -> RMSNorm over channels -> channels-last
        # (hyena_nd.py:570-583) as one HIP pass per direction, against the reference's torch ops on the same GPU
        from nvsubquadratic_amd.norm_hip import hyena_output_norm

        B, Ch, X = 16, 384, 128
        y, v = (torch.randn(B, Ch, X, X, device=dev, generator=gen).to(torch.bfloat16).requires_grad_(True)
                for _ in range(2))
        w = (torch.rand(Ch, device=dev, generator=gen) + 0.5).requires_grad_(True)
        g = torch.randn(B, X, X, Ch, device=dev, generator=gen).to(torch.bfloat16)
        phase, dtype = "fwd+bwd", "f32"
        n = B * Ch * X * X
        nbytes = 8 * n * 2  # fwd: y, v in, out; bwd: g, y, v in, dy, dv out (bf16)
        desc = ("hyena-norm: Hyena output tail fwd+bwd, y * sigmoid(v) -> RMSNorm over C (eps 1e-6) -> [B, H, W, C], "
                "B=16 C=384 128^2 bf16, weight fp32")

        def clear():
            for t in (y, v, w):
                t.grad = None

        def step():
            clear()
            hyena_output_norm(y, v, w, 1e-6, "sigmoid").backward(g)

        def step_torch():
            clear()
            u = (y * torch.sigmoid(v)).movedim(1, -1)
            xf = u.float()
            out = (w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6))).to(u.dtype)
            out.contiguous().backward(g)

        if compare:
            extra["torch_ops_ms_per_step"] = round(statistics.mean(_time_steps(step_torch, steps, warmup)), 4)
    elif name == "hyena-groupnorm":
        # report-only (norms): the conv's input z = q * silu(k) -> GroupNorm(1, C) channels-first (hyena_nd.py:
        # 546-550, the reference configs' pixelhyena_norm), three HIP passes per direction, against torch's ops
        from nvsubquadratic_amd.norm_hip import gated_channel_groupnorm

        B, Ch, X = 16, 384, 128
        y, v = (torch.randn(B, Ch, X, X, device=dev, generator=gen).to(torch.bfloat16).requires_grad_(True)
                for _ in range(2))
        w = (torch.rand(Ch, device=dev, generator=gen) + 0.5).requires_grad_(True)
        bia = (0.1 * torch.randn(Ch, device=dev, generator=gen)).requires_grad_(True)
        g = torch.randn(B, Ch, X, X, device=dev, generator=gen).to(torch.bfloat16)
        phase, dtype = "fwd+bwd", "f32"
        n = B * Ch * X * X
        nbytes = 8 * n * 2  # fwd: y, v in, out; bwd: g, y, v in, dy, dv out (bf16)
        desc = ("hyena-groupnorm: Hyena conv input fwd+bwd, q * silu(k) -> GroupNorm(1, C) (eps 1e-5) channels-first, "
                "B=16 C=384 128^2 bf16, weight and bias fp32")

        def clear():
            for t in (y, v, w, bia):
                t.grad = None

        def step():
            clear()
            gated_channel_groupnorm(y, v, w, bia, 1, 1e-5, "silu").backward(g)

        def step_torch():
            clear()
            z = y * torch.nn.functional.silu(v)
            torch.nn.functional.group_norm(z, 1, w.to(z.dtype), bia.to(z.dtype), 1e-5).backward(g)

        if compare:
            extra["torch_ops_ms_per_step"] = round(statistics.mean(_time_steps(step_torch, steps, warmup)), 4)
    else:
        raise SystemExit(f"unknown workload {name}")
    ms_list = _time_steps(step, steps, warmup)
    ms = statistics.mean(ms_list)
    gbs = nbytes / (ms * 1e-3) / 1e9
    if compare and name in ("cfg1", "cfg2", "cfg4", "cfg5"):
        _log("reference torch path on the GPU")
        extra["torch_gpu_ms_per_step"] = _torch_gpu_ms(step_torch)
        extra["speedup_vs_torch_gpu"] = round(extra["torch_gpu_ms_per_step"] / ms, 2)
    if name in _COUNTER_PROFILES:
        extra["roofline_traffic_source"] = f"profiles/{_COUNTER_PROFILES[name]}"
    if cpu and name in ("cfg1", "cfg2", "cfg4", "cfg5"):
        _log("cpu baseline")
        extra["cpu_baseline"] = cpu_baseline_other(name)
    print(json.dumps({
        "metric": f"{name} {phase} algorithmic HBM GB/s, 1 MI355X",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 4), "ms_median": round(statistics.median(ms_list), 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
        "data": "synthetic", "config": {"workload": desc},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": nbytes,
                     "traffic": counter_traffic(_COUNTER_PROFILES[name]) if name in _COUNTER_PROFILES else None},
        **extra,
    }), flush=True)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-compare", action="store_true",
                    help="skip the comparison variants (the reference's torch path on the GPU, unfused compositions)")
    ap.add_argument("--cpu-channels", type=int, default=1024)
    ap.add_argument("--cpu-iters", type=int, default=3)
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--workload", default="cfg3", choices=["cfg1", "cfg2", "cfg2-fwd-bwd", "cfg3", "cfg4", "cfg5",
                                                              "cfg4-circular", "well-rb", "hyena-gated",
                                                              "hyena-gated-2d", "siren-1d", "siren-conv-1d",
                                                              "hyena-norm", "hyena-groupnorm"])
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py measures one GPU only: the causal FFT conv is depthwise and shards over channels with no "
            "communication; multi-GPU runs are not part of this build.",
            file=sys.stderr,
        )
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.workload != "cfg3":
        other_workload(args.workload, args.steps, args.warmup, cpu=not args.no_cpu, compare=not args.no_compare)
        return

    from nvsubquadratic_amd import _lib
    from nvsubquadratic_amd import fftconv_hip as F
    from nvsubquadratic_amd.workloads import algorithmic_bytes_causal1d, causal1d_case_fast, fft_flops_causal1d

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, D, L, K = CFG["B"], CFG["D"], CFG["L"], CFG["K"]
    _log("generating inputs on the GPU")
    c = causal1d_case_fast(B, D, L, torch.bfloat16, (CFG["a_lo"], CFG["a_hi"]), dev, seed=0)
    y = torch.empty_like(c.x)
    gx = torch.empty_like(c.x)
    gk = torch.empty_like(c.k)
    gs = torch.empty(D, dtype=torch.float32, device=dev)
    lib = _lib.get_lib()
    ws_bytes = max(lib.nsq_fftconv1d_causal_workspace_bytes(B, D, L, K, d) for d in (0, 1))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    _log(f"workspace {ws_bytes / 2**30:.1f} GiB")

    # The forward gets the backward-sized workspace, so it keeps its transformed
    # x and k there and the backward reuses them (as autograd would).
    def fwd():
        F.causal_fftconv1d_fwd_raw(c.x, c.k, c.s, y, ws)

    def bwd():
        F.causal_fftconv1d_bwd_raw(c.g, c.x, c.k, c.s, gx, gk, gs, ws, fwd_state=True)

    for _ in range(args.warmup):
        fwd()
        bwd()
    torch.cuda.synchronize()
    _log(f"warmup done ({args.warmup} steps)")

    stream = torch.cuda.current_stream(dev)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3 * args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev[3 * i].record(stream)
        fwd()
        ev[3 * i + 1].record(stream)
        bwd()
        ev[3 * i + 2].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    fwd_ms = [ev[3 * i].elapsed_time(ev[3 * i + 1]) for i in range(args.steps)]
    bwd_ms = [ev[3 * i + 1].elapsed_time(ev[3 * i + 2]) for i in range(args.steps)]
    step_ms = [a + b for a, b in zip(fwd_ms, bwd_ms)]
    ms = statistics.mean(step_ms)
    _log(f"timed {args.steps} steps: {ms:.3f} ms/step (events), wall {wall * 1e3 / args.steps:.3f} ms/step")

    nbytes = algorithmic_bytes_causal1d(B, D, L, K, 2, "fwd+bwd")
    gbs = nbytes / (ms * 1e-3) / 1e9
    flops = fft_flops_causal1d(B, D, L, K, "fwd+bwd")
    out = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "cfg3: causal FFT long conv fwd+bwd, B=1 D=4096 L=262144 K=262144, FFT length 2^19, "
                        "x/grad bf16, filter fp32, shortcut bf16",
            "B": B, "D": D, "L": L, "K": K, "io_dtype": "bf16", "filter_dtype": "fp32",
        },
        "phases_ms": {
            "fwd": round(statistics.mean(fwd_ms), 4),
            "bwd": round(statistics.mean(bwd_ms), 4),
            "fwd_median": round(statistics.median(fwd_ms), 4),
            "bwd_median": round(statistics.median(bwd_ms), 4),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "scope": "fwd+bwd launch sequence (all kernels of both calls); algorithmic bytes "
                     f"{nbytes} per step; traffic = HBM bytes per step from "
                     "profiles/fftconv1d_causal_cfg3_fwd_bwd_traffic.txt",
            "fft_tflops_radix2_count": round(flops / (ms * 1e-3) / 1e12, 2),
        },
    }
    if not args.no_compare:
        _log("reference torch path on the GPU")
        xg, kg, sg = (t.detach().requires_grad_(True) for t in (c.x, c.k, c.s))

        def step_torch():
            xg.grad = kg.grad = sg.grad = None
            _torch_causal_fftconv1d(xg, kg, sg).backward(c.g)

        out["torch_gpu_ms_per_step"] = _torch_gpu_ms(step_torch, steps=3)
        out["speedup_vs_torch_gpu"] = round(out["torch_gpu_ms_per_step"] / ms, 2)
    if not args.no_cpu:
        _log("cpu baseline")
        out["cpu_baseline"] = cpu_baseline(args.cpu_channels, args.cpu_iters)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
