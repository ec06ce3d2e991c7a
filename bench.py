#!/usr/bin/env python3
"""Benchmark of the Converse2D forward hot path on one MI355X.

Headline (value): Converse2D forward throughput in Gpix*ch/s on the roofline workload
(cfg3): B=16, C=64, 256x256, k=5, scale=1, padding=2 circular, fp32, synthetic N(0,1)
input, softmax-normalised seeded psf, zero bias.  One step = one module-level Converse2D forward
of that batch (padding, solve and crop fused; inputs resident in HBM).

The same JSON line carries:
  roofline      the Converse2D kernel's algorithmic bytes / measured average duration (HIP events on
                the launch stream) against 8 TB/s, plus HBM traffic per launch from the committed
                rocprofv3 PMC summary (profiles/traffic.json) when present
  cpu_baseline  the reference's own C++ op (oracle/_ref, built from the reference source) timed on
                this host's cores on the same workload, in a subprocess (its op namespace collides
                with this package's); falls back to the numpy oracle ("port") if it is not built
  extra         LayerNorm and 1x1+GELU rooflines at the cfg3 shape, single-layer cfg1 and cfg2 timings,
                Converse-DnCNN (cfg4) and Converse-USRNet (cfg5) images/s

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-model]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK = 8.0e12
# dense fp16 matrix-core peak; the 1x1 kernels form each fp32 product from three fp16 products
# (split fp16: hi and lo parts), so their matrix-core fraction counts 3 fp16 flops per flop
FP16_MFMA_PEAK = 2.5e15

CFG3 = dict(B=16, C=64, H=256, W=256, k=5, scale=1, padding=2, mode="circular", eps=1e-5)


def cfg3_bytes(c=CFG3):
    B, C, H, W, k, s = c["B"], c["C"], c["H"], c["W"], c["k"], c["scale"]
    return 4 * B * C * H * W + 4 * B * C * H * s * W * s + 4 * C * (k * k + 1)


def make_cfg3_inputs(torch):
    """Seeded on the CPU (generator seeds 0 and 1) so the GPU run and the CPU baseline see the same
    tensors."""
    return make_layer_inputs(torch, "cfg3")


# ------------------------------------------------------------------------------------------------
# CPU baseline worker (separate process: loads the reference op library, never this package)
# ------------------------------------------------------------------------------------------------
LAYER_CFGS = {
    # name: (B, C, H, W, k, scale, padding, input distribution)
    "cfg1": (1, 64, 128, 128, 5, 1, 2, "uniform"),
    "cfg2": (8, 64, 64, 64, 3, 2, 1, "normal"),
    "cfg3": (16, 64, 256, 256, 5, 1, 2, "normal"),
}


def make_layer_inputs(torch, name):
    """Seeded on the CPU (generator seeds 0 and 1: input, then softmax psf), zero bias."""
    B, C, H, W, k, s, p, dist = LAYER_CFGS[name]
    g0 = torch.Generator().manual_seed(0)
    x = torch.rand(B, C, H, W, generator=g0) if dist == "uniform" else torch.randn(B, C, H, W, generator=g0)
    g1 = torch.Generator().manual_seed(1)
    w = torch.softmax(torch.randn(1, C, k * k, generator=g1), dim=-1).reshape(1, C, k, k)
    return x, w, torch.zeros(1, C, 1, 1)


def _cpu_model_name():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_model_worker(args):
    """cfg4 / cfg5 on the host: this package's model classes with the PyTorch backend (the reference's
    own pure-PyTorch op sequence, restated) on CPU tensors, one image of each benchmark batch."""
    import torch

    os.environ["CONVERSE2D_BACKEND"] = "pytorch"
    cores = min(os.cpu_count() or 1, args.cpu_threads)
    torch.set_num_threads(cores)
    cpu = torch.device("cpu")
    out = {}
    m, x = make_dncnn(torch, cpu, batch=1)
    m2, x2, k2 = make_usrnet(torch, cpu, batch=1)
    for name, fn, per in (("cfg4", lambda: m(x), "Converse-DnCNN 1x256x256 (one image of the cfg4 batch)"),
                          ("cfg5", lambda: m2(x2, k2, 4), "Converse-USRNet 3x64x64 -> 256x256 x4, KernelNet(25) "
                                                          "(one image of the cfg5 batch)")):
        with torch.no_grad():
            t0 = time.perf_counter()
            fn()
            t = time.perf_counter() - t0
        out[name] = {"value": 1.0 / t, "unit": "images/s", "cores": torch.get_num_threads(), "kind": "port",
                     "sample": per + ", fp32, CONVERSE2D_BACKEND=pytorch on CPU tensors, 1 timed call",
                     "ms_per_image": t * 1e3}
    out["cpu_model"] = _cpu_model_name()
    print(json.dumps(out))


def cpu_worker(args):
    import torch
    import torch.nn.functional as F

    cores = min(os.cpu_count() or 1, args.cpu_threads)
    torch.set_num_threads(cores)
    name = args.cpu_case
    B, C, H, W, k, s, p, _ = LAYER_CFGS[name]
    c = dict(CFG3)
    x, w, b = make_layer_inputs(torch, name)
    ref_so = os.path.join(ROOT, "oracle", "_ref", "converse2d_ref.so")
    if os.path.exists(ref_so):
        torch.ops.load_library(ref_so)
        kind = "reference"

        def step():
            y = F.pad(x, [p] * 4, mode=c["mode"])
            x0 = y if s == 1 else F.interpolate(y, scale_factor=s, mode="nearest")
            out = torch.ops.converse2d.forward(y, x0, w, b, s, c["eps"])
            return out[..., p * s:-p * s, p * s:-p * s]
    else:
        sys.path.insert(0, ROOT)
        import numpy as np

        from oracle import converse_oracle as O
        kind = "port"
        xn, wn, bn = x.numpy(), w.numpy(), b.numpy()

        def step():
            return O.converse2d_module(xn, wn, bn, s, p, c["mode"], c["eps"], np.float32)

    iters = args.cpu_iters if name == "cfg3" else 4 * args.cpu_iters
    times = []
    with torch.no_grad():
        step()  # warmup
        for _ in range(iters):
            t0 = time.perf_counter()
            step()
            times.append(time.perf_counter() - t0)
    mean = statistics.mean(times)
    npix = B * C * H * s * W * s
    print(json.dumps({
        "value": npix / mean / 1e9, "unit": "Gpix*ch/s", "cores": torch.get_num_threads(), "kind": kind,
        "sample": f"{name} full batch (B{B} C{C} {H}x{W} k{k} s{s} p{p} circular, fp32), F.pad + reference "
                  f"converse2d::forward + crop, 1 warmup + {iters} timed calls, mean",
        "ms_per_call": mean * 1e3, "p50_ms": statistics.median(times) * 1e3, "cpu_model": _cpu_model_name(),
        "os_cpu_count": os.cpu_count()}))


def run_cpu_baseline(args, case="cfg3"):
    flag = ["--cpu-model-worker"] if case == "models" else ["--cpu-worker", "--cpu-case", case]
    cmd = [sys.executable, os.path.abspath(__file__), *flag, "--cpu-iters", str(args.cpu_iters),
           "--cpu-threads", str(args.cpu_threads)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        return {"value": None, "error": r.stderr[-400:]}
    return json.loads(r.stdout.strip().splitlines()[-1])


# ------------------------------------------------------------------------------------------------
# GPU measurements
# ------------------------------------------------------------------------------------------------
def spin_up(torch, fn, seconds):
    """Runs fn back to back for `seconds` of wall time before anything is measured.  From idle the GPU
    needs a fraction of a second of sustained load to reach its steady clock: measured on the box, the
    cfg3 forward went from 0.225 to 0.188 ms per call over its first ~0.5 s of back-to-back calls, so a
    run of a few dozen calls straight after start-up times the clock ramp, not the kernel.  Returns the
    number of calls made."""
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            fn()
        n += 20
        torch.cuda.synchronize()
    return n


def time_events(torch, fn, iters):
    """Average duration per call from HIP events on the current stream (the library launches on it)."""
    st = torch.cuda.current_stream()
    fn()
    fn()
    st.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(iters):
        fn()
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) / iters * 1e-3


def load_traffic(name):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


def synthetic_image(torch, g, H=256, W=256):
    """Smooth synthetic image in [0, 1]: the sum of 8 sinusoids (frequency U[1, 16] cycles per image,
    random orientation and phase) plus 4-8 random axis-aligned constant patches, min-max normalised."""
    yy, xx = torch.meshgrid(torch.arange(H, dtype=torch.float64) / H, torch.arange(W, dtype=torch.float64) / W,
                            indexing="ij")
    img = torch.zeros(H, W, dtype=torch.float64)
    for _ in range(8):
        f = 1 + 15 * torch.rand(1, generator=g, dtype=torch.float64)
        th = math.pi * torch.rand(1, generator=g, dtype=torch.float64)
        ph = 2 * math.pi * torch.rand(1, generator=g, dtype=torch.float64)
        img += torch.sin(2 * math.pi * f * (xx * torch.cos(th) + yy * torch.sin(th)) + ph)
    for _ in range(int(torch.randint(4, 9, (1,), generator=g))):
        r0, c0 = (int(v) for v in torch.randint(0, H - 16, (2,), generator=g))
        hh, ww = (int(v) for v in torch.randint(16, H // 2, (2,), generator=g))
        img[r0:r0 + hh, c0:c0 + ww] = 4 * (torch.rand(1, generator=g, dtype=torch.float64) - 0.5)
    img = (img - img.min()) / (img.max() - img.min())
    return img.float()


def make_dncnn(torch, dev, batch=8):
    """Converse-DnCNN (cfg4): default constructor (k7, p6, circular, 20 blocks, 796,353 params),
    random init (seed 0), B=8 synthetic 1x256x256 images plus N(0, (25/255)^2) noise, not clipped.
    batch < 8 gives the first images of the same batch."""
    sys.path.insert(0, ROOT)
    from conversenet_amd.converse_dncnn import ConverseDnCNN

    torch.manual_seed(0)
    m = ConverseDnCNN().to(dev).eval()
    g = torch.Generator().manual_seed(0)
    clean = torch.stack([synthetic_image(torch, g)[None] for _ in range(8)])
    x = (clean + torch.randn(clean.shape, generator=g) * (25 / 255))[:batch].to(dev)
    return m, x


def make_usrnet(torch, dev, batch=4):
    """Converse-USRNet (cfg5) with KernelNet(kernel_size=25), random init (seed 0), alpha1 / alpha2 /
    d.alpha drawn from N(0, 0.1) so the body blocks contribute.  Input: B=4 RGB 256x256 synthetic images
    blurred circularly by a seeded 25x25 anisotropic Gaussian (sigma1, sigma2 ~ U[0.7, 3], angle ~ U[0, pi),
    centred at (12, 12), sum 1), decimated [0::4, 0::4], plus N(0, (2.55/255)^2); the kernel is the
    model's second input, scale factor 4.  batch < 4 gives the first images of the same batch."""
    sys.path.insert(0, ROOT)
    from conversenet_amd.converse_usrnet import ConverseUSRNet

    torch.manual_seed(0)
    m = ConverseUSRNet(kernel_size=25)
    with torch.no_grad():
        for prm in (m.d.alpha, *[b.alpha1 for b in m.p.m_body], *[b.alpha2 for b in m.p.m_body]):
            prm.normal_(0, 0.1)
    m = m.to(dev).eval()
    g = torch.Generator().manual_seed(0)
    xs, ks = [], []
    for _ in range(batch):
        hr = torch.stack([synthetic_image(torch, g) for _ in range(3)]).double()
        s1, s2 = (0.7 + 2.3 * torch.rand(2, generator=g, dtype=torch.float64)).tolist()
        th = float(math.pi * torch.rand(1, generator=g, dtype=torch.float64))
        yy, xx = torch.meshgrid(torch.arange(25, dtype=torch.float64) - 12, torch.arange(25, dtype=torch.float64) - 12,
                                indexing="ij")
        u = xx * math.cos(th) + yy * math.sin(th)
        v = -xx * math.sin(th) + yy * math.cos(th)
        k = torch.exp(-0.5 * (u ** 2 / s1 ** 2 + v ** 2 / s2 ** 2))
        k = k / k.sum()
        kp = torch.zeros(256, 256, dtype=torch.float64)
        kp[:25, :25] = k
        kp = torch.roll(kp, shifts=(-12, -12), dims=(0, 1))
        blur = torch.fft.ifftn(torch.fft.fftn(hr, dim=(-2, -1)) * torch.fft.fftn(kp), dim=(-2, -1)).real
        lr = blur[:, 0::4, 0::4] + torch.randn(3, 64, 64, generator=g, dtype=torch.float64) * (2.55 / 255)
        xs.append(lr.float())
        ks.append(k.float()[None])
    return m, torch.stack(xs).to(dev), torch.stack(ks).to(dev)


def bench_model(torch, dev, iters=12):
    """Converse-DnCNN (cfg4) images/s, after 0.5 s of back-to-back forwards (steady clock)."""
    m, x = make_dncnn(torch, dev)
    with torch.no_grad():
        spin_up(torch, lambda: m(x), 0.5)
        t = time_events(torch, lambda: m(x), iters)
    return {"workload": "cfg4 Converse-DnCNN B8 1x256x256 fp32 (k7 p6, 20 blocks)", "ms_per_batch": t * 1e3,
            "images_per_s": 8 / t, "params": sum(p.numel() for p in m.parameters()), "iters": iters}


def bench_usrnet(torch, dev, iters=12):
    """Converse-USRNet (cfg5) images/s, after 0.5 s of back-to-back forwards (steady clock)."""
    m, x, k = make_usrnet(torch, dev)
    with torch.no_grad():
        spin_up(torch, lambda: m(x, k, 4), 0.5)
        t = time_events(torch, lambda: m(x, k, 4), iters)
    return {"workload": "cfg5 Converse-USRNet B4 3x64x64 -> 256x256 x4, KernelNet(25) fp32", "ms_per_batch": t * 1e3,
            "images_per_s": 4 / t, "params": sum(p.numel() for p in m.parameters()), "iters": iters}


def time_events_flushed(torch, fn, iters, flush):
    """Median duration of single calls, each preceded by a pass over a buffer larger than the 256 MB
    MALL (Infinity Cache), so every call starts with its inputs and tables out of the caches."""
    st = torch.cuda.current_stream()
    fn()
    st.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for e0, e1 in ev:
        flush()
        e0.record(st)
        fn()
        e1.record(st)
    st.synchronize()
    return statistics.median(e0.elapsed_time(e1) for e0, e1 in ev) * 1e-3


def bench_layer(torch, Fh, dev, name, iters, flush):
    """One Converse2D layer (module level, cached table) at a survey configuration: time and Gpix*ch/s,
    back to back (MALL-warm: cfg1's 8.4 MB and cfg2's 42 MB stay in the 256 MB MALL between calls) and
    with the MALL flushed before each call."""
    B, C, H, W, k, s, p, _ = LAYER_CFGS[name]
    x, w, b = (t.to(dev) for t in make_layer_inputs(torch, name))
    b = b.reshape(-1)
    fn = lambda: Fh.converse2d_fused(x, w, b, s, p, "circular", 1e-5)
    t = time_events(torch, fn, iters)
    tf = time_events_flushed(torch, fn, max(10, iters // 2), flush)
    nbytes = 4 * B * C * H * W + 4 * B * C * H * s * W * s + 4 * C * (k * k + 1)
    npix = B * C * H * s * W * s
    return {"workload": f"Converse2D B{B} C{C} {H}x{W} k{k} s{s} p{p} circular", "route": _route(Fh, x, w, s, p),
            "ms_mall_warm": t * 1e3, "Gpix*ch/s_mall_warm": npix / t / 1e9, "frac_hbm_mall_warm": nbytes / t / HBM_PEAK,
            "ms": tf * 1e3, "Gpix*ch/s": npix / tf / 1e9, "GB/s": nbytes / tf / 1e9, "frac_hbm": nbytes / tf / HBM_PEAK,
            "timing": "ms / Gpix*ch/s / frac_hbm: median single call after a 1 GiB read-modify-write pass "
                      "(MALL flushed); *_mall_warm: back-to-back calls"}


def _route(Fh, x, w, s, p):
    from conversenet_amd import _lib
    B, C, H, W = x.shape
    r = _lib.load().cvn_converse2d_route(B, C, H, W, w.shape[0], w.shape[2], w.shape[3], s, p)
    return {1: "fused", 2: "pfa268", 3: "generic"}.get(r, str(r))


def bench_copy(torch, Fh, dev, iters):
    """Attainable HBM bandwidth on this box: the library's copy kernel over 256 MiB (read) + 256 MiB
    (written), far beyond the MALL."""
    src = torch.randn(COPY_FLOATS, device=dev)
    dst = torch.empty_like(src)
    t = time_events(torch, lambda: Fh.copy_(dst, src), iters)
    return {"bytes": 8 * COPY_FLOATS, "ms": t * 1e3, "GB/s": 8 * COPY_FLOATS / t / 1e9,
            "frac_hbm": 8 * COPY_FLOATS / t / HBM_PEAK}


def bench_speed_grid(torch, dev, iters):
    """The reference's own timing grid (test/test_speed.py:137-146, 253-271): the op
    torch.ops.converse2d.forward(x, x0 = nearest(x), psf, 0, s) on B8 C8 256x256 for s in {1, 2, 3} and
    k in {3, 5, 7}, fp32, psf softmax-normalised (torch.manual_seed(0) as there), throughput
    B * (H s) * (W s) / t in Gpix/s (channels not counted, as there).  Forward only."""
    import torch.nn.functional as F
    from conversenet_amd import _lib
    lib = _lib.load()
    out = {"note": "op-level bytes = x (B C H W) + x0 and out (B C Hs Ws each), fp32; route: fused (s = 1, "
                   "x0 is x), op_planned (compile-time plans) or generic"}
    B, C, H, W = 8, 8, 256, 256
    for s in (1, 2, 3):
        for k in (3, 5, 7):
            torch.manual_seed(0)
            x = torch.randn(B, C, H, W, device=dev)
            x0 = x if s == 1 else F.interpolate(x, scale_factor=s, mode="nearest")
            w = torch.softmax(torch.randn(1, C, k * k, device=dev), dim=-1).view(1, C, k, k).contiguous()
            b = torch.zeros(1, C, 1, 1, device=dev)
            with torch.no_grad():
                t = time_events(torch, lambda: torch.ops.converse2d.forward(x, x0, w, b, s, 1e-5), iters)
            nbytes = 4 * B * C * H * W * (1 + (2 * s * s if s > 1 else 1))
            route = "fused" if s == 1 else {_lib.ROUTE_OP_PLANNED: "op_planned", _lib.ROUTE_GENERIC: "generic"}.get(
                lib.cvn_converse2d_op_route(H, W, s), "?")
            out[f"s{s}_k{k}"] = {"fwd_ms": t * 1e3, "fwd_gpix_per_s": B * H * s * W * s / t / 1e9, "route": route,
                                 "bytes": nbytes, "frac_hbm": nbytes / t / HBM_PEAK}
    return out


def bench_backward(torch, Fh, dev, x, w, bias, c, iters):
    """Converse2D backward at the cfg3 shape (the reference trains through autograd of its composite
    op, converse2d.cpp:223-227; test_speed.py:95-100 times forward + backward): the library's backward
    alone (all three gradients, and grad_x only), forward + backward through the autograd Function, and
    the same forward + backward through torch autograd of the reference op sequence (torch.fft on the
    GPU) for comparison."""
    from conversenet_amd import composite
    g = torch.Generator(device=dev).manual_seed(4)
    go = torch.randn(x.shape, device=dev, generator=g)
    b4 = bias.reshape(1, -1, 1, 1)
    s, p, mode, eps = c["scale"], c["padding"], c["mode"], c["eps"]
    out = {"workload": "cfg3 Converse2D backward, B16 C64 256x256 k5 s1 p2 circular, fp32"}
    bwd = lambda: Fh.converse2d_backward(go, x, w, b4, s, p, mode, eps)  # noqa: E731
    spin_up(torch, bwd, 0.5)  # the preceding measurements leave gaps in which the clock drops
    out["hip_backward_all_ms"] = time_events(torch, bwd, iters) * 1e3
    out["hip_backward_x_ms"] = time_events(
        torch, lambda: Fh.converse2d_backward(go, x, w, b4, s, p, mode, eps, True, False, False), iters) * 1e3
    xr, wr, br = (t.detach().clone().requires_grad_(True) for t in (x, w, b4))

    def hip_step():
        Fh.converse2d_train(xr, wr, br, s, p, mode, eps).backward(go)

    def torch_step():
        composite.converse2d_module(xr, wr, br, s, p, mode, eps).backward(go)

    out["hip_forward_backward_ms"] = time_events(torch, hip_step, iters) * 1e3
    out["torch_autograd_forward_backward_ms"] = time_events(torch, torch_step, max(2, iters // 2)) * 1e3
    out["speedup_vs_torch_autograd"] = out["torch_autograd_forward_backward_ms"] / out["hip_forward_backward_ms"]
    return out


def bench_block_pointwise(torch, Fh, dev, iters):
    """The channel-mixing kernels of one ConverseBlockAlphaVariant at the Converse-USRNet body shape
    (B4 C64 256x256, hidden 128): LN + 1x1 64->128 + GELU, 1x1 128->64 + alpha-scaled residual, the
    fused LN -> 1x1 -> GELU -> 1x1 -> residual branch, and the last two as the one tail kernel the
    blocks run.  Bytes are the algorithmic HBM bytes
    (each activation read or written once), FLOPs the 1x1 products (2 per multiply-add)."""
    B, C, H, W = 4, 64, 256, 256
    npx = B * H * W
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(B, C, H, W, device=dev, generator=g)
    h = torch.randn(B, 2 * C, H, W, device=dev, generator=g)
    w1 = torch.randn(2 * C, C, 1, 1, device=dev, generator=g) / 8
    b1 = torch.randn(2 * C, device=dev, generator=g)
    w2 = torch.randn(C, 2 * C, 1, 1, device=dev, generator=g) / 11
    b2 = torch.randn(C, device=dev, generator=g)
    lw, lb = torch.ones(C, device=dev), torch.zeros(C, device=dev)
    al = torch.randn(C, device=dev, generator=g)
    y = torch.empty_like(x)
    cases = {
        "ln_conv1x1_64_128_gelu": (lambda: Fh.conv1x1(x, w1, b1, act="gelu", ln=(lw, lb, 1e-5)),
                                   4 * npx * (C + 2 * C), 2 * npx * C * 2 * C),
        "conv1x1_128_64_residual": (lambda: Fh.conv1x1(h, w2, b2, residual=x, res_scale=al),
                                    4 * npx * (2 * C + C + C), 2 * npx * C * 2 * C),
        "ln_mlp_64_128_residual": (lambda: Fh.ln_mlp_residual(x, lw, lb, 1e-5, w1, b1, w2, b2, res_scale=al, out=y),
                                   4 * npx * 2 * C, 4 * npx * C * 2 * C),
        # the last two in one kernel (what the blocks run): reads h and x, writes the block output
        "tail_conv1x1_128_64_ln_mlp": (lambda: Fh.conv_ln_mlp_residual(h, x, w2, b2, lw, lb, 1e-5, w1, b1, w2, b2,
                                                                       al, al, out=y),
                                       4 * npx * (2 * C + C + C), 6 * npx * C * 2 * C),
    }
    out = {"workload": "ConverseBlockAlphaVariant channel mixing, B4 C64 256x256, hidden 128, fp32"}
    for name, (fn, nbytes, flops) in cases.items():
        t = time_events(torch, fn, iters)
        out[name] = {"us": t * 1e6, "GB/s": nbytes / t / 1e9, "frac_hbm": nbytes / t / HBM_PEAK,
                     "TFLOP/s": flops / t / 1e12, "frac_mfma_split_fp16": 3 * flops / t / FP16_MFMA_PEAK}
    return out


def only_kernel(torch, Fh, args, dev, x, step):
    """Runs one kernel family alone (warmup + steps) for rocprofv3 runs; prints a short JSON line.
    copy: the calibration copy kernel over COPY_FLOATS floats (bytes moved = 8 * COPY_FLOATS)."""
    if args.only == "converse2d":
        fn = step
    elif args.only == "layernorm":
        lw, lb = torch.ones(64, device=dev), torch.zeros(64, device=dev)
        fn = lambda: Fh.layernorm_cf(x, lw, lb, 1e-6)
    elif args.only == "conv1x1":
        torch.manual_seed(2)
        conv = torch.nn.Conv2d(64, 64, 1).to(dev)
        fn = lambda: Fh.conv1x1(x, conv.weight, conv.bias, act="gelu")
    elif args.only == "copy":
        src = torch.randn(COPY_FLOATS, device=dev)
        dst = torch.empty_like(src)
        fn = lambda: Fh.copy_(dst, src)
    elif args.only == "dncnn":
        m, xin = make_dncnn(torch, dev)
        torch.set_grad_enabled(False)
        fn = lambda: m(xin)
    elif args.only == "backward":
        g = torch.Generator(device=dev).manual_seed(4)
        go = torch.randn(x.shape, device=dev, generator=g)
        c, w, b = CFG3, step.w, step.b
        fn = lambda: Fh.converse2d_backward(go, x, w, b.reshape(1, -1, 1, 1), c["scale"], c["padding"], c["mode"],
                                            c["eps"])
    elif args.only == "usrnet":
        m, xin, kin = make_usrnet(torch, dev)
        torch.set_grad_enabled(False)
        fn = lambda: m(xin, kin, 4)
    elif args.only in ("cfg1", "cfg2"):
        B, C, H, W, k, s, p, _ = LAYER_CFGS[args.only]
        xl, wl, bl = (t.to(dev) for t in make_layer_inputs(torch, args.only))
        fn = lambda: Fh.converse2d_fused(xl, wl, bl.reshape(-1), s, p, "circular", 1e-5)
    elif args.only == "pfa268":
        # one Converse-DnCNN layer: B8 C128 256x256 k7 p6 circular (268 x 268 planes)
        g = torch.Generator().manual_seed(0)
        xl = torch.randn(8, 128, 256, 256, generator=g).to(dev)
        wl = torch.softmax(torch.randn(1, 128, 49, generator=g), -1).reshape(1, 128, 7, 7).to(dev)
        bl = torch.zeros(128, device=dev)
        fn = lambda: Fh.converse2d_fused(xl, wl, bl, 1, 6, "circular", 1e-5)
    elif args.only == "oppath":
        # torch.ops.converse2d.forward at cfg3 on the padded input (x0 = padded input), op table cached
        import torch.nn.functional as F
        c = CFG3
        y = F.pad(x, [c["padding"]] * 4, mode=c["mode"])
        b4 = step.b.reshape(1, -1, 1, 1)
        torch.set_grad_enabled(False)
        fn = lambda: torch.ops.converse2d.forward(y, y, step.w, b4, 1, c["eps"])
    elif args.only == "grid":
        # one point of the reference's speed grid: B8 C8 256x256, s = --grid-scale, k = 5, x0 = nearest(x)
        import torch.nn.functional as F
        torch.manual_seed(0)
        gs = args.grid_scale
        xg = torch.randn(8, 8, 256, 256, device=dev)
        x0 = xg if gs == 1 else F.interpolate(xg, scale_factor=gs, mode="nearest")
        wg = torch.softmax(torch.randn(1, 8, 25, device=dev), dim=-1).view(1, 8, 5, 5).contiguous()
        bg = torch.zeros(1, 8, 1, 1, device=dev)
        torch.set_grad_enabled(False)
        fn = lambda: torch.ops.converse2d.forward(xg, x0, wg, bg, gs, 1e-5)
    elif args.only == "tail":
        # the block tail with the next block's head at Converse-DnCNN's shape (B8, 64 / 128 channels, 256x256)
        g = torch.Generator(device=dev).manual_seed(3)
        t = torch.randn(8, 128, 256, 256, device=dev, generator=g)
        xr = torch.randn(8, 64, 256, 256, device=dev, generator=g)
        w0 = torch.randn(64, 128, 1, 1, device=dev, generator=g) / 11
        w1 = torch.randn(128, 64, 1, 1, device=dev, generator=g) / 8
        b0, b1 = torch.randn(64, device=dev, generator=g), torch.randn(128, device=dev, generator=g)
        lw, lb = torch.ones(64, device=dev), torch.zeros(64, device=dev)
        fn = lambda: Fh.conv_ln_mlp_residual(t, xr, w0, b0, lw, lb, 1e-5, w1, b1, w0, b0,
                                             head=(lw, lb, 1e-5, w1, b1))
    else:
        raise SystemExit(f"unknown --only {args.only}")
    spin_up(torch, fn, args.spinup)
    for _ in range(args.warmup):
        fn()
    torch.cuda.synchronize()
    t = time_events(torch, fn, args.steps)
    print(json.dumps({"only": args.only, "steps": args.steps, "ms_per_call": t * 1e3}))
    return 0


COPY_FLOATS = 64 * 1024 * 1024  # 256 MiB read + 256 MiB written per copy


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--spinup", type=float, default=1.5,
                    help="seconds of back-to-back calls before the warmup steps (GPU clock ramp); 0 for PMC runs")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-model", action="store_true")
    ap.add_argument("--cpu-worker", action="store_true")
    ap.add_argument("--cpu-case", default="cfg3", choices=sorted(LAYER_CFGS))
    ap.add_argument("--cpu-model-worker", action="store_true")
    ap.add_argument("--cpu-iters", type=int, default=3)
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--only", choices=["converse2d", "layernorm", "conv1x1", "copy", "dncnn", "usrnet", "backward",
                                       "cfg1", "cfg2", "pfa268", "tail", "oppath", "grid"],
                    help="run one kernel family alone (for rocprofv3)")
    ap.add_argument("--grid-scale", type=int, default=2, choices=[1, 2, 3],
                    help="scale of the speed-grid point --only grid runs")
    args = ap.parse_args()

    if args.cpu_worker:
        cpu_worker(args)
        return 0
    if args.cpu_model_worker:
        cpu_model_worker(args)
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the Converse2D path shards over the batch with no exchange, "
              "so every GPU runs this same per-GPU workload; run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    sys.path.insert(0, ROOT)
    from conversenet_amd import functional as Fh

    dev = torch.device("cuda", 0)
    c = CFG3
    x, w, b = (t.to(dev) for t in make_cfg3_inputs(torch))
    bias = b.reshape(-1)

    def step():
        return Fh.converse2d_fused(x, w, bias, c["scale"], c["padding"], c["mode"], c["eps"])
    step.w, step.b = w, bias

    if args.only:
        return only_kernel(torch, Fh, args, dev, x, step)

    spun = spin_up(torch, step, args.spinup)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    per_call = time_events(torch, step, args.steps)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps
    npix = c["B"] * c["C"] * c["H"] * c["scale"] * c["W"] * c["scale"]
    nbytes = cfg3_bytes()
    achieved = nbytes / per_call
    roofline = {"bound": "hbm", "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": achieved / HBM_PEAK, "traffic": load_traffic("converse2d_cfg3"),
                "kernel": "converse2d forward (all launches of one call)", "bytes_per_launch": nbytes}

    extra = {}
    # transfer-table build (runs once per weight change; cached across calls like the reference OTF)
    t_tab = time_events(torch, lambda: Fh.converse2d_fused(x, w, bias, c["scale"], c["padding"], c["mode"],
                                                           c["eps"], cache=False), max(5, args.steps // 4))
    extra["converse2d_uncached_ms"] = t_tab * 1e3
    extra["transfer_table_ms"] = (t_tab - per_call) * 1e3
    # LayerNorm (eps 1e-6) and 1x1 64->64 + GELU at the cfg3 shape
    lw = torch.ones(c["C"], device=dev)
    lb = torch.zeros(c["C"], device=dev)
    t_ln = time_events(torch, lambda: Fh.layernorm_cf(x, lw, lb, 1e-6), max(10, args.steps // 2))
    ln_bytes = 8 * x.numel() + 8 * c["C"]
    torch.manual_seed(2)
    conv = torch.nn.Conv2d(64, 64, 1).to(dev)
    t_cv = time_events(torch, lambda: Fh.conv1x1(x, conv.weight, conv.bias, act="gelu"), max(10, args.steps // 2))
    cv_bytes = 4 * x.numel() * 2 + 4 * (64 * 64 + 64)
    cv_flops = 2 * x.numel() * 64
    extra["layernorm_cf"] = {"ms": t_ln * 1e3, "GB/s": ln_bytes / t_ln / 1e9, "frac_hbm": ln_bytes / t_ln / HBM_PEAK}
    extra["conv1x1_gelu_64"] = {"ms": t_cv * 1e3, "GB/s": cv_bytes / t_cv / 1e9,
                                "frac_hbm": cv_bytes / t_cv / HBM_PEAK, "TFLOP/s": cv_flops / t_cv / 1e12,
                                "frac_mfma_split_fp16": 3 * cv_flops / t_cv / FP16_MFMA_PEAK}
    extra["block_pointwise"] = bench_block_pointwise(torch, Fh, dev, max(10, args.steps // 2))
    extra["converse2d_backward"] = bench_backward(torch, Fh, dev, x, w, bias, c, max(10, args.steps // 2))
    if not args.no_model:
        extra["converse_dncnn"] = bench_model(torch, dev)
        extra["converse_usrnet"] = bench_usrnet(torch, dev)
    flush_buf = torch.empty(256 * 1024 * 1024, device=dev)  # 1 GiB

    def flush():
        flush_buf.add_(1.0)

    extra["cfg1"] = bench_layer(torch, Fh, dev, "cfg1", max(20, args.steps), flush)
    extra["cfg2"] = bench_layer(torch, Fh, dev, "cfg2", max(20, args.steps), flush)
    del flush_buf
    extra["copy"] = bench_copy(torch, Fh, dev, max(10, args.steps // 2))
    # the operator path (what the reference's own Converse2D calls through torch.ops.converse2d.forward):
    # padding and x0 = nearest in torch, the library's op kernels with the cached op table
    import torch.nn.functional as F
    y = F.pad(x, [c["padding"]] * 4, mode=c["mode"])
    b4 = bias.reshape(1, -1, 1, 1)
    with torch.no_grad():
        t_op = time_events(torch, lambda: torch.ops.converse2d.forward(y, y, w, b4, 1, c["eps"]),
                           max(5, args.steps // 5))
    extra["cfg3_operator_path"] = {"ms": t_op * 1e3, "Gpix*ch/s": npix * (260 * 260) / (256 * 256) / t_op / 1e9,
                                   "note": "converse2d::forward on the padded 260x260 input (x0 = padded input), "
                                           "uncropped output, op table cached; padding not timed"}
    extra["reference_speed_grid"] = bench_speed_grid(torch, dev, max(10, args.steps // 5))

    cpu = None
    if not args.no_cpu:
        cpu = run_cpu_baseline(args)
        for name in ("cfg1", "cfg2"):
            extra[name]["cpu_baseline"] = run_cpu_baseline(args, name)
        if not args.no_model:
            models = run_cpu_baseline(args, "models")
            for name, key in (("cfg4", "converse_dncnn"), ("cfg5", "converse_usrnet")):
                if name in models and key in extra:
                    extra[key]["cpu_baseline"] = models[name]

    line = {
        "metric": "Converse2D fwd Gpix*ch/s", "value": npix / per_call / 1e9, "unit": "Gpix*ch/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": per_call * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": "cfg3 Converse2D forward B16 C64 256x256 k5 s1 p2 circular (module-level: pad, "
                               "solve, crop)", "B": c["B"], "C": c["C"], "H": c["H"], "W": c["W"], "k": c["k"],
                   "scale": c["scale"], "padding": c["padding"], "padding_mode": c["mode"], "parallelism": "none"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "wall_ms_per_step": wall * 1e3,
        "spinup": {"seconds": args.spinup, "calls": spun,
                   "note": "back-to-back steps before the warmup steps, so the timed steps run at the GPU's "
                           "steady clock"},
        "extra": extra,
        "host": platform.node(),
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
