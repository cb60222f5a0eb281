#!/usr/bin/env python3
"""Benchmark: sparse conv3x3 us/layer + HBM GB/s at 99% spike sparsity.

Default workload (N=1 GPU): the Spiking-ResNet50 layer1 3x3 conv shape at
T=16, batch 32 (512 frames of 64x56x56 fp32 binary spikes, i.i.d.
Bernoulli(0.01) = 99% sparsity) -> 64 channels, Kaiming-normal fp32 weights,
through SparseConv2d (Stage-1 prescan + Stage-2 gather conv).  Inputs are
resident in HBM before timing; data is synthetic.

Prints ONE JSON line on stdout.  Extra per-config lines go to stderr and
into the JSON's "extra" object.  Baselines: MIOpen (F.conv2d on the same
GPU) and the CPU oracle (F.conv2d on host cores, bounded sample).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

import torch  # noqa: E402

METRIC = "sparse conv3x3 µs/layer + HBM GB/s at 99% spike sparsity, vs MIOpen & CPU"
HBM_PEAK_GBS = 8000.0

WORKLOADS = {
    # name: (frames, C_in, H, W, C_out, k, s, generator, density, images)
    "resnet50_layer1_conv3x3": (512, 64, 56, 56, 64, 3, 1, "iid", 0.01, 32),
    "config1_conv3x3": (32, 64, 32, 32, 64, 3, 1, "iid", 0.02, 8),
    "resnet50_layer2_conv3x3": (512, 128, 28, 28, 128, 3, 1, "iid", 0.01, 32),
    "resnet50_layer3_conv3x3": (512, 256, 14, 14, 256, 3, 1, "iid", 0.01, 32),
    "resnet50_layer2_0_conv3x3_s2": (512, 128, 56, 56, 128, 3, 2, "iid", 0.01, 32),
    "resnet50_layer3_0_conv3x3_s2": (512, 256, 28, 28, 256, 3, 2, "iid", 0.01, 32),
    "resnet50_layer4_0_conv3x3_s2": (512, 512, 14, 14, 512, 3, 2, "iid", 0.01, 32),
    "config2_conv1x1": (512, 256, 56, 56, 64, 1, 1, "clustered", 0.0, 32),
    # Time-step bursts as in the live network (one step of 16 dense): the
    # dense-tile branch's workloads.
    "resnet50_layer3_0_conv3x3_s2_bursty": (512, 256, 28, 28, 256, 3, 2, "bursty", 0.01, 32),
    "resnet50_layer4_0_conv3x3_s2_bursty": (512, 512, 14, 14, 512, 3, 2, "bursty", 0.01, 32),
}
LIF_WORKLOAD = "config4_conv3x3_lif"  # T=8, N=64, C 128->128, 28x28, Bernoulli(0.005)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_input(shape, gen, density, dev, seed=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    if gen == "iid":
        return (torch.rand(shape, generator=g, device=dev) < density).float()
    if gen == "bursty":
        # Frames t * 32 + n of T = 16 steps: step 11 at 10x the mean density,
        # step 5 at 3.2x, the other fourteen at 0.2x (mean = density).
        n = shape[0]
        p = torch.full((n, 1, 1, 1), 0.2 * density, device=dev)
        per = n // 16
        p[11 * per:12 * per] = 10.0 * density
        p[5 * per:6 * per] = 3.2 * density
        return (torch.rand(shape, generator=g, device=dev) < p).float()
    # Clustered: 16x16 blocks active with p=0.03,
    # Bernoulli(0.3) inside active blocks.
    n, c, h, w = shape
    gh, gw = -(-h // 16), -(-w // 16)
    gate = (torch.rand((n, c, gh, gw), generator=g, device=dev) < 0.03).float()
    gate = gate.repeat_interleave(16, 2).repeat_interleave(16, 3)[:, :, :h, :w]
    return gate * (torch.rand(shape, generator=g, device=dev) < 0.3).float()


def make_conv(c_in, c_out, k, s, dev, half_weights=False):
    torch.manual_seed(1)
    conv = torch.nn.Conv2d(c_in, c_out, k, s, (k - 1) // 2, bias=False)
    torch.nn.init.kaiming_normal_(conv.weight, mode="fan_out", nonlinearity="relu")
    if half_weights:
        conv = conv.half()
    return conv.to(dev)


MIN_TIMED_MS = 2.0  # smallest timed region: amortises the first launch's latency and the event pair


def time_gpu(fn, steps, warmup):
    """ms per step over `steps` back-to-back steps after `warmup`; when those
    take under MIN_TIMED_MS (the small layers), the timed region is
    lengthened to at least MIN_TIMED_MS of work."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    while True:
        start.record()
        for _ in range(steps):
            fn()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end)
        if ms >= MIN_TIMED_MS:
            return ms / steps  # ms per step
        steps = int(steps * MIN_TIMED_MS / max(ms, 1e-3) * 1.2) + 1


def kernel_times(fn, steps):
    """Average per-launch duration of each library kernel, from HIP events
    the library records on the launch stream around every kernel."""
    from sparseflow_amd import _lib

    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    try:
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        stats = _lib.timing_collect()
    finally:
        _lib.timing_enable(False)
    return {k: (cnt, ms / cnt) for k, (cnt, ms) in stats.items() if cnt > 0}


def bench_conv(name, steps, warmup, dev, with_miopen=True):
    from sparseflow_amd.Ops.sparse_conv2d import SparseConv2d

    frames, c_in, h, w, c_out, k, s, gen, dens, images = WORKLOADS[name]
    half_w = name.startswith("config2")
    x = make_input((frames, c_in, h, w), gen, dens, dev)
    conv = make_conv(c_in, c_out, k, s, dev, half_weights=half_w)
    sp = SparseConv2d.from_dense(conv).to(dev)
    sp.set_inference_mode(True)
    h_out, w_out = (h + 2 * ((k - 1) // 2) - k) // s + 1, (w + 2 * ((k - 1) // 2) - k) // s + 1
    x_bytes = x.numel() * 4
    y_bytes = frames * c_out * h_out * w_out * 4
    w_bytes = c_out * c_in * k * k * 4
    alg_bytes = x_bytes + w_bytes + y_bytes

    with torch.no_grad():
        step = lambda: sp(x)  # noqa: E731
        ms = time_gpu(step, steps, warmup)
        kt = kernel_times(step, max(5, min(steps, 20)))
        miopen_ms = None
        if with_miopen:
            log(f"[bench] {name}: sparse path timed; MIOpen baseline next")
            torch.backends.cudnn.benchmark = True
            wd = conv.weight.float()
            dense = lambda: torch.nn.functional.conv2d(x, wd, None, s, (k - 1) // 2)  # noqa: E731
            miopen_ms = time_gpu(dense, max(5, steps // 2), 3)
    density = float(x.mean().item())
    kernels_us = {k2: v[1] * 1e3 for k2, v in kt.items()}
    # Algorithmic bytes per launch: the prescan reads x; a Stage-2 kernel
    # reads W and writes y; the fused kernel (prescan inside) also reads x.
    kernel_bytes = {k2: (x_bytes if k2.startswith("prescan") else
                         x_bytes + y_bytes + w_bytes if k2 == "conv_rows_fused" else y_bytes + w_bytes) for k2 in kt}
    res = {
        "workload": name,
        "us_per_layer": ms * 1e3,
        "images_per_s": images / (ms * 1e-3),
        "frames_per_s": frames / (ms * 1e-3),
        "hbm_gbs": alg_bytes / (ms * 1e-3) / 1e9,
        "hbm_frac": alg_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "alg_bytes": alg_bytes,
        "input_density": density,
        "kernels_us": kernels_us,
        "kernel_bytes": kernel_bytes,
        "traffic": {k2: measured_traffic(name, k2) for k2 in kt},
        "miopen_us": None if miopen_ms is None else miopen_ms * 1e3,
        "speedup_vs_miopen": None if miopen_ms is None else miopen_ms / ms,
    }
    del x, sp
    return res


def bench_lif(steps, warmup, dev, with_miopen=True):
    from sparseflow_amd.Kernels.fused_conv_lif import sparse_fused_conv_lif_multistep
    from sparseflow_amd import _lib

    T, N, C, H, W, Co = 8, 64, 128, 28, 28, 128
    x = make_input((T * N, C, H, W), "iid", 0.005, dev).reshape(T, N, C, H, W)
    conv = make_conv(C, Co, 3, 1, dev)
    wt = _lib.tap_major_weight(conv.weight)
    ws = torch.empty(_lib.conv_lif_workspace_size(_lib.conv_desc(N, C, H, W, Co, H, W, 3, 1, 1, 0, 0), T),
                     dtype=torch.uint8, device=dev)
    alg = x.numel() * 4 + Co * C * 9 * 4 + T * N * Co * H * W * 4 + N * Co * H * W * 4
    with torch.no_grad():
        step = lambda: sparse_fused_conv_lif_multistep(x, conv.weight, None, w_tap=wt, workspace=ws)  # noqa: E731
        ms = time_gpu(step, steps, warmup)
        kt = kernel_times(step, max(5, min(steps, 20)))
        miopen_ms = None
        if with_miopen:
            log(f"[bench] {LIF_WORKLOAD}: sparse path timed; MIOpen baseline next")
            torch.backends.cudnn.benchmark = True
            xf = x.reshape(T * N, C, H, W)

            def dense():
                cur = torch.nn.functional.conv2d(xf, conv.weight, None, 1, 1).reshape(T, N, Co, H, W)
                v = torch.zeros(N, Co, H, W, device=dev)
                for t in range(T):
                    hmem = v + (cur[t] - v) / 2.0
                    s_t = (hmem >= 1.0).float()
                    v = torch.where(s_t.bool(), torch.zeros_like(hmem), hmem)
                return v

            miopen_ms = time_gpu(dense, max(5, steps // 2), 3)
    return {
        "workload": LIF_WORKLOAD,
        "us_per_layer": ms * 1e3,
        "images_per_s": N / (ms * 1e-3),
        "hbm_gbs": alg / (ms * 1e-3) / 1e9,
        "hbm_frac": alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "alg_bytes": alg,
        "kernels_us": {k: v[1] * 1e3 for k, v in kt.items()},
        "traffic": {k: measured_traffic(LIF_WORKLOAD, k) for k in kt},
        "miopen_us": None if miopen_ms is None else miopen_ms * 1e3,
        "speedup_vs_miopen": None if miopen_ms is None else miopen_ms / ms,
    }


def cpu_baseline(name, target_seconds=12.0):
    """The oracle's dense conv (F.conv2d in fp32 on host cores) -- the
    reference's CPU fallback path -- on a bounded sample of the workload."""
    from oracle.conv import conv2d_ref

    frames, c_in, h, w, c_out, k, s, gen, dens, _ = WORKLOADS[name]
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    sample = min(frames, 64)
    x = make_input((sample, c_in, h, w), gen, dens, torch.device("cpu"))
    conv = make_conv(c_in, c_out, k, s, torch.device("cpu"))
    wt = conv.weight.detach()
    for _ in range(2):
        conv2d_ref(x, wt, None, s, (k - 1) // 2, dtype=torch.float32)
    times = []
    t_end = time.perf_counter() + target_seconds
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        conv2d_ref(x, wt, None, s, (k - 1) // 2, dtype=torch.float32)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": med * (frames / sample) * 1e6,
        "unit": "us/layer",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{sample} of {frames} frames of {name}, F.conv2d fp32 via oracle.conv.conv2d_ref, "
                  f"median of {len(times)} runs after 2 warmup, scaled x{frames / sample:g}; "
                  f"os.cpu_count()={os.cpu_count()}, cpu='{cpu_model}'",
    }


E2E_WORKLOAD = "resnet50_e2e"  # T=16, batch 32, 3x224x224, images/s
# The same network with every neuron layer's threshold calibrated to ~1% spike
# density (random init at v_th = 1 is silent past the first neuron layer).
E2E_LIVE_WORKLOAD = "resnet50_e2e_live"
E2E_LIVE_DENSITY = 0.01
ATTN_WORKLOAD = "config5_spikformer_block"  # T=4, N=64, 196 tokens, dim 384, 12 heads, Bernoulli(0.1)


# The 3x3 sparse convs whose live inputs the live run times on their own:
# one per stage shape (stride 1 and the stride-2 first blocks).
LIVE_LAYERS = ("layer1.0.conv2", "layer2.0.conv2", "layer2.1.conv2", "layer3.0.conv2", "layer3.1.conv2",
               "layer4.0.conv2")


def spike_spread(x, stride, T):
    """How the spikes of x [frames, C, H, W] (frames = t*N + n) are spread,
    computed on the CPU: density per frame and per time step, channel
    concentration, and the count of active (tap, channel) pairs per output
    pixel of a 3x3 conv (stride `stride`, padding 1) -- the walk length of
    that pixel -- with its ratio of tile maximum to tile mean over tiles of
    64 consecutive output pixels (a lane = pixel wavefront walks as long as
    its busiest pixel)."""
    x = x.detach().float().cpu()
    F_, C, H, W = x.shape
    dens = float(x.mean())
    pf = x.mean(dim=(1, 2, 3))
    pt = pf.reshape(T, -1).mean(1)
    pc = x.mean(dim=(0, 2, 3))
    top = torch.sort(pc, descending=True).values
    k10 = max(1, C // 10)
    per_px = x.sum(1, keepdim=True)                                   # active channels per input pixel
    rf = torch.nn.functional.conv2d(per_px, torch.ones(1, 1, 3, 3), stride=stride, padding=1)[:, 0]
    flat = rf.reshape(-1)
    n64 = flat.numel() // 64 * 64
    tiles = flat[:n64].reshape(-1, 64)
    tm = tiles.mean(1)
    busy = tm > 0
    # Tiles the pixel-tile kernel hands to the matrix cores (C_in > 128): a
    # pixel with 16 or more active (tap, channel) pairs among channels 0..31.
    rf32 = torch.nn.functional.conv2d(x[:, :32].sum(1, keepdim=True), torch.ones(1, 1, 3, 3), stride=stride,
                                      padding=1)[:, 0].reshape(-1)
    hot = (rf32 >= 16).float()
    hot = torch.nn.functional.pad(hot, (0, (-hot.numel()) % 64)).reshape(-1, 64).amax(1)
    return {
        "density": round(dens, 6),
        "frame_density_cv": round(float(pf.std() / max(pf.mean(), 1e-12)), 3),
        "frame_density_max_over_mean": round(float(pf.max() / max(pf.mean(), 1e-12)), 2),
        "density_by_step": [round(float(v), 5) for v in pt],
        "dead_channel_frac": round(float((pc == 0).float().mean()), 3),
        "top10pct_channel_spike_share": round(float(top[:k10].sum() / max(top.sum(), 1e-12)), 3),
        "rf_count_mean": round(float(flat.mean()), 2),
        "rf_count_p99": round(float(torch.quantile(flat[:1 << 22], 0.99)), 1),
        "rf_count_max": int(flat.max()),
        "tile_max_over_mean": round(float((tiles.max(1).values[busy] / tm[busy]).mean()), 2) if busy.any() else 0.0,
        "dense_tiles": int(hot.sum()) if C > 128 else 0,
        "tiles": int(hot.numel()),
    }


def live_layer_study(model, img, dev, steps, T):
    """The 3x3 sparse convs of the calibrated network (LIVE_LAYERS) on the
    inputs they receive in its forward, timed on their own next to i.i.d.
    Bernoulli input of the same shape and density; per-kernel times from the
    library's HIP events; how the spikes are spread (spike_spread) for both
    inputs."""
    from sparseflow_amd.neuron import reset_net

    mods = dict(model.named_modules())
    captured = {}
    hooks = [mods[n].register_forward_pre_hook(lambda _m, a, n=n: captured.__setitem__(n, a[0].detach().clone()))
             for n in LIVE_LAYERS if n in mods]
    with torch.no_grad():
        reset_net(model)
        model(img)
    for h in hooks:
        h.remove()
    out = {}
    for name in LIVE_LAYERS:
        if name not in captured:
            continue
        x = captured.pop(name)  # a copy: no neuron-handed map, so the module prescans it
        mod = mods[name]
        s = mod.stride[0]
        live = spike_spread(x, s, T)
        xi = make_input(tuple(x.shape), "iid", live["density"], dev, seed=7)
        with torch.no_grad():
            live_us = time_gpu(lambda: mod(x), steps, 3) * 1e3
            iid_us = time_gpu(lambda: mod(xi), steps, 3) * 1e3
            kl = kernel_times(lambda: mod(x), max(3, steps // 2))
            ki = kernel_times(lambda: mod(xi), max(3, steps // 2))
        iid = spike_spread(xi, s, T)
        out[name] = {
            "shape": list(x.shape), "stride": s, "c_out": mod.out_channels,
            "us_live": round(live_us, 1), "us_iid": round(iid_us, 1), "live_over_iid": round(live_us / iid_us, 2),
            "kernels_us_live": {k: round(v[1] * 1e3, 1) for k, v in kl.items()},
            "kernels_us_iid": {k: round(v[1] * 1e3, 1) for k, v in ki.items()},
            "spread_live": live,
            "spread_iid": {k: iid[k] for k in ("frame_density_cv", "dead_channel_frac", "top10pct_channel_spike_share",
                                               "rf_count_mean", "rf_count_p99", "rf_count_max", "tile_max_over_mean",
                                               "dense_tiles")},
        }
        log(f"[bench] live layer {name}: live {live_us:.1f} us, iid {iid_us:.1f} us; "
            f"tile max/mean live {live['tile_max_over_mean']} iid {iid['tile_max_over_mean']}")
        del x, xi
    return out


def spike_flips(sparse_model, dense_model, img):
    """Per neuron layer, the fraction of spikes that differ between the
    optimized and the dense model on the same input (a spike that flips at a
    threshold tie propagates to the layers after it)."""
    from sparseflow_amd.neuron import LIFNode, reset_net

    def record(m):
        outs = {}
        hooks = [mod.register_forward_hook(lambda _m, _i, o, n=name: outs.__setitem__(n, o > 0.5))
                 for name, mod in m.named_modules() if isinstance(mod, LIFNode)]
        with torch.no_grad():
            reset_net(m)
            m(img)
        for h in hooks:
            h.remove()
        return outs

    a, b = record(sparse_model), record(dense_model)
    return {n: float((a[n] != b[n]).float().mean()) for n in a if n in b}


def bench_e2e(steps, warmup, dev, with_dense=True, T=16, batch=32, live=False):
    """Spiking-ResNet50 forward (random init, BN folded, multi-step LIF
    tau=2 v_th=1 hard reset) through optimize(): images/s = batch / t.
    live=True first calibrates every neuron layer's threshold to
    E2E_LIVE_DENSITY spikes (Models.calibrate_lif_thresholds_) on a separate
    calibration batch, then times the network on another batch and reports
    the densities measured on that one; the dense baseline has the same
    thresholds.  The live run also times single layers on their live inputs
    (live_layer_study) and counts spike flips against the dense model
    (spike_flips, on two images)."""
    import copy

    import sparseflow_amd as sf
    from sparseflow_amd.Models import calibrate_lif_thresholds_, fold_bn_, fuse_conv_lif_, spiking_resnet50
    from sparseflow_amd.neuron import LIFNode, reset_net

    t0 = time.time()
    # The dense convs (stem, stride-2 downsamples, layer4) and the baseline
    # use MIOpen's default algorithm choice; an exhaustive search over every
    # layer shape at 512 frames takes minutes.
    torch.backends.cudnn.benchmark = False
    torch.manual_seed(0)
    model = fold_bn_(spiking_resnet50(T=T)).to(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    img = torch.randn(batch, 3, 224, 224, generator=g, device=dev)
    calib = None
    if live:
        # Calibrated on other images than the timed ones.
        gc = torch.Generator(device=dev).manual_seed(1)
        img_cal = torch.randn(batch, 3, 224, 224, generator=gc, device=dev)
        calib = calibrate_lif_thresholds_(model, img_cal, target_density=E2E_LIVE_DENSITY)
        del img_cal
        log(f"[bench] e2e live: thresholds calibrated to {E2E_LIVE_DENSITY} in {time.time() - t0:.1f} s")
    dense = copy.deepcopy(model) if with_dense else None
    sf.optimize(model, sample_input=img, verbose=False)
    n_sparse = sum(type(m).__name__ == "SparseConv2d" for m in model.modules())
    torch.cuda.synchronize()
    log(f"[bench] e2e: model built and optimized ({n_sparse} sparse convs) in {time.time() - t0:.1f} s")

    def run(m):
        reset_net(m)
        return m(img)

    densities = {}
    hooks = [mod.register_forward_hook(lambda _m, _i, o, n=name: densities.__setitem__(n, float(o.float().mean())))
             for name, mod in model.named_modules() if isinstance(mod, LIFNode)]
    with torch.no_grad():
        out = run(model)
    for h in hooks:
        h.remove()
    torch.cuda.synchronize()
    log(f"[bench] e2e: first forward done at {time.time() - t0:.1f} s")
    flips = None
    if live and dense is not None:
        flips = spike_flips(model, dense, img[:2])
        log(f"[bench] e2e live: spike flips vs dense at batch 2, max layer {max(flips.values()):.2e}")
    with torch.no_grad():
        ums = time_gpu(lambda: run(model), steps, warmup)
        log(f"[bench] e2e: unfused {ums:.2f} ms per forward ({time.time() - t0:.1f} s)")
        # Bottleneck 1x1 conv + LIF pairs as one fused launch each.
        n_fused = fuse_conv_lif_(model)
        fout = run(model)
        ms = time_gpu(lambda: run(model), steps, warmup)
        log(f"[bench] e2e: fused ({n_fused} conv-LIF pairs) {ms:.2f} ms per forward ({time.time() - t0:.1f} s)")
        res = {
            "workload": E2E_LIVE_WORKLOAD if live else E2E_WORKLOAD, "T": T, "batch": batch, "ms_per_forward": ms,
            "images_per_s": batch / (ms * 1e-3), "sparse_convs": n_sparse,
            "fused_conv_lif_pairs": n_fused, "unfused_ms_per_forward": ums,
            "max_abs_logit_diff_fused_vs_unfused": float((fout - out).abs().max()),
            "mean_spike_density": sum(densities.values()) / max(1, len(densities)),
            "spike_density_by_layer": {k: round(v, 5) for k, v in densities.items()},
        }
        if flips is not None:
            res["spike_flip_frac_vs_dense_batch2"] = {k: float(f"{v:.3g}") for k, v in flips.items()}
        if calib is not None:
            res["threshold_calibration"] = {
                "target_density": E2E_LIVE_DENSITY,
                "calibration_input": "a separate batch (seed 1); timed input seed 0",
                "method": "per neuron layer, in network order: bisection of v_threshold on the layer's input "
                          "currents over 2^20 sampled neurons (Models.calibrate_lif_thresholds_)",
                "v_threshold_min": round(min(v for v, _ in calib.values()), 4),
                "v_threshold_max": round(max(v for v, _ in calib.values()), 4),
            }
        if dense is not None:
            ref = run(dense)
            torch.cuda.synchronize()
            log(f"[bench] e2e: dense first forward done at {time.time() - t0:.1f} s")
            dms = time_gpu(lambda: run(dense), max(2, steps // 2), 1)
            res["dense_ms_per_forward"] = dms
            res["dense_images_per_s"] = batch / (dms * 1e-3)
            res["speedup_vs_dense"] = dms / ms
            res["max_abs_logit_diff_vs_dense"] = float((out - ref).abs().max())
            res["max_abs_logit_vs_dense"] = float(ref.abs().max())
            del dense
        if live:
            torch.cuda.empty_cache()
            res["live_layers"] = live_layer_study(model, img, dev, max(5, steps * 2), T)
    return res


def bench_attn(steps, warmup, dev, with_dense=True, T=4, N=64, tokens=196, dim=384, heads=12, p=0.1):
    """Spikformer-style block at BASELINE config 5: binary Q/K/V Bernoulli(p)
    [T*N, heads, tokens, dim/heads]; the q/k/v/proj projections as sparse
    Linear on spike tokens [T*N*tokens, dim]; Q @ K^T and attn @ V as sparse
    batched matmuls; the patch-embed stem conv3x3 3 -> dim on N(0,1) 32x32
    frames.  Each op is timed sparse and dense (hipBLASLt / rocBLAS / MIOpen
    through torch) on the same tensors."""
    from sparseflow_amd import _lib
    from sparseflow_amd.Kernels.attention import sparse_attn_v_forward, sparse_qk_forward, sparse_spike_attention_forward
    from sparseflow_amd.Kernels.linear import sparse_linear_forward, split_weight_bf16, tap_weight
    from sparseflow_amd.Ops.sparse_conv2d import SparseConv2d

    hd = dim // heads
    bt = T * N
    g = torch.Generator(device=dev).manual_seed(5)
    qkv = [(torch.rand(bt, heads, tokens, hd, generator=g, device=dev) < p).float() for _ in range(3)]
    x_tok = (torch.rand(bt * tokens, dim, generator=g, device=dev) < p).float()
    h_tok = (torch.rand(bt * tokens, 4 * dim, generator=g, device=dev) < p).float()
    lin = torch.nn.Linear(dim, dim).to(dev)
    fc1 = torch.nn.Linear(dim, 4 * dim).to(dev)
    fc2 = torch.nn.Linear(4 * dim, dim).to(dev)
    wt = tap_weight(lin.weight)
    splits = {id(m): split_weight_bf16(m.weight) for m in (lin, fc1, fc2)}
    ws = torch.empty(_lib.linear_workspace_size(bt * tokens, 4 * dim), dtype=torch.uint8, device=dev)

    def lin_case(m, x):
        # The library's own kernel choice ("auto": the row bitmap for the wide fc1).
        return (lambda: sparse_linear_forward(x, m.weight, m.bias, w_split=splits[id(m)], kernel="auto"),
                lambda: torch.nn.functional.linear(x, m.weight, m.bias),
                x.numel() * 4 + m.weight.numel() * 4 + x.shape[0] * m.out_features * 4)
    scale = hd ** -0.5
    ops = {}
    with torch.no_grad():
        attn = sparse_qk_forward(qkv[0], qkv[1], scale)[0]
        cases = {
            "linear_384x384": lin_case(lin, x_tok),
            "linear_384x384_walk": (
                lambda: sparse_linear_forward(x_tok, lin.weight, lin.bias, w_t=wt, workspace=ws, kernel="walk"),
                lambda: torch.nn.functional.linear(x_tok, lin.weight, lin.bias),
                x_tok.numel() * 4 + dim * dim * 4 + bt * tokens * dim * 4),
            "mlp_fc1_384x1536": lin_case(fc1, x_tok),
            "mlp_fc2_1536x384": lin_case(fc2, h_tok),
            "qk": (
                lambda: sparse_qk_forward(qkv[0], qkv[1], scale),
                lambda: torch.matmul(qkv[0], qkv[1].transpose(-2, -1)) * scale,
                2 * qkv[0].numel() * 4 + bt * heads * tokens * tokens * 4),
            "av": (
                lambda: sparse_attn_v_forward(attn, qkv[2]),
                lambda: torch.matmul(attn, qkv[2]),
                attn.numel() * 4 + 2 * qkv[2].numel() * 4),
            # q, k, v read once, y written once: the fused form of qk + av.
            "attention_fused": (
                lambda: sparse_spike_attention_forward(qkv[0], qkv[1], qkv[2], scale),
                lambda: torch.matmul(torch.matmul(qkv[0], qkv[1].transpose(-2, -1)) * scale, qkv[2]),
                4 * qkv[0].numel() * 4),
        }
        for name, (sp_fn, dn_fn, alg) in cases.items():
            ms = time_gpu(sp_fn, steps, warmup)
            kt = kernel_times(sp_fn, max(5, min(steps, 20)))
            dms = time_gpu(dn_fn, max(5, steps // 2), 3) if with_dense else None
            ops[name] = {"us": ms * 1e3, "dense_us": None if dms is None else dms * 1e3,
                         "speedup_vs_dense": None if dms is None else dms / ms,
                         "hbm_gbs": alg / (ms * 1e-3) / 1e9, "alg_bytes": alg,
                         "kernels_us": {k: v[1] * 1e3 for k, v in kt.items()}}
            log(f"[bench] attn {name}: {ms * 1e3:.1f} us (dense {'-' if dms is None else f'{dms * 1e3:.1f}'} us)")
        del attn
        torch.cuda.empty_cache()
        # Patch-embed stem: conv3x3 3 -> dim on dense N(0,1) frames.
        img = torch.randn(bt, 3, 32, 32, generator=g, device=dev)
        conv = make_conv(3, dim, 3, 1, dev)
        sp = SparseConv2d.from_dense(conv).to(dev)
        sp.set_inference_mode(True)
        ms = time_gpu(lambda: sp(img), steps, warmup)
        kt = kernel_times(lambda: sp(img), max(5, min(steps, 20)))
        torch.backends.cudnn.benchmark = True
        wd = conv.weight.float()
        dms = time_gpu(lambda: torch.nn.functional.conv2d(img, wd, None, 1, 1), max(5, steps // 2), 3) \
            if with_dense else None
        torch.backends.cudnn.benchmark = False
        stem_y = bt * dim * 32 * 32 * 4
        ops["stem_conv3x3_3to384"] = {"us": ms * 1e3, "dense_us": None if dms is None else dms * 1e3,
                                      "speedup_vs_dense": None if dms is None else dms / ms,
                                      "kernels_us": {k: v[1] * 1e3 for k, v in kt.items()},
                                      "alg_bytes": img.numel() * 4 + dim * 27 * 4 + stem_y,
                                      "hbm_gbs": (img.numel() * 4 + dim * 27 * 4 + stem_y) / (ms * 1e-3) / 1e9}
        log(f"[bench] attn stem_conv3x3_3to384: {ms * 1e3:.1f} us (dense {'-' if dms is None else f'{dms * 1e3:.1f}'}"
            f" us) kernels {ops['stem_conv3x3_3to384']['kernels_us']}")
    # One Spikformer block's matmul work: q, k, v, proj projections, the
    # attention core (fused; the dense reference runs qk then av) and the MLP.
    mlp = ops["mlp_fc1_384x1536"]["us"] + ops["mlp_fc2_1536x384"]["us"]
    blk = 4 * ops["linear_384x384"]["us"] + ops["attention_fused"]["us"] + mlp
    res = {"workload": ATTN_WORKLOAD, "T": T, "N": N, "tokens": tokens, "dim": dim, "heads": heads,
           "spike_p": p, "ops": ops, "block_matmul_us": blk}
    if with_dense:
        dblk = (4 * ops["linear_384x384"]["dense_us"] + ops["qk"]["dense_us"] + ops["av"]["dense_us"]
                + ops["mlp_fc1_384x1536"]["dense_us"] + ops["mlp_fc2_1536x384"]["dense_us"])
        res["block_matmul_dense_us"] = dblk
        res["block_matmul_speedup_vs_dense"] = dblk / blk
    return res


def measured_traffic(workload, kernel):
    """HBM bytes per launch (fetched + written) of `kernel` on `workload` as
    measured by the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    (profiles/traffic.json), or None when no profile of that kernel on that
    workload is committed."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(workload, {}).get(kernel)
    except (OSError, ValueError):
        return None
    if not rec:
        return None
    return int(rec["fetch_bytes"]) + int(rec["write_bytes"])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="resnet50_layer1_conv3x3", choices=sorted(WORKLOADS))
    ap.add_argument("--extra", default="all", help="'all', 'none' or comma-separated workload names (+ "
                                                   f"{LIF_WORKLOAD}, {ATTN_WORKLOAD}, {E2E_WORKLOAD}, "
                                                   f"{E2E_LIVE_WORKLOAD})")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-miopen", action="store_true", help="skip the MIOpen baselines")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a device-to-device copy of known size (for PMC byte calibration)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: every box in this setup has a single MI355X and the "
              "spike-sparse conv path needs no collective (frames shard independently). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda", 0)
    from sparseflow_amd import _lib

    _lib.lib()  # fail loudly if the native library is missing

    log(f"[bench] primary workload {args.workload}: steps={args.steps} warmup={args.warmup}")
    main_res = bench_conv(args.workload, args.steps, args.warmup, dev, with_miopen=not args.no_miopen)
    log(f"[bench] {json.dumps(main_res)}")

    if args.copy_calibration:
        n = 1 << 28  # 1 GiB of fp32
        a = torch.empty(n, device=dev)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: {n * 4} bytes read + {n * 4} bytes written per copy")
        del a, b

    extra = {}
    names = []
    if args.extra == "all":
        names = [n for n in WORKLOADS if n != args.workload] + [LIF_WORKLOAD, ATTN_WORKLOAD, E2E_WORKLOAD,
                                                                E2E_LIVE_WORKLOAD]
    elif args.extra != "none":
        names = [n.strip() for n in args.extra.split(",") if n.strip()]
    for name in names:
        torch.cuda.empty_cache()
        steps = max(5, args.steps // 2)
        if name == LIF_WORKLOAD:
            r = bench_lif(steps, 3, dev, with_miopen=not args.no_miopen)
        elif name == ATTN_WORKLOAD:
            r = bench_attn(steps, 3, dev, with_dense=not args.no_miopen)
        elif name in (E2E_WORKLOAD, E2E_LIVE_WORKLOAD):
            r = bench_e2e(max(3, steps // 5), 2, dev, with_dense=not args.no_miopen, live=name == E2E_LIVE_WORKLOAD)
        else:
            r = bench_conv(name, steps, 3, dev, with_miopen=not args.no_miopen)
        extra[name] = r
        log(f"[bench] {json.dumps(r)}")

    # Roofline of the dominant kernel (the one with the largest average launch
    # duration) from the library's per-launch HIP events.
    kus = main_res["kernels_us"]
    dom = max(kus, key=lambda k: kus[k])
    dom_bytes = main_res["kernel_bytes"][dom]
    achieved = dom_bytes / (kus[dom] * 1e-6) / 1e9 if kus[dom] > 0 else 0.0
    roofline = {
        "bound": "hbm",
        "kernel": dom,
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": measured_traffic(args.workload, dom),
        "avg_launch_us": round(kus[dom], 2),
        "alg_bytes_per_launch": dom_bytes,
    }
    cpu = None if args.no_cpu else cpu_baseline(args.workload)
    frames, c_in, h, w, c_out, k, s, gen, dens, images = WORKLOADS[args.workload]
    line = {
        "metric": METRIC,
        "value": round(main_res["us_per_layer"], 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_res["us_per_layer"] / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: i.i.d. Bernoulli spikes generated on device, random Kaiming-normal weights",
        "config": {
            "workload": args.workload,
            "frames": frames, "T": 16, "batch": images, "c_in": c_in, "h": h, "w": w, "c_out": c_out,
            "kernel": k, "stride": s, "spike_density": round(main_res["input_density"], 5),
        },
        "hbm_gbs": round(main_res["hbm_gbs"], 1),
        "hbm_frac": round(main_res["hbm_frac"], 4),
        "images_per_s": round(main_res["images_per_s"], 1),
        "miopen_us": None if main_res["miopen_us"] is None else round(main_res["miopen_us"], 2),
        "speedup_vs_miopen": None if main_res["speedup_vs_miopen"] is None else round(main_res["speedup_vs_miopen"], 2),
        "kernels_us": {k2: round(v, 2) for k2, v in kus.items()},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
