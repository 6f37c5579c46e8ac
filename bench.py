#!/usr/bin/env python3
"""Forward+backward benchmark of the MI355X gs3d rasterizer.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workloads all|headline]

Headline workload: 3,000,000 Gaussians, SH degree 3, four 1920x1080 cameras
on a radius-5 ring around 64 Gaussian clusters (synthetic data drawn from a
fixed seed; see dsl_splat_amd.synthetic).  A step is one gs3d.rasterize call
over all four cameras plus the backward pass of loss = sum(image * W) with W
~ N(0,1) over every rendered channel; inputs are resident in HBM before the
timed region.

The other benchmark workloads (10k Gaussians at 256x256 RGB; 500k at 720p
SH3 with absgrad; 1M at 1600x1200 with 32 feature channels and a camera-z
channel; 2M at 1080p SH3 with 5% large Gaussians, pose gradients and
absgrad) are timed the same way and reported under "workloads".

Prints one JSON line: the headline ms/iter (lower is better), forward and
backward ms, stage spans measured with HIP events inside the timed steps,
their algorithmic bytes and fraction of HBM peak, the (pixel, Gaussian) pair
counts of the blend stages, the HBM roofline of the projection kernel, and a
CPU baseline (the C++ oracle on the host cores over a bounded sample).
"""

import argparse
import json
import math
import os
import statistics
import sys
import time

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, 8 TB/s
ROOFLINE_KERNEL = "gs3d::project_fwd_kernel<true> (EWA projection + metadata of every view, one launch)"
# rocprofv3 FETCH_SIZE / WRITE_SIZE summary of that kernel on the headline workload.
TRAFFIC_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "project_fwd_kernel_traffic_3M_1080p_4view.md")
HEADLINE = "sh3_1080p_4view"
# Benchmark workloads in order (synthetic.make_scene names).
WORKLOADS = ("small", "sh3_720p", "sh3_1080p_4view", "feat32", "pose_fanout")
HBM_STAGES = ("project", "order", "bin", "project_bwd")
WARM_MS = 300.0  # warm-up of the other workloads, in milliseconds of steps
FANOUT = "pose_fanout"  # 2M Gaussians, 5% of them large: the workload the tile modes are for


def measured_traffic(workload, n):
    """HBM bytes per launch of the projection kernel, measured with rocprofv3
    counters (committed summary; headline workload only), or None."""
    if workload != HEADLINE or n is not None or not os.path.exists(TRAFFIC_SUMMARY):
        return None
    with open(TRAFFIC_SUMMARY) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    return None


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", default=HEADLINE, help="headline workload")
    p.add_argument("--workloads", choices=("all", "headline"), default="all",
                   help="also time the other benchmark workloads")
    p.add_argument("--workload-steps", type=int, default=5, help="timed steps of each other workload")
    p.add_argument("--n", type=int, default=None, help="override the headline Gaussian count")
    p.add_argument("--cpu-baseline", choices=("on", "off"), default="on")
    p.add_argument("--tile-mode", choices=("radius", "snugbox", "accutile"), default="radius",
                   help="tile_mode of the headline steps (the other modes are timed for comparison)")
    p.add_argument("--mode-steps", type=int, default=5,
                   help="timed steps per other tile mode on the headline workload (0 skips them)")
    p.add_argument("--copy-calibration-mib", type=int, default=0,
                   help="also run a device copy of this many MiB (counter calibration under rocprofv3)")
    return p.parse_args()


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def make_inputs(workload, n, device):
    import torch
    from dsl_splat_amd import synthetic

    scene = synthetic.make_scene(workload, n=n)
    scene.to(device)
    leaves = dict(
        means=scene.means.clone().requires_grad_(True),
        quats=scene.quats.clone().requires_grad_(True),
        scales=scene.scales.clone().requires_grad_(True),
        opacities=scene.opacities.clone().requires_grad_(True),
    )
    colors = (scene.sh_coeffs if scene.sh_coeffs is not None else scene.features).clone().requires_grad_(True)
    extra = None if scene.extra_features is None else scene.extra_features[0].clone().requires_grad_(True)
    viewmats = scene.viewmats.clone().requires_grad_(scene.pose_grad)
    torch.cuda.synchronize()
    return scene, leaves, colors, extra, viewmats


def step_fn(scene, leaves, colors, extra, viewmats, tile_mode="radius"):
    import torch
    from dsl_splat_amd import gs3d

    sh = scene.sh_coeffs is not None
    # loss = sum(image * W) over every rendered channel, taken as one dot
    # product per output plane against contiguous slices of W prepared here,
    # outside the timed step.
    W = scene.loss_weights
    D = 3 if sh else colors.shape[-1]
    w_features = W[..., :D].contiguous().reshape(-1)
    w_extra = W[..., D:-1].contiguous().reshape(-1) if extra is not None else None
    w_alpha = W[..., -1:].contiguous().reshape(-1)

    def forward():
        res = gs3d.rasterize(leaves["means"], leaves["quats"], leaves["scales"], leaves["opacities"], viewmats,
                             scene.Ks, scene.width, scene.height, features=None if sh else colors,
                             sh_coeffs=colors if sh else None, sh_degree=scene.sh_degree,
                             extra_features=extra, absgrad=scene.absgrad, tile_mode=tile_mode)
        forward.meta = res.meta
        loss = torch.dot(res.features.reshape(-1), w_features) + torch.dot(res.alpha.reshape(-1), w_alpha)
        if res.extra_features is not None:
            loss = loss + torch.dot(res.extra_features.reshape(-1), w_extra)
        return loss

    def backward(loss):
        loss.backward()
        for t in list(leaves.values()) + [colors, extra, viewmats]:
            if t is not None:
                t.grad = None

    return forward, backward


def time_steps(forward, backward, steps, warmup, stage_events=False):
    """ms per step between two synchronisations, then, over a second pass of
    as many steps, forward and backward HIP event spans and with stage_events
    the median span of every stage recorded inside the steps.  Steps follow
    each other as in a training loop, without a synchronisation between them
    (each forward synchronises once, on its pair totals), so the host
    prepares step i+1 while step i's backward runs."""
    import torch
    from dsl_splat_amd import profiling

    for _ in range(warmup):
        backward(forward())
    torch.cuda.synchronize()
    events = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(3)) for _ in range(steps)]
    recorder = profiling.StageEvents() if stage_events else None
    # ms: the steps alone between two synchronisations.  Recording events
    # costs host time, which a small frame's host-bound step would pay, so
    # the forward/backward and stage spans come from a second pass.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        backward(forward())
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1000.0 / steps
    t0 = time.perf_counter()
    if recorder is not None:
        recorder.__enter__()
    for e0, e1, e2 in events:
        e0.record()
        loss = forward()
        e1.record()
        backward(loss)
        e2.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    if recorder is not None:
        recorder.__exit__(None, None, None)
    out = dict(ms=ms, evented_ms=(t1 - t0) * 1000.0 / steps,
               fwd_ms=sum(a.elapsed_time(b) for a, b, _ in events) / steps,
               bwd_ms=sum(b.elapsed_time(c) for _, b, c in events) / steps)
    if recorder is not None:
        out["stages"] = {k: statistics.median(v) for k, v in recorder.spans().items() if v}
    return out


def frame_info(scene):
    """Projection and binning of the workload's frame (the calls the
    rasterizer makes) for the byte accounting, and the blend's pair counts
    from the counting forward pass (outside any timed region)."""
    import torch
    from dsl_splat_amd.gs3d import lists as tile_lists, projection as gproj, render as grender
    from dsl_splat_amd.splatting import binning, cameras

    deg, sh = scene.sh_degree, scene.sh_coeffs
    views, n = scene.viewmats.shape[0], len(scene.means)
    with torch.no_grad():
        full, inverse, centers, errors = cameras.launch_prepare(scene.viewmats, scene.Ks, scene.width, scene.height,
                                                                deg is not None and deg > 0)
        st = gproj.project_views(scene.means, scene.quats, scene.scales, scene.opacities, scene.viewmats, full,
                                 scene.Ks, scene.width, scene.height, 0.2, math.inf, 0.0, sh=sh, sh_degree=deg or 0,
                                 camera_centers=centers if deg else None, metadata=True, normalize_quats=True)
        key_bits = torch.zeros(1, dtype=torch.int32, device=st.radii.device)
        order, offsets, totals = binning.order_rows(st.centers, st.radii, st.depths, scene.width, scene.height,
                                                    key_bits_out=key_bits)
        group_pairs, count = totals.cpu().tolist()
        ranges, ids = binning.bin_rows(st.centers, st.radii, order, offsets, group_pairs, count, scene.width,
                                       scene.height)
        feats = st.colors if sh is not None else scene.features
        pairs = grender.pair_counts(ranges, ids, st.centers, st.conics, feats, scene.width, scene.height,
                                    extra=scene.extra_features)
        tiles = binning.tile_count(scene.width, scene.height, views)
        capped = {}
        if tile_lists.applies(count, tiles):
            # The steady-state frames of the timed steps write lists capped
            # by the same cameras' stops: the ids they keep, and the group
            # items their write pass reads.
            stops = torch.empty((views, tiles // views), dtype=torch.int32, device=st.radii.device)
            grender.render_views(ranges, ids, st.centers, st.conics, feats, scene.width, scene.height,
                                 extra=scene.extra_features, lists=tile_lists.CappedLists([], (), 0, None, stops))
            launch = binning.prepare_bin_rows(st.centers, st.radii, order, offsets, scene.width, scene.height)
            binning.launch_bin_rows(launch, group_pairs, count, caps=stops.view(-1))
            capped = dict(items_loaded=binning.capped_items_loaded(launch),
                          ids_written=int(tile_lists.capped_lengths(stops, ranges[:, 1] - ranges[:, 0]).sum()))
            del launch
        torch.cuda.synchronize()
    groups = views * (((scene.width + 15) // 16 + 7) // 8) * (((scene.height + 15) // 16 + 7) // 8)
    info = dict(pairs=count, group_pairs=group_pairs, groups=groups, tiles=tiles,
                group_passes=1 if groups <= 1024 else math.ceil(int(groups - 1).bit_length() / 8),
                rows=views * n, visible=int((st.radii > 0).sum()), blend_pairs=pairs,
                # radix passes of the depth order in the timed steps (they sort
                # the key bits the frame's kept rows need)
                order_passes=binning.order_pass_count(max(9, int(key_bits.item()))), capped=capped)
    return info, dict(full=full, st=st, ranges=ranges, ids=ids, feats=feats)


def stage_bytes(scene, info):
    """Algorithmic bytes of every HBM-bound stage: what its kernels must read
    and write once each."""
    M, S, T, R, V = info["pairs"], info["group_pairs"], info["tiles"], info["rows"], info["visible"]
    cap = info["capped"]
    sh = scene.sh_coeffs
    views, n = scene.viewmats.shape[0], len(scene.means)
    K = 0 if sh is None else sh.shape[-2]
    sh_in = 0 if sh is None else (n if sh.ndim == 3 else views * n) * K * 3 * 4
    return {
        # params 44 B/G (+ SH once for all views) in; per view centers 8, conics+opacity 16, radii 4,
        # tiles 4, depth 4, means2d 8, meta opacity 4, meta conic 12 (+ colour 12) out
        "project": n * 44 + sh_in + views * n * (60 + (12 if sh is not None else 0)),
        # keys and records (depth 4 + centre 8 + radius 4 in, key 4 + record 8 out); the first radix
        # pass reads every row's key for its histogram (4) and (key, record) (12) and writes the V
        # rows that touch a tile (12); the later passes (two or three, by the key bits the kept rows
        # need) over those V rows (key 4 for the histogram, (key, record) 12 in and 12 out); group
        # counts at the sorted positions (4) and filler records + zero counts after them
        # ((R - V) x 12); inclusive scan of the counts (4 in, 4 out)
        "order": R * (28 + 4 + 12 + 8) + V * (12 + (info["order_passes"] - 1) * 28 + 4) + (R - V) * 12,
        # items: records and offsets in (12 B/row), items out (8 B/item); group sort (keys read for the
        # histogram 8 + read and written 16 per pass; one 10-bit pass up to 1024 groups, whose digit
        # scan gives the group ranges, else 8-bit passes and a range search, 8 B/item); the count pass
        # reads the items (8 B); the write pass reads the items of the chunks it needs (8 B; all of
        # them for whole lists) and writes the ids it keeps (4 B/pair; all pairs for whole lists);
        # tile totals/starts/ranges (16 B/tile), and the caps (4 B/tile) for capped lists
        "bin": R * 12 + S * (8 + 24 * info["group_passes"] + (8 if info["group_passes"] == 1 else 16))
               + cap.get("items_loaded", S) * 8 + cap.get("ids_written", M) * 4 + T * (20 if cap else 16),
        # params 44 + SH 4K*3 in, per view radii 4 + centre/conic grads 24 (+ colour grads 12) in;
        # grads 44 + SH out
        "project_bwd": n * 88 + 2 * sh_in + views * n * (28 + (12 if sh is not None else 0)),
    }


def stage_report(stages, by, info):
    out = {}
    for k, ms in stages.items():
        entry = dict(ms=round(ms, 4))
        if k in by:
            gbps = by[k] / (ms * 1e-3) / 1e9
            entry.update(bytes=by[k], gbps=round(gbps, 1), frac=round(gbps / HBM_PEAK_GBPS, 4))
        if k == "order":
            entry["radix_passes"] = info["order_passes"]
        if k in ("render_fwd", "render_bwd"):
            p = info["blend_pairs"]
            entry.update(visited_pairs_per_us=round(p["visited"] / (ms * 1e3), 1),
                         accepted_pairs_per_us=round(p["accepted"] / (ms * 1e3), 1))
        out[k] = entry
    return out


def kernel_timings(scene, frame):
    """The roofline kernel alone, and the forward blend with and without
    contribution statistics, with HIP events on the launch stream."""
    import torch
    from dsl_splat_amd.gs3d import projection as gproj, render as grender
    from dsl_splat_amd.statistics import PreparedStatistics

    views, n = scene.viewmats.shape[0], len(scene.means)
    full, st, ranges, ids, feats = (frame[k] for k in ("full", "st", "ranges", "ids", "feats"))
    out = {}
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.no_grad():
        # Back-to-back launches that rotate over three copies of the
        # parameters (3 x 132 MB) and three sets of outputs (3 x 720 MB):
        # every launch reads its inputs from HBM (the two launches in between
        # wrote 1.4 GB, far more than the L2 and the Infinity Cache hold) and
        # pays for writing back the dirty lines the previous launch left, as
        # inside a training step.  Only the last launch's lines still in the
        # caches at the end event go unpaid: about 1/20 of one launch's output
        # at most.  Without coefficients the call launches the projection
        # kernel only.
        launches, copies = 20, 3
        params = [tuple(t.clone() for t in (scene.means, scene.quats, scene.scales, scene.opacities))
                  for _ in range(copies)]
        project = lambda p: gproj.project_views(*p, scene.viewmats, full, scene.Ks, scene.width, scene.height, 0.2,
                                                math.inf, 0.0, metadata=True, normalize_quats=True)
        keep = [project(p) for p in params]
        # A 2 GiB read ahead of the first launch keeps the device busy while
        # the host enqueues the first launches, so no idle time falls
        # between the events.
        flush = torch.ones(512 << 20, dtype=torch.float32, device=scene.means.device)
        torch.cuda.synchronize()
        flush.amax()
        e0.record()
        for i in range(launches):
            # project_views allocates its outputs; the caching allocator
            # hands back the blocks freed copies launches earlier, so the
            # output sets rotate as the parameter copies do.
            keep[i % copies] = None
            keep[i % copies] = project(params[i % copies])
        e1.record()
        torch.cuda.synchronize()
        out["project_kernel"] = e0.elapsed_time(e1) / launches
        del params, keep
        # A plain 2 GiB device copy on the same GPU: the bandwidth a
        # streaming kernel reaches here, beside the 8 TB/s peak.
        dst = torch.empty_like(flush)
        dst.copy_(flush)
        e0.record()
        for _ in range(10):
            dst.copy_(flush)
        e1.record()
        torch.cuda.synchronize()
        out["copy_gbps"] = 2 * flush.numel() * 4 / (e0.elapsed_time(e1) / 10 * 1e-3) / 1e9
        del flush, dst
        # Contribution statistics (a masked count and a weighted sum over
        # per-view pixel maps) observed by the forward blend, against the
        # plain forward blend, both back-to-back.
        g = torch.Generator().manual_seed(9)
        hw = scene.width * scene.height
        pv = torch.stack([(torch.rand((views, hw), generator=g) < 0.5).float(), torch.rand((views, hw), generator=g)],
                         1).to(scene.means.device)
        stats = PreparedStatistics((0, 1), pv, torch.zeros((views, 1, n), dtype=torch.int32, device=pv.device),
                                   torch.zeros((views, 1, n), device=pv.device))
        for key, kw in (("render_fwd_kernel", {}), ("render_fwd_stats_kernel", {"statistics": stats})):
            blend = lambda: grender.render_views(ranges, ids, st.centers, st.conics, feats, scene.width,
                                                 scene.height, extra=scene.extra_features, **kw)
            blend()
            e0.record()
            for _ in range(5):
                blend()
            e1.record()
            torch.cuda.synchronize()
            out[key] = e0.elapsed_time(e1) / 5
    return out


def sort_pairs_timing(scene, frame, reps=5):
    """The reference's own binning sequence on one camera's real tile pairs:
    gs3d_sort_pairs_u64 (stable LSD radix sort of the (tile << 32 | depth
    bits) keys with their Gaussian ids over bits [0, 32 + bit_length(T))) +
    gs3d_tile_ranges, the entry points a caller of the reference's
    primitives/tiling.py:67-100 binds.  The keys come from gs3d_emit_keys on
    the first camera's projected rows; each repetition restores the unsorted
    keys and zeroes the ranges outside the timed region."""
    import torch
    from dsl_splat_amd.primitives import tiling
    from dsl_splat_amd.splatting import binning

    st = frame["st"]
    W, H = scene.width, scene.height
    T = binning.tile_count(W, H, 1)
    with torch.no_grad():
        offsets, count = tiling.scan_counts(st.tile_counts[0])
        keys, ids = binning.emit_keys(st.centers[0], st.radii[0], st.depths[0], offsets, count, W, H)
        keys0, ids0 = keys[:count].clone(), ids[:count].clone()
        ranges = torch.zeros((T, 2), dtype=torch.int32, device=keys.device)
        end_bit = 32 + int(T).bit_length()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ms = []
        for i in range(reps + 1):
            keys[:count].copy_(keys0)
            ids[:count].copy_(ids0)
            ranges.zero_()
            e0.record()
            tiling.sort_pairs(keys, ids, count, end_bit)
            tiling.identify_ranges(keys[:count], ranges)
            e1.record()
            torch.cuda.synchronize()
            if i:
                ms.append(e0.elapsed_time(e1))
        passes = (end_bit + 7) // 8
        nbytes = (24 * passes + 8) * count + 8 * T
        t = statistics.median(ms)
        gbps = nbytes / (t * 1e-3) / 1e9
        del keys, ids, keys0, ids0
    return dict(pairs=count, end_bit=end_bit, passes=passes, tiles=T, ms=round(t, 4), bytes=nbytes,
                gbps=round(gbps, 1), frac=round(gbps / HBM_PEAK_GBPS, 4),
                note="gs3d_sort_pairs_u64 + gs3d_tile_ranges on camera 1's keys from gs3d_emit_keys (the "
                     "reference's sort_tile_pairs); bytes (24 P + 8) M + 8 T, median of "
                     f"{reps} repetitions")


def cpu_baseline(scene, workload):
    """The C++ oracle (fwd+bwd, OpenMP on the host cores): the workload's
    first camera at full N and resolution, scaled by the camera count for
    several cameras (they are independent in the algorithm); for the two
    small workloads one warm-up and the median of 3 iterations."""
    import numpy as np  # noqa: F401
    import torch

    import oracle

    oracle.build()
    cores = len(os.sched_getaffinity(0))
    oracle.set_threads(cores)
    npy = lambda t: t.detach().cpu().numpy()
    V, K = npy(scene.viewmats[:1]), npy(scene.Ks[:1])
    W, H = scene.width, scene.height
    sh, deg = scene.sh_coeffs, scene.sh_degree
    means, quats, scales, opac = npy(scene.means), npy(scene.quats), npy(scene.scales), npy(scene.opacities)
    shn = None if sh is None else npy(sh)
    feats = None if scene.features is None else npy(scene.features)
    extra = None if scene.extra_features is None else npy(scene.extra_features[0])
    up = npy(scene.loss_weights[:1])

    def once():
        t0 = time.perf_counter()
        full, inverse, centers, err = oracle.camera_prepare(V, K, W, H, bool(deg))
        proj = oracle.project_fwd(means, quats, scales, opac, V, full, K, W, H, sh=shn, sh_degree=deg or 0,
                                  camera_centers=centers if deg else None, metadata=True, normalize_quats=True)
        offsets, total = oracle.scan_i32(proj["tiles"].ravel())
        keys, vals = oracle.emit_keys(proj["centers"], proj["radii"], proj["depths"], offsets, total, W, H)
        T = ((W + 15) // 16) * ((H + 15) // 16)
        sk, sv = oracle.sort_pairs(keys, vals, 32 + int(T).bit_length())
        del keys, vals
        ranges = oracle.tile_ranges(sk, T)
        del sk
        blended = proj["colors"] if shn is not None else feats
        image, final_t, contrib = oracle.render_fwd(W, H, ranges, sv, proj["centers"], proj["conics"], blended,
                                                    extra=extra)
        t1 = time.perf_counter()
        g = oracle.render_bwd(W, H, ranges, sv, proj["centers"], proj["conics"], blended, final_t, contrib, up,
                              extra=extra, absgrad=scene.absgrad)
        oracle.project_bwd(means, quats, scales, opac, V, full, K, W, H, proj["radii"], g["centers"], g["conics"],
                           sh=shn, sh_degree=deg or 0, camera_centers=centers if deg else None,
                           grad_colors=g["features"] if shn is not None else None, normalize_quats=True)
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1

    small = workload in ("small", "sh3_720p")
    if small:
        once()
        runs = sorted((once() for _ in range(3)), key=lambda r: r[0] + r[1])
        fwd, bwd = runs[1]
        how = "median of 3 iterations after one warm-up"
    else:
        fwd, bwd = once()
        how = "one iteration"
    views = scene.viewmats.shape[0]
    scope = f"camera 1 of {views} (full N, {W}x{H}), scaled x{views}" if views > 1 else f"full frame {W}x{H}"
    return dict(value=round((fwd + bwd) * 1000.0 * views, 1), unit="ms", cores=cores, kind="port",
                sample=f"C++ oracle fwd+bwd, {scope}; {how}; {(fwd + bwd):.2f} s measured",
                fwd_ms=round(fwd * 1000.0 * views, 1), bwd_ms=round(bwd * 1000.0 * views, 1))


def describe(scene, workload):
    views = scene.viewmats.shape[0]
    colour = f"SH degree {scene.sh_degree}" if scene.sh_coeffs is not None else \
        f"{scene.features.shape[-1]} feature channels" + (" + camera-z channel" if scene.extra_features is not None
                                                         else "")
    extras = [s for s, on in (("absgrad", scene.absgrad), ("pose gradients", scene.pose_grad)) if on]
    return (f"{workload}: N={len(scene.means)}, {views} camera{'s' if views > 1 else ''}, "
            f"{scene.width}x{scene.height}, {colour}" + (", " + ", ".join(extras) if extras else "") +
            ", fwd+bwd of sum(image*W)")


def run_workload(workload, n, device, steps, warmup, cpu, tile_mode="radius", min_timed_ms=0.0):
    """Timed steps (clean, then with stage events) and the workload's
    accounting; returns (entry, scene, frame, inputs).  With min_timed_ms
    the step count grows (to at most 100) until the timed steps take about
    that long: short steps are otherwise dominated by host jitter."""
    import torch

    log(f"[bench] {workload}: building inputs")
    inputs = make_inputs(workload, n, device)
    scene = inputs[0]
    forward, backward = step_fn(*inputs, tile_mode)
    if min_timed_ms > 0:
        probe = time_steps(forward, backward, 2, warmup)
        steps = max(steps, min(100, math.ceil(min_timed_ms / max(probe["ms"], 1e-3))))
        # Short steps reach their steady rate only after a few hundred
        # milliseconds of back-to-back steps (clocks ramp up): warm up for
        # about that long, as a training loop would have.
        warmup = max(1, min(400, math.ceil(WARM_MS / max(probe["ms"], 1e-3))))
    log(f"[bench] {workload}: {warmup} warm-up + {steps} timed steps")
    clean = time_steps(forward, backward, steps, warmup)
    staged = time_steps(forward, backward, steps, 1, stage_events=True)
    info, frame = frame_info(scene)
    if info["capped"]:
        # The same steps writing whole lists: what a camera's first frame
        # costs, and the step without capped lists.
        from dsl_splat_amd.gs3d import lists as tile_lists

        enabled, tile_lists.ENABLED = tile_lists.ENABLED, False
        try:
            info["capped"]["ms_whole_lists"] = round(time_steps(forward, backward, steps, 1)["ms"], 3)
        finally:
            tile_lists.ENABLED = enabled
    by = stage_bytes(scene, info)
    stages = stage_report(staged["stages"], by, info)
    hbm = [k for k in ("project", "order", "bin") if k in stages]
    t13 = sum(stages[k]["ms"] for k in hbm)
    b13 = sum(by[k] for k in hbm)
    entry = dict(
        config=describe(scene, workload),
        steps=steps,
        ms=round(clean["ms"], 3), fwd_ms=round(clean["fwd_ms"], 3), bwd_ms=round(clean["bwd_ms"], 3),
        staged_ms=round(staged["evented_ms"], 3),
        stages=stages,
        stages_1_3={"ms": round(t13, 4), "bytes": b13, "gbps": round(b13 / (t13 * 1e-3) / 1e9, 1),
                    "frac": round(b13 / (t13 * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                    "note": "project + order + bin spans inside the steps (bin starts at the end of the depth "
                            "order and includes the host's read of the pair totals, reported alone as "
                            "totals_read)"},
        pairs=dict(tile_pairs=info["pairs"], group_items=info["group_pairs"], visible_rows=info["visible"],
                   rows=info["rows"], **info["blend_pairs"]),
        capped_lists=info["capped"] or None,
    )
    torch.cuda.synchronize()
    if cpu:
        log(f"[bench] {workload}: CPU baseline (oracle)")
        entry["cpu_baseline"] = cpu_baseline(scene, workload)
    return entry, scene, frame, inputs, forward


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "multi-GPU sharding of this path is a design note, not a built feature", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    cpu = args.cpu_baseline == "on"
    head, scene, frame, inputs, forward = run_workload(args.workload, args.n, device, args.steps, args.warmup, cpu,
                                                       args.tile_mode)
    modes = {args.tile_mode: dict(ms=head["ms"], pairs=int(forward.meta["tiles_per_gauss"].sum()))}
    for mode in ("radius", "snugbox", "accutile"):
        if mode == args.tile_mode or args.mode_steps <= 0:
            continue
        log(f"[bench] tile_mode={mode}: {args.mode_steps} steps")
        f_m, b_m = step_fn(*inputs, mode)
        t = time_steps(f_m, b_m, args.mode_steps, 1)
        modes[mode] = dict(ms=round(t["ms"], 3), pairs=int(f_m.meta["tiles_per_gauss"].sum()))
    log("[bench] kernel timings")
    kt = kernel_timings(scene, frame)
    log("[bench] reference-convention pair sort")
    sort_pairs = sort_pairs_timing(scene, frame)
    if args.copy_calibration_mib > 0:
        src = torch.ones(args.copy_calibration_mib << 18, device=device)
        dst = torch.empty_like(src)
        torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: {src.numel() * 4} bytes read and written")
        del src, dst
    del frame, inputs
    torch.cuda.empty_cache()
    others = {}
    if args.workloads == "all":
        for wl in WORKLOADS:
            if wl == args.workload:
                continue
            entry, _, _, wl_inputs, wl_forward = run_workload(wl, None, device, args.workload_steps, 2, cpu,
                                                               min_timed_ms=50.0)
            if wl == FANOUT and args.mode_steps > 0:
                # The tile modes cut the pair count most where Gaussians fan
                # out over many tiles.
                modes_wl = {"radius": dict(ms=entry["ms"], pairs=int(wl_forward.meta["tiles_per_gauss"].sum()))}
                for mode in ("snugbox", "accutile"):
                    log(f"[bench] {wl} tile_mode={mode}: {entry['steps']} steps")
                    f_m, b_m = step_fn(*wl_inputs, mode)
                    t = time_steps(f_m, b_m, entry["steps"], 1, stage_events=True)
                    modes_wl[mode] = dict(ms=round(t["ms"], 3), pairs=int(f_m.meta["tiles_per_gauss"].sum()),
                                          stages={k: round(v, 4) for k, v in t["stages"].items()})
                entry["tile_modes"] = modes_wl
            del wl_inputs, wl_forward
            others[wl] = entry
            torch.cuda.empty_cache()
    # The roofline object is the projection forward kernel: HBM-bound, one
    # launch per step, params 44 B/G in and 60 B per view out (the colour
    # kernel's bytes are in the "project" stage); every other stage's
    # bandwidth is in "stages".
    n_g, n_v = len(scene.means), scene.viewmats.shape[0]
    kernel_bytes = n_g * 44 + n_v * n_g * 60
    kernel_ms = kt["project_kernel"]
    achieved = kernel_bytes / (kernel_ms * 1e-3) / 1e9
    result = {
        "metric": "3DGS fwd+bwd ms/iter @3M Gaussians 1080p SH3; sort/proj HBM GB/s",
        "value": head["ms"],
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms"],
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded)",
        "config": {
            "workload": head["config"],
            "gaussians": n_g, "cameras": n_v, "width": scene.width, "height": scene.height,
            "sh_degree": scene.sh_degree, "tile_mode": args.tile_mode,
        },
        "fwd_ms": head["fwd_ms"],
        "bwd_ms": head["bwd_ms"],
        "roofline": {
            "bound": "hbm",
            "kernel": ROOFLINE_KERNEL,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(args.workload, args.n),
            "ms": round(kernel_ms, 4),
            "bytes": kernel_bytes,
            "note": "parameters read once for all views (44 B/G) and 60 B per (view, Gaussian) written; the "
                    "colour kernel's bytes are in stages.project. Time base: HIP events around 20 back-to-back "
                    "launches rotating over 3 parameter copies and 3 output sets (inputs from HBM, each launch "
                    "pays the previous one's write-back), averaged",
            "copy_gbps": round(kt["copy_gbps"], 1),
            "copy_note": "a 2 GiB device-to-device copy (read + write) timed on the same GPU, for context",
        },
        "stages": head["stages"],
        "stages_1_3": head["stages_1_3"],
        "staged_ms": head["staged_ms"],
        "pairs": head["pairs"],
        "capped_lists": head["capped_lists"],
        "tile_modes": modes,
        "sort_pairs": sort_pairs,
        "statistics": {"requests": "masked count + weighted sum, per-view maps",
                       "render_fwd_ms": round(kt["render_fwd_kernel"], 4),
                       "render_fwd_stats_ms": round(kt["render_fwd_stats_kernel"], 4)},
        "cpu_baseline": head.get("cpu_baseline"),
        "workloads": others,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
