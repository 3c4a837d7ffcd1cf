"""Benchmark of the xsimgs hot path on one MI355X.

Headline: Mpix/s of the 1920x1080, 1M-Gaussian SH3 forward+backward frame (config cfg2): one
step is activations -> SH -> UT projection -> binning (count, scan, depth order, expand, tile
sort) -> tile offsets -> rays -> eval3d forward -> eval3d backward -> SH backward -> activation
gradients, with every input resident in HBM before timing starts.

Also reported: per-stage times (HIP events on the stream the kernels run on) with achieved
algorithmic HBM GB/s against the 8 TB/s peak, a `roofline` object for the dominant kernel, and
a `cpu_baseline` of the same frame run by the CPU oracle on this host's cores.

The same line carries `configs`: the other benchmark configurations measured the same way (cfg1
forward only; cfg3 the 2048x128 lidar range image; cfg4 the six-camera rig; cfg2_frustum the cfg2
scene with every Gaussian inside the field of view), each with ms per frame, Mpix/s, Gaussians/s,
per-stage times, the roofline of its dominant kernel and a CPU-oracle baseline on a bounded sample.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--configs cfg1,cfg3,...]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--config", default="cfg2")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--stage-reps", type=int, default=20)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--configs", default="cfg1,cfg3,cfg4,cfg2_frustum",
                   help="comma list of further configurations reported under `configs` ('' for none)")
    p.add_argument("--config-steps", type=int, default=5)
    p.add_argument("--profile-stages", default="", help="comma list of stages to run alone (for rocprof)")
    p.add_argument("--per-camera", action="store_true",
                   help="render camera rigs one camera per call (the reference caller's loop) instead of batched")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only run a plain 256 MiB device copy 5 times (scale of the rocprofv3 byte counters)")
    p.add_argument("--calibrate-valu", action="store_true",
                   help="only measure the VALU issue ceiling at 1-8 waves per SIMD and the shader clock")
    return p.parse_args()


# FP32 work the compositor kernels execute per (pixel, Gaussian) pair, counted from their arithmetic
# (fma two, add / mul / min / max / compare / exp / rcp one each; fixed tile origin): alpha evaluation
# 42 for every evaluated pair (M rd 15, |grd|^2 5, capped reciprocal 2, grd x gro 9, its squared norm
# 5, exponent scale 2, exp / opacity / clamp / threshold 4); forward composite 13 + 2 per colour
# channel for every composited pair (hit distance 6, depth 2, transmittance and tests 5); backward
# 72 + 4 per colour channel for every composited pair without ray gradients (hit distance and the
# 1 / (1 - alpha) transmittance 10, dL/dalpha 6, the collapsed alpha and hit vectors 21, mean
# gradient 7 (the lane's M^T product shared by its four pixels), the symmetric M gradient from the
# ray offset 24, opacity and buffer 4). Evaluated and composited counts come from the kernels
# themselves (pair_counts), so pairs skipped unevaluated by the culling are not counted.
FLOPS_EVAL = 42
FLOPS_FWD_CONTRIB = 13          # + 2 per colour channel
FLOPS_BWD_CONTRIB = 72          # + 4 per colour channel
# MI355X's published FP32 peak: 1024 SIMDs issue a wave64 FMA every 2 cycles at 2.4 GHz. The kernels
# are also priced against the FMA rate this GPU measurably sustains (valu_ceiling), which runs below it
# because the clock drops under a full VALU load.
FP32_VALU_PEAK_TFLOPS = 157.3
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "eval3d_bwd_cfg2_traffic.json")


def calibrate_copy(torch):
    n = 64 << 20                                   # 64 Mi floats = 256 MiB each way
    x = torch.ones(n, device="cuda:0")
    y = torch.empty_like(x)
    for _ in range(5):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read": 4 * n, "bytes_written": 4 * n, "launches": 5}))


def valu_ceiling(torch, waves_per_simd, iters=8192):
    """The VALU issue ceiling measured on this GPU: `xsg_bench_valu_ceiling` puts `waves_per_simd`
    wavefronts on every SIMD, each issuing 16 * iters independent FP32 FMAs (no packed FP32). Returns
    the wave64 VALU instructions issued per microsecond per SIMD, the FMA rate in TFLOP/s and the
    shader clock the launch ran at (s_memtime against the 100 MHz real-time counter)."""
    from xsimgs_amd import _C
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks = cus * waves_per_simd
    out = torch.empty(blocks * 256, device="cuda:0")
    stamps = torch.zeros(4 * blocks, dtype=torch.int64, device="cuda:0")
    _C.bench_valu_ceiling(blocks, iters, out, stamps)
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    _C.bench_valu_ceiling(blocks, iters, out, stamps)
    e.record()
    e.synchronize()
    ms = s.elapsed_time(e)
    st = stamps.view(-1, 4).cpu().double()
    mhz = float(((st[:, 1] - st[:, 0]) / (st[:, 3] - st[:, 2])).mean()) * 100.0
    insts = blocks * 4 * iters * 16                      # wave64 VALU instructions of the launch
    return {"waves_per_simd": waves_per_simd, "ms": round(ms, 4),
            "inst_per_us_per_simd": round(insts / (4 * cus) / (ms * 1e3), 1),
            "fma_tflops": round(insts * 64 * 2 / (ms * 1e-3) / 1e12, 1), "clock_mhz": round(mhz)}


def calibrate_valu(torch):
    rows = [valu_ceiling(torch, w) for w in range(1, 9)]
    print(json.dumps({"calibration": "valu", "rows": rows}))


def event_time_ms(fn, reps, torch):
    """Average ms per call of fn, bracketed by events on the current stream (the kernels' stream)."""
    fn()
    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / reps


def extension_rows(torch, _C, frame, synthetic, st, sc, cam_spec, means, scales, quats, opac, W, H, reps, dev):
    """Timing of the rows that widen the frame: camera-pose gradients of the frame's rays, rays and UT
    projection through the distorted perspective and fisheye models, and the packed instance mask and
    rigid per-instance copy (fwd, bwd) over the frame's Gaussians."""
    N = means.shape[0]
    rows = {}

    def row(name, fn, nbytes):
        with torch.no_grad():
            t = event_time_ms(fn, reps, torch)
        gbs = nbytes / (t * 1e-3) / 1e9
        rows[name] = {"ms": round(t, 4), "alg_bytes": int(nbytes), "GB/s": round(gbs, 1),
                      "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}

    g = torch.Generator(device=dev).manual_seed(5)
    # camera-pose gradients: backward of the frame's rays into the pack (24 B of ray gradients per pixel)
    cam = st.cams[0]
    pack = cam.pack.detach().clone().requires_grad_(True)
    with torch.enable_grad():
        ro, rd = cam.ext_cls.camera_rays(pack, W, H)
    gro = torch.randn(H, W, 3, device=dev, generator=g)
    grd = torch.randn(H, W, 3, device=dev, generator=g)

    def rays_bwd():
        torch.autograd.grad((ro, rd), pack, (gro, grd), retain_graph=True)
    with torch.enable_grad():
        row("camera_rays_bwd", rays_bwd, 24 * W * H)
    # distorted models on the frame's Gaussians and pixels
    for kind, impl, dist in (("distorted", [0.66, 1.17, 0.5, 0.5], [-0.28, 0.07, 1e-3, -5e-4, 0.01, 0.02, -0.004,
                                                                    0.001]),
                             ("fisheye", [0.3, 0.53, 0.5, 0.5], [0.03, -0.005, 0.001, -0.0001])):
        spec = synthetic.CameraSpec(kind, W, H, q=cam_spec.q, t=cam_spec.t, impl=impl, dist=dist,
                                    max_radius=1.5 if kind == "distorted" else None)
        c = frame.make_camera(spec, dev)
        row(f"ut_projection_{kind}", lambda c=c: c.ut_gs_projection(means, scales, quats, W, H, opacity=opac),
            65 * N)
        row(f"rays_{kind}", lambda c=c: c.camera_rays(W, H), 24 * W * H)
    # upstream producers: instances of 500 Gaussians, stored instance by instance
    k = max(1, N // 500)
    ids = (torch.arange(N, device=dev, dtype=torch.int32) * k // N).contiguous()
    imask = torch.rand(k, device=dev, generator=g) < 0.9
    row("packed_mask_from_instances", lambda: _C.packed_mask_from_instances(ids, imask), 4 * N + N // 8)
    rot = torch.nn.functional.normalize(torch.randn(N, 4, device=dev, generator=g), dim=1)
    iq = torch.nn.functional.normalize(torch.randn(k, 4, device=dev, generator=g), dim=1)
    it, iv, iw = (torch.randn(k, 3, device=dev, generator=g) for _ in range(3))
    outs = [torch.zeros(N, 3, device=dev), torch.zeros(N, 4, device=dev), torch.zeros(N, 3, device=dev),
            torch.zeros(N, dtype=torch.bool, device=dev)]
    pos = means.contiguous()
    row("rigid_transform_fwd", lambda: _C.copy_gs_rigid_transform_fwd(pos, rot, ids, iq, it, iv, iw, imask, *outs, 0),
        (12 + 16 + 4) * N + (12 + 16 + 12 + 1) * N)
    vp, vr, vv = (torch.randn_like(o, ) for o in outs[:3])
    row("rigid_transform_bwd", lambda: _C.copy_gs_rigid_transform_bwd(pos, rot, ids, iq, iw, imask, 0, None, None,
                                                                      vp, vr, vv),
        (12 + 16 + 4 + 12 + 16 + 12) * N + (12 + 16) * N)
    return rows


def binning_alg_bytes(kind, n, n_isects, n_tiles, n_flag2=0, keys=False):
    """Bytes the binning cannot avoid: read each Gaussian's projection once (means2d 8, radii 8, depth 4,
    + flag 1 for the lidar / spherical kinds), write tiles_per_gauss (4) once, write each intersection's
    id (4; and its key, 8 more, when the keys are asked for -- the frame's binning takes the tile offsets
    instead) once, write each tile's offset (4) once; a seam Gaussian's re-projection reads its point,
    scale, quaternion and opacity (44). The depth pre-order, run expansion and scans the implementation
    adds are not priced, so the fraction is that of the unavoidable traffic."""
    per_g = 24 + (1 if kind != "pinhole" else 0)
    return per_g * n + (12 if keys else 4) * n_isects + 4 * n_tiles + 44 * n_flag2


def sh_bwd_alg_bytes(K, n, v_colors):
    """The SH backward's unavoidable bytes: every Gaussian's position and colour gradient read (24),
    its position gradient (12) and coefficient gradients (12 K) written; the coefficients (12 K) read
    only for a Gaussian whose colour gradient is not zero (for the others every output is zero)."""
    n_need = int((v_colors != 0).any(dim=-1).sum())
    return (36 + 12 * K) * n + 12 * K * n_need


def bench_config(name, args, steps, warmup, reps, torch, np, cpu=True, extensions=False):
    import xsimgs_amd  # noqa: F401  (fails loudly without the native libraries)
    from xsimgs_amd import _C, frame, synthetic
    from xsimgs_amd.rendering import rasterize as rz
    from xsimgs_amd.rendering import rasterize_dynamic as rzd  # noqa: F401

    dev = torch.device("cuda:0")
    sc = synthetic.make(name, seed=args.seed)
    cam_spec = sc.cameras[0]
    W, H = cam_spec.width, cam_spec.height
    st = frame.prepare(sc, dev)
    n_cams = len(sc.cameras)
    backward = sc.backward
    grads = None
    if backward:
        grads = [tuple(g.to(dev) for g in (sc.grad_rgb[i], sc.grad_depth[i], sc.grad_alpha[i]))
                 for i in range(n_cams)]
    # a rig of regular-tiling cameras renders batched: one binning and one compositor launch per pass
    # over every camera (one SH evaluation when they share the origin)
    rig = frame.rig_batchable(st) and not args.per_camera
    rig_grads = tuple(torch.stack([g[k] for g in grads]) for k in range(3)) if (rig and backward) else None

    def step():
        frame.zero_grads(st)
        if rig:
            if backward:
                frame.render_rig(st, backward=True, grads=rig_grads)
            else:
                with torch.no_grad():
                    frame.render_rig(st)
            return
        for ci in range(n_cams):
            if backward:
                frame.render_frame(st, backward=True, grads=grads[ci], cam_index=ci)
            else:
                with torch.no_grad():
                    frame.render_frame(st, backward=False, cam_index=ci)

    # the compositor calls are bracketed by HIP events on the stream they run on (torch's current
    # stream), inside the timed steps
    live = {"eval3d_fwd": [], "eval3d_bwd": []}
    sym = ({"eval3d_fwd": "rasterize_eval3d_fwd_batched", "eval3d_bwd": "rasterize_eval3d_bwd_batched"} if rig else
           {"eval3d_fwd": "rasterize_eval3d_fwd", "eval3d_bwd": "rasterize_eval3d_bwd"})
    orig = {k: getattr(rz, v) for k, v in sym.items()}

    def timed(kname):
        fn = orig[kname]

        def call(*a, **k):
            ev0 = torch.cuda.Event(enable_timing=True)
            ev1 = torch.cuda.Event(enable_timing=True)
            ev0.record()
            out = fn(*a, **k)
            ev1.record()
            live[kname].append((ev0, ev1))
            return out
        return call

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    for k, v in sym.items():
        setattr(rz, v, timed(k))
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for k, v in sym.items():
        setattr(rz, v, orig[k])
    ms = (t1 - t0) * 1e3 / steps
    live_ms = {k: sum(a.elapsed_time(b) for a, b in v) / len(v) for k, v in live.items() if v}
    mpix = W * H * n_cams / (ms * 1e-3) / 1e6

    # ---------------------------------------------------------------- per-stage timing (per camera)
    N = sc.n
    K = sc.sh_coeffs.shape[1] if sc.sh_coeffs is not None else 0
    tsx, tsy = sc.tile_size
    ntx, nty = (W + tsx - 1) // tsx, (H + tsy - 1) // tsy
    kind = cam_spec.kind
    stage_rows, info = {}, []
    with torch.no_grad():
        means, quats = st.means.detach(), st.quats.detach()
        scales = torch.exp(st.log_scales.detach())
        opac = torch.sigmoid(st.opacity_logits.detach())
        sh = st.sh.detach() if st.sh is not None else None
        for ci in range(n_cams):   # the compositor's loaded work of every camera (its algorithmic bytes)
            cam = st.cams[ci]
            origin = cam.pose.t
            colors = (_C.spherical_harmonics_fused_fwd(sc.sh_degree, origin, means, sh, None, False)
                      if sh is not None else st.colors.detach())
            cdim = colors.shape[-1]
            flags, radii, m2, dep = cam.ut_gs_projection(means, scales, quats, W, H, opacity=opac,
                                                         use_phm=sc.use_phm)
            tpg, ids, fl = cam.isect_gs_tiles(means, scales, quats, W, H, flags, radii, m2, dep, opacity=opac,
                                              tile_size_x=tsx, tile_size_y=tsy)
            off = _C.isect_offset_encode(ids, ntx, nty)
            ro, rd = cam.camera_rays(W, H)
            pairs = torch.zeros(2, dtype=torch.int64, device=dev)
            # the per-tile work estimates the forward writes for the backward, as the autograd functions pass them
            tw = torch.empty(off.numel(), dtype=torch.int32, device=dev)
            rgb, depth, alpha, last = _C.rasterize_eval3d_fwd(means, quats, scales, colors.unsqueeze(0),
                                                              opac.view(1, -1), W, H, tsx, tsy, ro, rd, off, fl,
                                                              pair_counts=pairs, tile_work=tw)
            c = dict(cam=cam, origin=origin, colors=colors, cdim=cdim, proj=(flags, radii, m2, dep), ids=ids, fl=fl,
                     off=off, tw=tw, ro=ro, rd=rd, alpha=alpha, last=last, n_isects=int(fl.numel()),
                     visible=int((tpg > 0).sum()), n_flag2=int((flags == 2).sum()))
            c["fwd_evaluated"], c["contributing"] = (int(x) for x in pairs.cpu())
            n_isects = c["n_isects"]
            starts = off.view(-1).long()
            ends = torch.cat([starts[1:], torch.tensor([n_isects], device=dev)])
            lt = torch.nn.functional.pad(last, (0, ntx * tsx - W, 0, nty * tsy - H)).view(nty, tsy, ntx, tsx)
            tile_max = lt.amax(dim=(1, 3)).reshape(-1).long()
            rng = (ends - starts).clamp(min=0)
            # loaded intersections: the forward up to the batch holding the tile's last contribution and
            # its terminating element, the backward from the tile's largest last id down to the start
            c["bwd_loaded"] = int((tile_max - starts + 1).clamp(min=0).minimum(rng).sum())
            bs = tsx * tsy
            fwd_batches = ((tile_max - starts + 2).clamp(min=1) + bs - 1) // bs
            c["fwd_loaded"] = int(torch.minimum(rng, fwd_batches * bs).sum())
            if backward:
                g_rgb, g_d, g_a = grads[ci]
                bpairs = torch.zeros(2, dtype=torch.int64, device=dev)
                bo = _C.rasterize_eval3d_bwd(means, scales, quats, opac, colors, ro, rd, tsx, tsy, off, fl, alpha,
                                             last, g_rgb, g_d, g_a, False, pair_counts=bpairs, tile_work=tw)
                c["v_colors"] = bo[4]
                c["bwd_evaluated"], c["bwd_composited"] = (int(x) for x in bpairs.cpu())
            info.append(c)
        c0 = info[0]
        cam, origin, colors, cdim = c0["cam"], c0["origin"], c0["colors"], c0["cdim"]
        flags, radii, m2, dep = c0["proj"]
        ids, fl, off, tw, ro, rd, alpha, last = (c0[k] for k in ("ids", "fl", "off", "tw", "ro", "rd", "alpha", "last"))
        n_isects = c0["n_isects"]
        enc_reads = 8 * int(math.ceil(math.log2(n_isects + 1))) if n_isects else 0
        stages = {
            "sh_fwd": (lambda: _C.spherical_harmonics_fused_fwd(sc.sh_degree, origin, means, sh, None, False),
                       (24 + 12 * K) * N) if sh is not None else None,
            "ut_projection": (lambda: cam.ut_gs_projection(means, scales, quats, W, H, opacity=opac,
                                                            use_phm=sc.use_phm), 65 * N),
            "binning": (lambda: cam.isect_gs_tiles(means, scales, quats, W, H, flags, radii, m2, dep, opacity=opac,
                                                   tile_size_x=tsx, tile_size_y=tsy,
                                                   tile_offsets=torch.empty(nty, ntx, dtype=torch.int32,
                                                                            device=dev), keys=False),
                        binning_alg_bytes(kind, N, n_isects, ntx * nty, c0["n_flag2"])),
            "offset_encode": (lambda: _C.isect_offset_encode(ids, ntx, nty), (enc_reads + 4) * ntx * nty),
            "rays": (lambda: cam.camera_rays(W, H), 24 * W * H),
            "eval3d_fwd": (lambda: _C.rasterize_eval3d_fwd(means, quats, scales, colors.unsqueeze(0),
                                                           opac.view(1, -1), W, H, tsx, tsy, ro, rd, off, fl,
                                                           tile_work=tw),
                           (24 + 4 * cdim + 12) * W * H + (48 + 4 * cdim) * c0["fwd_loaded"]),
        }
        if backward:
            g_rgb, g_d, g_a = grads[0]
            stages["eval3d_bwd"] = (lambda: _C.rasterize_eval3d_bwd(means, scales, quats, opac, colors, ro, rd, tsx,
                                                                    tsy, off, fl, alpha, last, g_rgb, g_d, g_a,
                                                                    False, tile_work=tw),
                                    (24 + 8 + 4 * cdim + 8) * W * H + (48 + 4 * cdim) * c0["bwd_loaded"] +
                                    (11 + cdim) * 4 * N)
            if sh is not None:
                v_colors = c0["v_colors"]
                stages["sh_bwd"] = (lambda: _C.spherical_harmonics_fused_bwd(sc.sh_degree, origin, means, sh, None,
                                                                             False, v_colors, None,
                                                                             origin_grad=False),
                                    sh_bwd_alg_bytes(K, N, v_colors))
        per_frame = {"sh_fwd", "sh_bwd"}   # one call per frame: the scenes with SH have one camera or a rig
        if rig:
            # the batched stages over every camera of the rig; their bytes are the cameras' sum
            tot = lambda k: sum(c[k] for c in info)
            stk = lambda k: torch.stack([c[k] for c in info])
            radii_b, m2_b, dep_b = (torch.stack([c["proj"][j] for c in info]) for j in (1, 2, 3))
            ro_b, rd_b = stk("ro"), stk("rd")
            off_b = torch.empty((n_cams, nty, ntx), dtype=torch.int32, device=dev)
            _, _, fl_b = _C.isect_regular_tiles_batched(m2_b, radii_b, dep_b, W, H, tsx, tsy, tile_offsets=off_b)
            col_b = colors if frame.rig_shares_origin(st) else stk("colors")
            tw_b = torch.empty(off_b.numel(), dtype=torch.int32, device=dev)
            _, _, alpha_b, last_b = _C.rasterize_eval3d_fwd_batched(means, quats, scales, col_b, opac, W, H, tsx, tsy,
                                                                    ro_b, rd_b, off_b, fl_b, tile_work=tw_b)
            n_col = 1 if col_b.dim() == 2 else n_cams
            if len({type(c["cam"]) for c in info}) == 1:
                # the rig's cameras of one kind project in one launch, each Gaussian read once: its inputs
                # (44 B) once, every camera's outputs (21 B)
                packs_b = torch.cat([c["cam"].pack for c in info])
                cam0 = info[0]["cam"]
                stages["ut_projection"] = (
                    lambda: cam0.ext_cls.projection_utgs_rig(packs_b, means, None, scales, quats, opac, W, H),
                    44 * N + 21 * N * n_cams)
                per_frame |= {"ut_projection"}
            stages["binning"] = (
                lambda: _C.isect_regular_tiles_batched(m2_b, radii_b, dep_b, W, H, tsx, tsy,
                                                       tile_offsets=torch.empty_like(off_b), keys=False),
                sum(binning_alg_bytes(kind, N, c["n_isects"], ntx * nty, c["n_flag2"]) for c in info))
            stages["eval3d_fwd"] = (
                lambda: _C.rasterize_eval3d_fwd_batched(means, quats, scales, col_b, opac, W, H, tsx, tsy, ro_b,
                                                        rd_b, off_b, fl_b, tile_work=tw_b),
                n_cams * (24 + 4 * cdim + 12) * W * H + (48 + 4 * cdim) * tot("fwd_loaded"))
            per_frame |= {"binning", "eval3d_fwd", "eval3d_bwd"}
            if backward:
                gb = rig_grads
                stages["eval3d_bwd"] = (
                    lambda: _C.rasterize_eval3d_bwd_batched(means, scales, quats, opac, col_b, ro_b, rd_b, tsx, tsy,
                                                            off_b, fl_b, alpha_b, last_b, gb[0], gb[1], gb[2],
                                                            ray_grads=False, tile_work=tw_b),
                    n_cams * (24 + 8 + 4 * cdim + 8) * W * H + (48 + 4 * cdim) * tot("bwd_loaded") +
                    (11 + n_col * cdim) * 4 * N)
                if sh is not None and n_col == 1:
                    v_col_b = _C.rasterize_eval3d_bwd_batched(means, scales, quats, opac, col_b, ro_b, rd_b, tsx, tsy,
                                                              off_b, fl_b, alpha_b, last_b, gb[0], gb[1], gb[2],
                                                              ray_grads=False, tile_work=tw_b)[4]
                    stages["sh_bwd"] = (lambda: _C.spherical_harmonics_fused_bwd(sc.sh_degree, origin, means, sh,
                                                                                 None, False, v_col_b, None,
                                                                                 origin_grad=False),
                                        sh_bwd_alg_bytes(K, N, v_col_b))
        stages = {k: v for k, v in stages.items() if v is not None}
        timed_stages = stages
        if args.profile_stages:
            keep = set(args.profile_stages.split(","))
            timed_stages = {k: v for k, v in stages.items() if k in keep}
        for sname, (fn, nbytes) in timed_stages.items():
            t = event_time_ms(fn, reps, torch)
            gbs = nbytes / (t * 1e-3) / 1e9
            stage_rows[sname] = {"ms": round(t, 4), "alg_bytes": int(nbytes), "GB/s": round(gbs, 1),
                                 "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                                 "per": "frame" if (sname in per_frame or n_cams == 1) else "camera"}
    ext_rows = {}
    if extensions and not args.profile_stages and kind == "pinhole":
        ext_rows = extension_rows(torch, _C, frame, synthetic, st, sc, cam_spec, means, scales, quats, opac, W, H,
                                  reps, dev)

    # ---------------------------------------------------------------- roofline of the dominant kernel
    # algorithmic bytes and flops per launch: one camera's (averaged over the cameras) when each camera
    # is one launch, every camera's sum when the rig is one batched launch
    cdim = info[0]["cdim"]
    avg = lambda k: sum(c[k] for c in info) / len(info)
    per_launch = (lambda k: sum(c[k] for c in info)) if rig else avg
    npix = (n_cams if rig else 1) * W * H
    n_col = 1 if (not rig or frame.rig_shares_origin(st) or sh is None) else n_cams
    alg = {"eval3d_fwd": (24 + 4 * cdim + 12) * npix + (48 + 4 * cdim) * per_launch("fwd_loaded")}
    flops = {"eval3d_fwd": FLOPS_EVAL * per_launch("fwd_evaluated") +
             (FLOPS_FWD_CONTRIB + 2 * cdim) * per_launch("contributing")}
    if backward:
        alg["eval3d_bwd"] = ((24 + 8 + 4 * cdim + 8) * npix + (48 + 4 * cdim) * per_launch("bwd_loaded") +
                             (11 + n_col * cdim) * 4 * N)
        flops["eval3d_bwd"] = (FLOPS_EVAL * per_launch("bwd_evaluated") +
                               (FLOPS_BWD_CONTRIB + 4 * cdim) * per_launch("bwd_composited"))
    dom = max(live_ms, key=live_ms.get)
    t_dom = live_ms[dom]
    gbs = alg[dom] / (t_dom * 1e-3) / 1e9
    tfl = flops[dom] / (t_dom * 1e-3) / 1e12
    roofline = {"kernel": dom, "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                "launch_ms": round(t_dom, 4), "alg_bytes_per_launch": int(alg[dom]),
                "valu": {"achieved": round(tfl, 2), "peak": FP32_VALU_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tfl / FP32_VALU_PEAK_TFLOPS, 4), "flops_per_launch": int(flops[dom]),
                         "measured_fma_ceiling": args.valu_ceiling["fma_tflops"],
                         "frac_of_measured": round(tfl / args.valu_ceiling["fma_tflops"], 4)},
                "note": ("the compositor has no dense contraction (no MFMA) and is VALU / LDS / atomic bound: "
                         "the HBM fraction of its algorithmic bytes is reported as defined, beside it the FP32 "
                         "work it executes against the published FP32 peak and against the FMA rate measured "
                         "on this GPU (8 waves per SIMD)")}
    if os.path.exists(TRAFFIC_FILE) and name == "cfg2" and dom == "eval3d_bwd":
        with open(TRAFFIC_FILE) as fh:
            tr = json.load(fh)
        roofline["traffic"] = int(tr["fetch_kib_per_dispatch"] * 1024 * tr["fetch_scale"] +
                                  tr["write_kib_per_dispatch"] * 1024 * tr["write_scale"])
        roofline["traffic_source"] = os.path.relpath(TRAFFIC_FILE, ROOT)
    pair_stats = {k: int(avg(k)) for k in ("fwd_evaluated", "contributing") + (
        ("bwd_evaluated", "bwd_composited") if backward else ())}

    # ---------------------------------------------------------------- CPU baseline (oracle, one camera's frame)
    cpu_row = None
    if cpu:
        cpu_row = cpu_baseline(sc, cam_spec, backward, np)
    return {
        "workload": f"{name}: {W}x{H} x{n_cams} cams, {N} Gaussians, "
                    f"{('SH' + str(sc.sh_degree)) if sc.sh_coeffs is not None else 'CDIM ' + str(cdim)}, "
                    f"{'fwd+bwd' if backward else 'fwd'}",
        "n_gaussians": N, "width": W, "height": H, "n_cams": n_cams, "tile": [tsx, tsy],
        "n_isects": int(avg("n_isects")), "visible_gaussians": int(avg("visible")),
        "ms_per_frame": round(ms, 4), "Mpix/s": round(mpix, 2),
        "Gaussians/s": round(N * n_cams / (ms * 1e-3), 1),
        "rig": ("batched: one binning and one compositor launch per pass over all cameras, one SH evaluation "
                "for the shared origin") if rig else None,
        "stages": stage_rows, "extensions": ext_rows,
        "live_ms": {k: round(v, 4) for k, v in live_ms.items()}, "pairs_per_camera": pair_stats,
        "roofline": roofline, "cpu_baseline": cpu_row, "notes": sc.notes,
    }


def cpu_baseline(sc, cam_spec, backward, np):
    """The CPU oracle on one camera's frame (activations and SH colours, UT, binning, tile offsets, rays,
    composite forward and, for the backward configurations, composite backward and SH backward), timed
    on this host. Threads: the host's CPUs up to 16 -- a one-GPU box's share of its CPUs."""
    from oracle import oracle as O
    host_cpus = os.cpu_count() or 1
    O.set_num_threads(min(host_cpus, 16))
    threads = O.num_threads()
    W, H = cam_spec.width, cam_spec.height
    tsx, tsy = sc.tile_size
    ntx, nty = (W + tsx - 1) // tsx, (H + tsy - 1) // tsy
    m, q, s, o = sc.means.numpy(), sc.quats.numpy(), sc.scales.numpy(), sc.opacity.numpy()
    tc0 = time.perf_counter()
    if sc.sh_coeffs is not None:
        col = O.sh_fwd(sc.sh_degree, np.asarray(cam_spec.t, np.float32), m, sc.sh_coeffs.numpy())
    else:
        col = sc.colors.numpy()
    f_, r_, m_, d_ = O.project_utgs(cam_spec, m, s, q, o, W, H, phm=sc.use_phm)
    if cam_spec.kind == "pinhole":
        _, ids_c, fl_c = O.isect_regular(m_, r_, d_, W, H, tsx, tsy)
    else:
        elev = cam_spec.beam_v.numpy()[::tsy] if cam_spec.kind == "lidar" else None
        _, ids_c, fl_c = O.isect_spherical_family(cam_spec.kind, cam_spec, m, s, q, o, f_, m_, r_, d_, tsx, tsy, W, H,
                                                  elev=elev)
    off_c = O.offset_encode(ids_c, ntx, nty)
    ro_c, rd_c = O.camera_rays(cam_spec, W, H)
    rgb_c, dep_c, alp_c, last_c = O.eval3d_fwd(m, q, s, col, o, ro_c, rd_c, off_c, fl_c, tsx, tsy)
    if backward:
        gc = O.eval3d_bwd(m, q, s, col, o, ro_c, rd_c, off_c, fl_c, alp_c, last_c, sc.grad_rgb[0].numpy(),
                          sc.grad_depth[0].numpy(), sc.grad_alpha[0].numpy(), tsx, tsy)
        if sc.sh_coeffs is not None:
            O.sh_bwd(sc.sh_degree, np.asarray(cam_spec.t, np.float32), m, sc.sh_coeffs.numpy(), gc["v_colors"])
    cpu_s = time.perf_counter() - tc0
    return {"value": round(W * H / cpu_s / 1e6, 4), "unit": "Mpix/s", "cores": threads, "host_cpus": host_cpus,
            "kind": "port",
            "sample": f"camera 0's frame of {sc.name} ({W}x{H}, {sc.n} Gaussians, {'fwd+bwd' if backward else 'fwd'}) "
                      f"on {threads} OpenMP threads of {host_cpus} host CPUs (a one-GPU box's share is 16): "
                      f"{cpu_s:.2f} s"}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: this build runs on one GPU only (asked for {args.gpus}); the path would shard "
              "by camera / tile rows with one gradient all-reduce, which is not built here.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    if args.calibrate_copy:
        calibrate_copy(torch)
        return
    if args.calibrate_valu:
        calibrate_valu(torch)
        return
    args.valu_ceiling = valu_ceiling(torch, 8)
    head = bench_config(args.config, args, args.steps, args.warmup, args.stage_reps, torch, np,
                        cpu=not args.no_cpu_baseline, extensions=True)
    configs = {}
    for name in [c for c in args.configs.split(",") if c and c != args.config] if not args.profile_stages else []:
        torch.cuda.empty_cache()
        configs[name] = bench_config(name, args, args.config_steps, 2, max(3, args.stage_reps // 4), torch, np,
                                     cpu=not args.no_cpu_baseline)
    out = {
        "metric": "Mpix/s fwd+bwd @1920x1080, 1M Gaussians SH3; achieved HBM GB/s per kernel",
        "value": head["Mpix/s"],
        "unit": "Mpix/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_frame"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded, BASELINE.json config definitions)",
        "config": {"workload": head["workload"], "n_gaussians": head["n_gaussians"], "width": head["width"],
                   "height": head["height"], "n_cams": head["n_cams"], "tile": head["tile"],
                   "n_isects": head["n_isects"], "visible_gaussians": head["visible_gaussians"],
                   "parallelism": "single GPU"},
        "Gaussians/s": head["Gaussians/s"],
        "stages": head["stages"],
        "extensions": head["extensions"],
        "live_ms": head["live_ms"],
        "pairs": head["pairs_per_camera"],
        "roofline": head["roofline"],
        "valu_ceiling": args.valu_ceiling,
        "cpu_baseline": head["cpu_baseline"],
        "configs": configs,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
