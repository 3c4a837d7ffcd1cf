"""ctypes front-end of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Loads ``xsg_oracle_f32.so`` / ``xsg_oracle_f64.so`` (built from ``xsg_oracle.c`` by
the Makefile beside this file) and wraps each restated reference kernel with a
numpy-in / numpy-out function. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg import this module; the product never does.
Every function below names the reference kernel it restates; the C source cites
the reference file:line of each step.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIBS = {}

KIND = {"pinhole": 0, "spherical": 1, "lidar": 2, "distorted": 3, "fisheye": 4}
MODE = {"central": 0, "negative": 1, "positive": 2}


def build(force: bool = False) -> None:
    """Compile both precisions with the Makefile beside this file."""
    targets = [os.path.join(HERE, f"xsg_oracle_{p}.so") for p in ("f32", "f64")]
    if force or not all(os.path.exists(t) for t in targets):
        subprocess.run(["make", "-s", "-C", HERE] + (["-B"] if force else []), check=True)


def _lib(prec: str = "f32"):
    if prec not in _LIBS:
        path = os.path.join(HERE, f"xsg_oracle_{prec}.so")
        if not os.path.exists(path):
            build()
        _LIBS[prec] = C.CDLL(path)
    return _LIBS[prec]


def _real(prec):
    return (C.c_float, np.float32) if prec == "f32" else (C.c_double, np.float64)


def _camera_struct(prec):
    ct, _ = _real(prec)

    class Cam(C.Structure):
        _fields_ = [("kind", C.c_int), ("q", ct * 4), ("t", ct * 3), ("v", ct * 3), ("w", ct * 3),
                    ("rolling", ct * 2), ("trigger_time", ct), ("pose_time", ct), ("impl", ct * 4),
                    ("beam_v", C.POINTER(ct)), ("n_beams", C.c_int), ("dist", ct * 8), ("max_radius_sq", ct)]
    return Cam


_CAM_TYPES = {}


def camera(spec, prec: str = "f32"):
    """Build the C camera struct from a ``xsimgs_amd.synthetic.CameraSpec``.

    The returned object keeps the beam array alive for the lidar camera.
    """
    if prec not in _CAM_TYPES:
        _CAM_TYPES[prec] = _camera_struct(prec)
    ct, nt = _real(prec)
    cam = _CAM_TYPES[prec]()
    cam.kind = KIND[spec.kind]
    for name, n in (("q", 4), ("t", 3), ("v", 3), ("w", 3), ("rolling", 2), ("impl", 4)):
        vals = getattr(spec, name)
        arr = getattr(cam, name)
        for i in range(n):
            arr[i] = float(vals[i])
    cam.trigger_time = float(spec.trigger_time)
    cam.pose_time = float(spec.pose_time)
    if spec.kind in ("distorted", "fisheye"):
        for i, x in enumerate(spec.dist):
            cam.dist[i] = float(x)
        cam.max_radius_sq = float(spec.max_radius) ** 2 if spec.max_radius is not None else 0.0
    cam._beam = None
    if spec.kind == "lidar":
        beam = np.ascontiguousarray(np.asarray(spec.beam_v, dtype=nt))
        cam._beam = beam
        cam.beam_v = beam.ctypes.data_as(C.POINTER(ct))
        cam.n_beams = beam.shape[0]
    return cam


def _p(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _arr(a, dtype):
    if a is None:
        return None
    if hasattr(a, "detach"):
        a = a.detach().cpu().numpy()
    return np.ascontiguousarray(np.asarray(a, dtype=dtype))


def ut_weights(alpha=0.1, beta=2.0, kappa=0.0, prec="f32"):
    """ut_weights (include/cameras/ut_kernels.h:17-36)."""
    ct, nt = _real(prec)
    out = np.zeros(4, nt)
    _lib(prec).orc_ut_weights(ct(alpha), ct(beta), ct(kappa), _p(out))
    return out


def project_utgs(spec, means, scales, quats, opacity, width, height, vel=None, ut=(0.1, 2.0, 0.0),
                 thr=1e-4, max_res=0.002, margin=1.0, phm=False, prec="f32", margins=False):
    """<Camera>.projection_utgs[_phm] (ut_kernels.h:187-305, ut_phm_kernels.h:13-173).

    Returns ``flags u8[N], radii[N,2], means2d[N,2], depths[N]`` (+ with ``margins`` a diagnostic
    per Gaussian: the smallest ratio of a validity decision's distance to its threshold over a bound
    on the float32 error of the compared value; below 1, float32 rounding can decide the flag either
    way. Meaningful in the f64 build).
    """
    ct, nt = _real(prec)
    lib = _lib(prec)
    cam = camera(spec, prec)
    means, scales, quats = _arr(means, nt), _arr(scales, nt), _arr(quats, nt)
    opacity, vel = _arr(opacity, nt), _arr(vel, nt)
    n = means.shape[0]
    w = ut_weights(*ut, prec=prec)
    flags = np.zeros(n, np.uint8)
    radii = np.zeros((n, 2), nt)
    m2 = np.zeros((n, 2), nt)
    dep = np.zeros(n, nt)
    mg = np.zeros(n, nt) if margins else None
    fn = lib.orc_project_utgs_phm if phm else lib.orc_project_utgs
    fn(C.byref(cam), C.c_int(n), _p(means), _p(vel), _p(scales), _p(quats), _p(opacity),
       ct(width), ct(height), _p(w), ct(thr), ct(max_res), ct(margin),
       _p(flags), _p(radii), _p(m2), _p(dep), _p(mg))
    if margins:
        return flags, radii, m2, dep, mg
    return flags, radii, m2, dep


def projection(spec, points, vel=None, thr=1e-4, max_res=0.002, margin=1.0, mode="central", no_jac=False,
               prec="f32"):
    """<Camera>.projection[_nojac] (projection_kernels.h:259-309): ``uvdt[N,4], mask[N]``."""
    ct, nt = _real(prec)
    cam = camera(spec, prec)
    points, vel = _arr(points, nt), _arr(vel, nt)
    n = points.shape[0]
    uvdt = np.zeros((n, 4), nt)
    mask = np.zeros(n, np.uint8)
    _lib(prec).orc_projection(C.byref(cam), C.c_int(n), _p(points), _p(vel), ct(thr), ct(max_res),
                              ct(margin), C.c_int(MODE[mode]), C.c_int(int(no_jac)), _p(uvdt), _p(mask))
    return uvdt, mask.astype(bool)


def camera_rays(spec, width, height, world_space=True, normalized=True, return_valid=False, prec="f32"):
    """<Camera>.camera_rays forward (ray_kernels.h:7-59): ``ray_o, ray_d`` as [H, W, 3] (and the
    per-pixel ``ray_valid`` mask with ``return_valid``)."""
    _, nt = _real(prec)
    cam = camera(spec, prec)
    ro = np.zeros((height, width, 3), nt)
    rd = np.zeros((height, width, 3), nt)
    valid = np.zeros((height, width), np.uint8)
    _lib(prec).orc_camera_rays(C.byref(cam), C.c_int(width), C.c_int(height), C.c_int(int(world_space)),
                               C.c_int(int(normalized)), _p(ro), _p(rd), _p(valid))
    return (ro, rd, valid.astype(bool)) if return_valid else (ro, rd)


def undistort_map(spec, width, height, normalized_range=False, prec="f32"):
    """<Camera>.undistort_map (distortion.h:33-56) of the distorted and fisheye models: [H, W, 2]."""
    _, nt = _real(prec)
    cam = camera(spec, prec)
    out = np.zeros((height, width, 2), nt)
    _lib(prec).orc_undistort_map(C.byref(cam), C.c_int(width), C.c_int(height), C.c_int(int(normalized_range)),
                                 _p(out))
    return out


CAMERA_GRAD_FIELDS = (("q", 4), ("t", 3), ("v", 3), ("w", 3), ("rolling", 2), ("trigger_time", 1),
                      ("pose_time", 1), ("impl", 4))


def camera_grad_fields(kind):
    """The camera's differentiable tensors in pack order, as (name, size): the model's own tensors
    follow the pose (distorted: intrinsics, 8 coefficients, max_radius_sq; fisheye: intrinsics, 4)."""
    if kind == "distorted":
        return CAMERA_GRAD_FIELDS + (("dist", 8), ("max_radius_sq", 1))
    if kind == "fisheye":
        return CAMERA_GRAD_FIELDS + (("dist", 4),)
    return CAMERA_GRAD_FIELDS


def grad_elements(kind):
    return sum(n for _, n in camera_grad_fields(kind))


def camera_rays_bwd(spec, width, height, d_ray_o, d_ray_d, world_space=True, normalized=True, prec="f32"):
    """camera_ray_backward_kernel_cuda (ray_kernels.h:61-161): the gradient of the rays w.r.t. the
    camera, summed over pixels, in ``camera_grad_fields(kind)`` order (``d_ray_o`` may be None)."""
    _, nt = _real(prec)
    cam = camera(spec, prec)
    d_ray_o, d_ray_d = _arr(d_ray_o, nt), _arr(d_ray_d, nt)
    out = np.zeros(grad_elements(spec.kind), nt)
    _lib(prec).orc_camera_rays_bwd(C.byref(cam), C.c_int(width), C.c_int(height), C.c_int(int(world_space)),
                                   C.c_int(int(normalized)), _p(d_ray_o), _p(d_ray_d), _p(out))
    return out


def pixel_uv(spec, width, height):
    """Pixel centres' uv (base_camera_impl.h:9-14; lidar v from the beam table, spherical.h:77-82)."""
    u = (np.arange(width, dtype=np.float64) + 0.5) / width
    if spec.kind == "lidar":
        v = np.asarray(spec.beam_v, np.float64)[:height]
    else:
        v = (np.arange(height, dtype=np.float64) + 0.5) / height
    return np.stack(np.broadcast_arrays(u[None, :], v[:, None]), -1)


def pixel_time(spec, width=None, height=None, uv=None, delta=False):
    """pixel_time[_delta][_from_uv] forward (camera.h:89-99), float64."""
    if uv is None:
        uv = pixel_uv(spec, width, height)
    uv = np.asarray(uv, np.float64)
    t = spec.trigger_time + uv[..., 0] * spec.rolling[0] + uv[..., 1] * spec.rolling[1]
    return t - spec.pose_time if delta else t


def pixel_time_bwd(spec, grad, width=0, height=0, uv=None, delta=False, prec="f32"):
    """pixel_time[_delta][_from_uv] backward (time_kernels.h:123-330): 21 camera values (as
    ``camera_rays_bwd``) and, with ``uv``, the uv gradient."""
    _, nt = _real(prec)
    cam = camera(spec, prec)
    grad = _arr(grad, nt)
    uv = _arr(uv, nt)
    out = np.zeros(grad_elements(spec.kind), nt)
    d_uv = np.zeros_like(uv) if uv is not None else None
    n = grad.size
    _lib(prec).orc_pixel_time_bwd(C.byref(cam), C.c_int(width), C.c_int(height), _p(uv), C.c_long(n),
                                  C.c_int(int(delta)), _p(grad), _p(out), _p(d_uv))
    return (out, d_uv) if uv is not None else out


def sh_fwd(degree, origin, positions, coeffs, dc=None, mask=None, layout_3kn=False, prec="f32"):
    """spherical_harmonics_fused_fwd (csrc/color/sh_fwd.cu:119-245)."""
    _, nt = _real(prec)
    origin, positions, coeffs, dc = _arr(origin, nt), _arr(positions, nt), _arr(coeffs, nt), _arr(dc, nt)
    mask = _arr(mask, np.uint32)
    n = coeffs.shape[2] if layout_3kn else coeffs.shape[0]
    dim = coeffs.shape[1]
    out = np.zeros((n, 3), nt)
    _lib(prec).orc_sh_fwd(C.c_int(degree), _p(origin), C.c_int(n), C.c_int(dim), _p(positions),
                          _p(coeffs), _p(dc), _p(mask), C.c_int(int(layout_3kn)), _p(out))
    return out


def sh_bwd(degree, origin, positions, coeffs, d_output, dc=None, mask=None, layout_3kn=False, prec="f32"):
    """spherical_harmonics_fused_bwd (csrc/color/sh_bwd.cu:250-376).

    Returns ``d_coeffs, d_coeffs_dc (or empty), d_positions, d_origin``.
    """
    _, nt = _real(prec)
    origin, positions, coeffs = _arr(origin, nt), _arr(positions, nt), _arr(coeffs, nt)
    d_output, dc, mask = _arr(d_output, nt), _arr(dc, nt), _arr(mask, np.uint32)
    n = coeffs.shape[2] if layout_3kn else coeffs.shape[0]
    dim = coeffs.shape[1]
    d_coeffs = np.zeros_like(coeffs)
    d_dc = np.zeros_like(dc) if dc is not None else np.zeros(0, nt)
    d_pos = np.zeros_like(positions)
    d_origin = np.zeros(3, nt)
    _lib(prec).orc_sh_bwd(C.c_int(degree), _p(origin), C.c_int(n), C.c_int(dim), _p(positions),
                          _p(coeffs), _p(mask), C.c_int(int(layout_3kn)), _p(d_output),
                          C.c_int(int(dc is not None)), _p(d_coeffs), _p(d_dc), _p(d_pos), _p(d_origin))
    return d_coeffs, d_dc, d_pos, d_origin


def tile_n_bits(n_tiles: int) -> int:
    return int(np.floor(np.log2(np.float32(n_tiles)))) + 1


def sort_pairs(keys, vals, end_bit):
    """Stable sort by key bits [0, end_bit): cub SortPairs as used in tiling_common.cu:102-162."""
    keys = np.ascontiguousarray(keys, dtype=np.int64).copy()
    vals = np.ascontiguousarray(vals, dtype=np.int32).copy()
    _lib("f32").orc_sort_pairs(C.c_int64(keys.shape[0]), _p(keys), _p(vals), C.c_int(end_bit))
    return keys, vals


def isect_regular(means2d, radii, depths, width, height, tsx, tsy, sort=True):
    """isect_regular_tiles (csrc/tiling/regular_tiling.cu:72-135)."""
    lib = _lib("f32")
    means2d, radii, depths = _arr(means2d, np.float32), _arr(radii, np.float32), _arr(depths, np.float32)
    n = depths.shape[0]
    tpg = np.zeros(n, np.int32)
    lib.orc_isect_regular_count(C.c_int(n), _p(means2d), _p(radii), C.c_int(width), C.c_int(height),
                                C.c_int(tsx), C.c_int(tsy), _p(tpg))
    cum = np.cumsum(tpg.astype(np.int64))
    n_isects = int(cum[-1]) if n else 0
    ids = np.zeros(n_isects, np.int64)
    fl = np.zeros(n_isects, np.int32)
    if n_isects:
        lib.orc_isect_regular_fill(C.c_int(n), _p(means2d), _p(radii), _p(depths), C.c_int(width),
                                   C.c_int(height), C.c_int(tsx), C.c_int(tsy), _p(cum), _p(ids), _p(fl))
    if sort and n_isects:
        ntiles = ((width + tsx - 1) // tsx) * ((height + tsy - 1) // tsy)
        ids, fl = sort_pairs(ids, fl, 32 + tile_n_bits(ntiles))
    return tpg, ids, fl


def isect_spherical_family(kind, spec, points, scale, quat, opacity, flags, means2d, radii, depths,
                           tsx, tsy, width, height, elev=None, vel=None, ut=(0.1, 2.0, 0.0), sort=True,
                           seam_margins=False):
    """isect_lidar_tiles (phm_lidar_tiling.cu:239-351) when kind == "lidar", else
    isect_spherical_tiles (phm_spherical_tiling.cu:179-291).

    With ``seam_margins`` returns instead, per Gaussian, the diagnostic margin of its second span
    (flag-2 Gaussians; inf elsewhere), computed by the f64 build: the smallest ratio of a decision of
    the PositiveDelta re-projection (validity, on-screen extent) or of the span's tile range (tile
    and elevation boundaries) to a bound on the float32 error of the compared value. Below 1, float32
    rounding can decide that span's tiles either way.
    """
    prec = "f64" if seam_margins else "f32"
    lib = _lib(prec)
    cam = camera(spec, prec)
    k = 0 if kind == "lidar" else 1
    f32 = np.float32
    rt = _real(prec)[1]
    points, scale, quat = _arr(points, rt), _arr(scale, rt), _arr(quat, rt)
    opacity, vel = _arr(opacity, rt), _arr(vel, rt)
    flags = _arr(flags, np.uint8)
    means2d, radii, depths = _arr(means2d, f32), _arr(radii, f32), _arr(depths, f32)
    elev = _arr(elev, f32) if elev is not None else np.zeros(1, f32)
    n_elev = elev.shape[0] if kind == "lidar" else 0
    w = ut_weights(*ut, prec=prec)
    n = depths.shape[0]
    tpg = np.zeros(n, np.int32)
    args = [C.c_int(k), C.byref(cam), _p(w), C.c_int(n), _p(points), _p(vel), _p(scale), _p(quat),
            _p(opacity), _p(flags), _p(means2d), _p(radii), _p(depths), _p(elev), C.c_int(n_elev),
            C.c_int(tsx), C.c_int(tsy), C.c_float(width), C.c_float(height)]
    if seam_margins:
        mg = np.full(n, np.inf, rt)
        lib.orc_isect_spherical_family(*args, None, _p(tpg), None, None, _p(mg))
        return mg
    lib.orc_isect_spherical_family(*args, None, _p(tpg), None, None, None)
    cum = np.cumsum(tpg.astype(np.int64))
    n_isects = int(cum[-1]) if n else 0
    ids = np.zeros(n_isects, np.int64)
    fl = np.zeros(n_isects, np.int32)
    if n_isects:
        lib.orc_isect_spherical_family(*args, _p(cum), None, _p(ids), _p(fl), None)
    if kind == "lidar":
        ntw = (int(width) + tsx - 1) // tsx
        ntiles = ntw * n_elev
    else:
        ntiles = int(np.ceil(np.float32(width) / np.float32(tsx))) * int(np.ceil(np.float32(height) / np.float32(tsy)))
    if sort and n_isects:
        ids, fl = sort_pairs(ids, fl, 32 + tile_n_bits(ntiles))
    return tpg, ids, fl


def offset_encode(isect_ids, n_tiles_w, n_tiles_h, n_cams=1):
    """isect_offset_encode (csrc/tiling/tiling_common.cu:25-99); [n_cams, th, tw] when n_cams > 1."""
    ids = np.ascontiguousarray(isect_ids, dtype=np.int64)
    n_tiles = n_tiles_w * n_tiles_h
    out = np.zeros(n_tiles * n_cams, np.int32)
    _lib("f32").orc_offset_encode(C.c_int64(ids.shape[0]), _p(ids), C.c_int(n_tiles), C.c_int(n_cams), _p(out))
    shape = (n_tiles_h, n_tiles_w) if n_cams == 1 else (n_cams, n_tiles_h, n_tiles_w)
    return out.reshape(shape)


def mask_radii(radii, mask=None, packed=None):
    """mask_radii / mask_radii_packed (csrc/tiling/mask_radii.cu:10-88), out of place."""
    radii = np.ascontiguousarray(radii, dtype=np.float32).copy()
    n = radii.shape[0]
    m = _arr(mask, np.uint8)
    pk = _arr(packed, np.uint32)
    _lib("f32").orc_mask_radii(C.c_int(n), _p(m), _p(pk), _p(radii))
    return radii


def _tiles(width, height, tile_w, tile_h):
    return (width + tile_w - 1) // tile_w, (height + tile_h - 1) // tile_h


def _tile_mask(tiles, ntw, nth):
    """uint8 [n_tiles] selecting the tiles to evaluate (None: every tile)."""
    if tiles is None:
        return None
    m = np.zeros(ntw * nth, np.uint8)
    m[np.asarray(tiles, np.int64)] = 1
    return m


def eval3d_fwd(means, quats, scales, colors, opacity, ray_o, ray_d, offsets, flatten_ids, tile_w=16,
               tile_h=16, velocity=None, ray_time_delta=None, prec="f32", counters=False, tiles=None,
               margins=False):
    """rasterize_eval3d_[dynamic_]fwd (eval3d_fwd.cu:34-308; eval3d_dynamic_fwd.cu:37-332).

    Returns ``rgb [H,W,C], depth [H,W], alpha [H,W], last_ids i32 [H,W]`` (+ counters
    ``[evaluated pairs, contributing pairs]`` when requested). ``tiles`` (tile indices) restricts
    the work to those tiles; pixels of other tiles stay zero. ``margins`` appends a diagnostic
    ``[H,W]``: per pixel the smallest ratio of a decision's distance to its threshold (alpha at
    1/255, the transmittance cut-off at 1e-4) over a bound on the float32 error of the compared
    value; below 1, float32 rounding can take that decision either way (meaningful in the f64 build).
    """
    _, nt = _real(prec)
    means, quats, scales = _arr(means, nt), _arr(quats, nt), _arr(scales, nt)
    colors, opacity = _arr(colors, nt), _arr(opacity, nt).reshape(-1)
    ray_o, ray_d = _arr(ray_o, nt), _arr(ray_d, nt)
    velocity, rtd = _arr(velocity, nt), _arr(ray_time_delta, nt)
    offsets = _arr(offsets, np.int32)
    flatten_ids = _arr(flatten_ids, np.int32)
    h, w = ray_o.shape[:2]
    cdim = 0 if colors is None else colors.shape[-1]
    ntw, nth = offsets.shape[-1], offsets.shape[-2]
    rgb = np.zeros((h, w, cdim), nt)
    dep = np.zeros((h, w), nt)
    alp = np.zeros((h, w), nt)
    last = np.zeros((h, w), np.int32)
    cnt = np.zeros(2, np.int64)
    tmask = _tile_mask(tiles, ntw, nth)   # kept alive across the call
    mg = np.full((h, w), np.inf, nt) if margins else None
    _lib(prec).orc_eval3d_fwd(C.c_int(cdim), C.c_int(means.shape[0]), _p(means), _p(quats), _p(scales),
                              _p(colors), _p(opacity), _p(velocity), _p(rtd), C.c_int(w), C.c_int(h),
                              C.c_int(tile_w), C.c_int(tile_h), _p(ray_o), _p(ray_d), _p(offsets),
                              C.c_int(ntw), C.c_int(nth), C.c_int64(flatten_ids.shape[0]),
                              _p(flatten_ids), _p(rgb), _p(dep), _p(alp), _p(last), _p(cnt), _p(tmask), _p(mg))
    out = (rgb, dep, alp, last)
    if counters:
        out = out + (cnt,)
    if margins:
        out = out + (mg,)
    return out


def eval3d_bwd(means, quats, scales, colors, opacity, ray_o, ray_d, offsets, flatten_ids, render_alpha,
               last_ids, v_rgb, v_depth, v_alpha, tile_w=16, tile_h=16, velocity=None,
               ray_time_delta=None, prec="f32", tiles=None, abs_sums=False, und_mode=0):
    """rasterize_eval3d_[dynamic_]bwd (eval3d_bwd.cu:66-403; eval3d_dynamic_bwd.cu:312-432).

    Returns a dict with ``v_means, v_quats, v_scales, v_opacity, v_colors, v_ray_o, v_ray_d``
    (+ ``v_velocity, v_time_delta`` in the dynamic case). ``tiles`` (tile indices) restricts the
    sum to the pixels of those tiles (the gradients of a loss whose upstream gradients are zero
    elsewhere). With ``abs_sums`` also ``abs``: for each of those names, the sum of the magnitudes
    of the per-pair contributions to each element (the conditioning of its float sum).
    ``und_mode`` 1 / 2 takes / drops every pair whose alpha test (1/255) or geometry gate (0.99)
    float32 rounding can decide either way (the forward's alpha error bound; f64 diagnostics).
    """
    _, nt = _real(prec)
    means, quats, scales = _arr(means, nt), _arr(quats, nt), _arr(scales, nt)
    colors, opacity = _arr(colors, nt), _arr(opacity, nt).reshape(-1)
    ray_o, ray_d = _arr(ray_o, nt), _arr(ray_d, nt)
    velocity, rtd = _arr(velocity, nt), _arr(ray_time_delta, nt)
    offsets, flatten_ids = _arr(offsets, np.int32), _arr(flatten_ids, np.int32)
    render_alpha, last_ids = _arr(render_alpha, nt), _arr(last_ids, np.int32)
    v_rgb, v_depth, v_alpha = _arr(v_rgb, nt), _arr(v_depth, nt), _arr(v_alpha, nt)
    h, w = ray_o.shape[:2]
    cdim = 0 if colors is None else colors.shape[-1]
    ntw, nth = offsets.shape[-1], offsets.shape[-2]
    n = means.shape[0]
    out = dict(v_means=np.zeros((n, 3), nt), v_quats=np.zeros((n, 4), nt), v_scales=np.zeros((n, 3), nt),
               v_opacity=np.zeros(n, nt), v_colors=np.zeros((n, cdim), nt) if cdim else None,
               v_ray_o=np.zeros((h, w, 3), nt), v_ray_d=np.zeros((h, w, 3), nt))
    if velocity is not None:
        out["v_velocity"] = np.zeros((n, 3), nt)
        out["v_time_delta"] = np.zeros((h, w), nt)
    tmask = _tile_mask(tiles, ntw, nth)   # kept alive across the call
    ag = 11 + cdim + (3 if velocity is not None else 0)
    abs_g = np.zeros((n, ag), nt) if abs_sums else None
    abs_px = np.zeros((h, w, 7), nt) if abs_sums else None
    _lib(prec).orc_eval3d_bwd(
        C.c_int(cdim), _p(means), _p(quats), _p(scales), _p(colors), _p(opacity), _p(velocity), _p(rtd),
        C.c_int(w), C.c_int(h), C.c_int(tile_w), C.c_int(tile_h), _p(ray_o), _p(ray_d), _p(offsets),
        C.c_int(ntw), C.c_int(nth), C.c_int64(flatten_ids.shape[0]), _p(flatten_ids), _p(render_alpha),
        _p(last_ids), _p(v_rgb), _p(v_depth), _p(v_alpha), _p(out["v_means"]), _p(out["v_quats"]),
        _p(out["v_scales"]), _p(out["v_opacity"]), _p(out["v_colors"]), _p(out["v_ray_o"]),
        _p(out["v_ray_d"]), _p(out.get("v_velocity")), _p(out.get("v_time_delta")), _p(tmask), _p(abs_g),
        _p(abs_px), C.c_int(und_mode))
    if abs_sums:
        a = dict(v_means=abs_g[:, 0:3], v_quats=abs_g[:, 3:7], v_scales=abs_g[:, 7:10], v_opacity=abs_g[:, 10],
                 v_colors=abs_g[:, 11:11 + cdim] if cdim else None, v_ray_o=abs_px[..., 0:3],
                 v_ray_d=abs_px[..., 3:6])
        if velocity is not None:
            a["v_velocity"] = abs_g[:, 11 + cdim:14 + cdim]
            a["v_time_delta"] = abs_px[..., 6]
        out["abs"] = a
    return out


def margin_pointer_live(prec: str = "f64") -> bool:
    """Whether the calling thread still holds a decision-margin pointer (test hook)."""
    return bool(_lib(prec).orc_margin_pointer_live())


def num_threads() -> int:
    return int(_lib("f32").orc_num_threads())


def set_num_threads(n: int) -> None:
    _lib("f32").orc_set_num_threads(C.c_int(n))


# ------------------------------------------------------------------ scene-assembly producers
def packed_mask_from_instances(instance_ids, instance_mask):
    """packed_mask_from_instances (csrc/nodes/gs_masking.cu:8-47): uint32[(N + 31) // 32]."""
    ids = _arr(instance_ids, np.int32).reshape(-1)
    m = _arr(instance_mask, np.uint8).reshape(-1)
    out = np.zeros((ids.size + 31) // 32, np.uint32)
    _lib("f32").orc_packed_mask_from_instances(C.c_long(ids.size), _p(ids), _p(m), C.c_long(m.size), _p(out))
    return out


def _offsets(per_instance_offsets, gs_inst_offsets):
    if (per_instance_offsets is None) != (gs_inst_offsets is None):
        raise ValueError("per_instance_offsets and gs_inst_offsets go together")
    return _arr(per_instance_offsets, np.int32), _arr(gs_inst_offsets, np.int32)


def rigid_fwd(positions, rotations, instance_id, inst_q, inst_t, inst_v, inst_w, inst_mask, out_positions,
              out_rotations, out_velocities=None, out_mask=None, buffer_offset=0, per_instance_offsets=None,
              gs_inst_offsets=None, prec="f32"):
    """copy_gs_rigid_transform_fwd (csrc/nodes/container.cu:13-75, 171-215) on copies of the output
    buffers, which are returned: ``out_positions, out_rotations, out_velocities, out_mask``."""
    _, nt = _real(prec)
    pos, rot = _arr(positions, nt), _arr(rotations, nt)
    ids = _arr(instance_id, np.int32)
    iq, it, iv, iw = (_arr(x, nt) for x in (inst_q, inst_t, inst_v, inst_w))
    im = _arr(inst_mask, np.uint8)
    po, go = _offsets(per_instance_offsets, gs_inst_offsets)
    op, orot = _arr(out_positions, nt).copy(), _arr(out_rotations, nt).copy()
    ov = _arr(out_velocities, nt).copy() if out_velocities is not None else None
    om = _arr(out_mask, np.uint8).copy() if out_mask is not None else None
    _lib(prec).orc_rigid_fwd(C.c_long(pos.shape[0]), _p(pos), _p(rot), _p(ids), _p(iq), _p(it), _p(iv), _p(iw),
                             _p(im), C.c_long(im.size), C.c_long(buffer_offset), _p(po), _p(go),
                             C.c_long(op.shape[0]), _p(op), _p(orot), _p(ov), _p(om))
    return op, orot, ov, (om.astype(bool) if om is not None else None)


def rigid_bwd(positions, rotations, instance_id, inst_q, inst_w, inst_mask, buffer_offset, per_instance_offsets,
              gs_inst_offsets, v_positions, v_rotations, v_velocities, prec="f32"):
    """copy_gs_rigid_transform_bwd (csrc/nodes/container.cu:78-160, 218-266): ``grad_positions,
    grad_rotations, grad_q, grad_t, grad_v, grad_w``."""
    _, nt = _real(prec)
    pos, rot = _arr(positions, nt), _arr(rotations, nt)
    ids = _arr(instance_id, np.int32)
    iq, iw = _arr(inst_q, nt), _arr(inst_w, nt)
    im = _arr(inst_mask, np.uint8)
    po, go = _offsets(per_instance_offsets, gs_inst_offsets)
    vp, vr = _arr(v_positions, nt), _arr(v_rotations, nt)
    vv = _arr(v_velocities, nt)
    n, k = pos.shape[0], iq.shape[0]
    gp, gr = np.zeros((n, 3), nt), np.zeros((n, 4), nt)
    gq, gt, gv, gw = np.zeros((k, 4), nt), np.zeros((k, 3), nt), np.zeros((k, 3), nt), np.zeros((k, 3), nt)
    _lib(prec).orc_rigid_bwd(C.c_long(n), _p(pos), _p(rot), _p(ids), _p(iq), _p(iw), _p(im), C.c_long(k),
                             C.c_long(buffer_offset), _p(po), _p(go), C.c_long(vp.shape[0]), _p(vp), _p(vr), _p(vv),
                             _p(gp), _p(gr), _p(gq), _p(gt), _p(gv), _p(gw))
    return gp, gr, gq, gt, gv, gw
