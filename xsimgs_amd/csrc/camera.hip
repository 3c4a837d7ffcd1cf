// Camera kernels: unscented-transform projection (plain and phase-modelled), point projection,
// per-pixel rays and pixel times. One thread per Gaussian / point / pixel, 256-thread blocks.
#include "xsg_common.h"

#include <algorithm>

namespace {

constexpr int kBlock = 256;

// One sigma point of a static pinhole camera (static_camera_projection in central mode) from its
// camera-space point: perspective divide as one reciprocal (1 ulp), the on-screen test, the
// fixed-point pixel-time steps, and the pixel position. The steps are those of the loop
// residual = (pose_time + p) - real_time, p -= residual, at most five, ending below thr: the first
// residual is pose_time - real_time (p starts at 0), and a static pose usually ends there (no
// rolling shutter) or after the second; later steps run only for the lanes that need them.
XSG_DEV bool static_pinhole_point(const Camera& c, const ProjParams& pp, f2 img, f3 pc, f2& px) {
    const float iz = __builtin_amdgcn_rcpf(pc.z);
    const float u = pc.x * c.i0 * iz + c.i2;
    const float v = pc.y * c.i1 * iz + c.i3;
    px = mk2(u * img.x, v * img.y);
    const bool on_screen = !((pc.z <= 0.0f) || (u < -pp.margin) || (u > 1.0f + pp.margin) || (v < -pp.margin) ||
                             (v > 1.0f + pp.margin));
    const float real_time = pixel_time(c, u, v);
    float residual = c.pose_time - real_time;
    if (!(fabsf(residual) < pp.thr)) {
        float p_time = -residual;
        residual = (c.pose_time + p_time) - real_time;
        for (int i = 2; i < 5 && !(fabsf(residual) < pp.thr); ++i) {
            p_time -= residual;
            residual = (c.pose_time + p_time) - real_time;
        }
    }
    return on_screen && fabsf(residual) < pp.max_res;
}

// ut_projection (central mode) for a static pinhole camera: the seven camera-space points are
// M (pw - t0) +- M d_i with M the pose's rotation, each projected by static_pinhole_point; the
// mean, covariance, radii and on-screen test as in ut_projection. Outputs as ut_projection's.
XSG_DEV bool ut_projection_static_pinhole(const Camera& c, const Mat3& m, const UtWeights& ut, f2 img,
                                          const ProjParams& pp, f3 pw, float opac, const f3 d[3], f2& mean2d,
                                          f2& radii, float& depth) {
    const f3 pc0 = mul(m, pw - c.t0);
    f2 pts[7];
    bool result = static_pinhole_point(c, pp, img, pc0, pts[0]);
    f2 cov_xx_xy = mk2(0.f, 0.f);
    float cov_yy = 0.f;
    if (result) {
        mean2d = mk2(ut.wm0 * pts[0].x, ut.wm0 * pts[0].y);
        depth = pc0.z;
        bool valid = true;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const f3 e = mul(m, d[k]);
            valid = static_pinhole_point(c, pp, img, pc0 + e, pts[1 + 2 * k]) && valid;
            valid = static_pinhole_point(c, pp, img, pc0 - e, pts[2 + 2 * k]) && valid;
        }
#pragma unroll
        for (int i = 1; i < 7; ++i) {
            mean2d.x += ut.wi * pts[i].x;
            mean2d.y += ut.wi * pts[i].y;
        }
        if (!valid) {
            result = false;
        } else {
            float vx = pts[0].x - mean2d.x, vy = pts[0].y - mean2d.y;
            float cx = ut.wc0 * (vx * vx), cxy = ut.wc0 * (vx * vy), cy = ut.wc0 * (vy * vy);
#pragma unroll
            for (int i = 1; i < 7; ++i) {
                vx = pts[i].x - mean2d.x; vy = pts[i].y - mean2d.y;
                cx += ut.wi * (vx * vx); cxy += ut.wi * (vx * vy); cy += ut.wi * (vy * vy);
            }
            const float det = cx * cy - cxy * cxy;
            if (det <= 0.0f || cx < 0 || cy < 0) result = false;
            cov_xx_xy = mk2(cx, cxy);
            cov_yy = cy;
        }
    }
    if (!result) return false;  // the caller keeps nothing of a failed projection
    const float extend = ut_extend(opac);
    radii = mk2(extend * hw_sqrt(fmaxf(0.0f, cov_xx_xy.x)), extend * hw_sqrt(fmaxf(0.0f, cov_yy)));
    const bool ix = !(((mean2d.x + radii.x) < 0) || (img.x < (mean2d.x - radii.x)));
    const bool iy = !(((mean2d.y + radii.y) < 0) || (img.y < (mean2d.y - radii.y)));
    return ix && iy;
}

// One Gaussian's inputs, read once (a rig's projection reuses them for every camera).
struct UtIn {
    f3 pw, pv, sc;
    float4 q;
    float op;
};

XSG_DEV UtIn load_ut_in(int64_t i, const float* __restrict__ means, const float* __restrict__ vel,
                        const float* __restrict__ scales, const float4* __restrict__ quats,
                        const float* __restrict__ opacity) {
    UtIn in;
    in.op = opacity ? opacity[i] : 1.0f;
    in.q = quats[i];
    in.sc = ld3(scales + 3 * i);
    in.pw = ld3(means + 3 * i);
    in.pv = vel ? ld3(vel + 3 * i) : mk3(0.f, 0.f, 0.f);
    return in;
}

template <int KIND>
XSG_DEV void ut_project_in(const UtIn& in, const Camera& cam, bool is_static, const Mat3& m, const ProjParams& pp,
                           const UtWeights& ut, f2 img, uint8_t& flag, f2& m2, f2& r2, float& depth) {
    flag = 0;
    m2 = mk2(0.f, 0.f);
    r2 = mk2(0.f, 0.f);
    depth = 0.f;
    if (in.op >= 1.0f / 255.0f) {
        f3 d[3];
        float dep = 0.f;
        f2 mm = mk2(0.f, 0.f), rr = mk2(0.f, 0.f);
        bool ok;
        if (KIND == XSG_CAM_PINHOLE && is_static) {
            ut_deltas_rsq(ut.sqrt_dl, in.q, in.sc, d);
            ok = ut_projection_static_pinhole(cam, m, ut, img, pp, in.pw, in.op, d, mm, rr, dep);
        } else {
            ut_deltas(ut.sqrt_dl, in.q, in.sc, d);
            float udist = 0.f;
            ok = ut_projection<KIND>(cam, XSG_MODE_CENTRAL, ut, img, pp, in.pw, in.pv, in.op, d, is_static, mm, rr,
                                     dep, udist);
        }
        if (ok) {
            flag = 1; m2 = mm; r2 = rr; depth = dep;
        }
    }
}

// unscented_transform_kernel (include/cameras/ut_kernels.h:187-246) over n_cams cameras of one kind
// (one for projection_utgs; a rig's cameras, an extension, for projection_utgs_rig): each thread reads
// its Gaussian once and projects it with every camera in camera order, so that a rig's projections
// equal the single-camera ones bit for bit (one compiled path). Outputs are [n_cams, n]
// camera-major; every element is written (zeros for culled Gaussians), which replaces the
// reference's zero-initialised allocations (ut_kernels.h:276-280) with a single pass. A static
// pinhole camera takes the lean path above. One thread per Gaussian (two per thread, sharing the
// camera set-up, measured slower: half as many wavefronts hide less latency; compacting the Gaussians
// that pass the centre test before the sigma points, too).
template <int KIND>
__global__ __launch_bounds__(kBlock) void ut_project_kernel(
    int n_cams, int64_t n, const float* __restrict__ packs, int64_t pack_stride, ProjParams pp, UtWeights ut, f2 img,
    const float* __restrict__ means, const float* __restrict__ vel, const float* __restrict__ scales,
    const float4* __restrict__ quats, const float* __restrict__ opacity, uint8_t* __restrict__ flags,
    float2* __restrict__ radii, float2* __restrict__ means2d, float* __restrict__ depths) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const UtIn in = load_ut_in(i, means, vel, scales, quats, opacity);
    for (int c = 0; c < n_cams; ++c) {  // uniform
        const Camera cam = load_camera(packs + (int64_t)c * pack_stride, KIND);
        const bool is_static = camera_is_static(cam, vel != nullptr);
        const Mat3 m = static_world_to_camera(cam);
        uint8_t flag;
        f2 m2, r2;
        float depth;
        ut_project_in<KIND>(in, cam, is_static, m, pp, ut, img, flag, m2, r2, depth);
        const int64_t o = (int64_t)c * n + i;
        flags[o] = flag;
        radii[o] = make_float2(r2.x, r2.y);
        means2d[o] = make_float2(m2.x, m2.y);
        depths[o] = depth;
    }
}

// unscented_transform_phm_kernel (include/cameras/ut_phm_kernels.h:13-114), one instantiation per kind
// of pose. A static pose shares the sigma points' (u, v, range) between the three phase modes and needs
// about half the registers of a moving one, so it has a kernel of its own; the host launches both (the
// moving one on a small grid-striding grid) and each returns at once for the other kind of pose,
// which only the device's copy of the camera tells.
template <int KIND, bool STATIC_POSE>
__global__ __launch_bounds__(kBlock) void ut_project_phm_kernel(
    int64_t n, const float* __restrict__ pack, ProjParams pp, UtWeights ut, f2 img,
    const float* __restrict__ means, const float* __restrict__ vel, const float* __restrict__ scales,
    const float4* __restrict__ quats, const float* __restrict__ opacity, uint8_t* __restrict__ flags,
    float2* __restrict__ radii, float2* __restrict__ means2d, float* __restrict__ depths) {
    const Camera cam = load_camera(pack, KIND);
    if (camera_is_static(cam, vel != nullptr) != STATIC_POSE) return;
    const PhaseUnwrap unwrap = phase_unwrap(cam);
    const float u_pi = float(M_PI) * img.x / fabsf(cam.i1);
    // the static kernel's grid covers the Gaussians once; a loop there would keep per-lane copies of the
    // camera terms live across iterations and cost occupancy
    const int64_t stride = STATIC_POSE ? n : (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        const float op = opacity ? opacity[i] : 1.0f;
        uint8_t flag = 0;
        f2 m_out = mk2(0.f, 0.f), r_out = mk2(0.f, 0.f);
        float d_out = 0.f;
        if (op >= 1.0f / 255.0f) {
            f3 d[3];
            ut_deltas(ut.sqrt_dl, quats[i], ld3(scales + 3 * i), d);
            const f3 pw = ld3(means + 3 * i);
            f2 rc = mk2(0.f, 0.f), rl = rc, rr = rc, mc = rc, ml = rc, mr = rc;
            float dc = 0.f, dl = 0.f, dr = 0.f, ud = 0.f;
            SigmaUv sa;
            f3 pv = mk3(0.f, 0.f, 0.f);
            const float ext = ut_extend(op);
            if constexpr (STATIC_POSE) sigma_uv(cam, pw, d, sa);
            else if (vel) pv = ld3(vel + 3 * i);
            auto project = [&](int mode, f2& m2, f2& r2, float& dd) {
                if constexpr (STATIC_POSE)
                    return ut_projection_sigma_uv(cam, unwrap, mode, ut, img, pp, ext, sa, m2, r2, dd, ud);
                else
                    return ut_projection<KIND>(cam, mode, ut, img, pp, pw, pv, op, d, false, m2, r2, dd, ud);
            };
            bool res = project(XSG_MODE_CENTRAL, mc, rc, dc);
            if (res) {
                const int r_c = int(res) * (int(ud > u_pi) + 1);
                int r_l, r_r;
                if (STATIC_POSE && fabsf(cam.roll_u) == 0.0f) {
                    // Global shutter: u_pose is 0.5 and every mode starts its time solve at +-0, so a
                    // side mode whose unwrap shifts none of the seven points repeats the central
                    // projection bit for bit. With roll_u 0 the negative mode shifts the points left of
                    // u_pose, the positive mode those right of it; most Gaussians lie on one side, so
                    // each lane projects the one side mode that differs (its own mode), and only
                    // Gaussians across u_pose project both.
                    bool lo = false, hi = false;
#pragma unroll
                    for (int k = 0; k < 7; ++k) {
                        lo |= sa.u[k] < unwrap.u_pose;
                        hi |= sa.u[k] > unwrap.u_pose;
                    }
                    f2 m1 = mk2(0.f, 0.f), r1 = m1, m2 = m1, r2 = m1;
                    float d1 = 0.f, d2 = 0.f;
                    int r_1 = r_c, r_2 = r_c;
                    if (lo || hi) {
                        res = project(lo ? XSG_MODE_NEGATIVE : XSG_MODE_POSITIVE, m1, r1, d1);
                        r_1 = int(res) * (int(ud > u_pi) + 1);
                    }
                    if (lo && hi) {
                        res = project(XSG_MODE_POSITIVE, m2, r2, d2);
                        r_2 = int(res) * (int(ud > u_pi) + 1);
                    }
                    ml = lo ? m1 : mc; rl = lo ? r1 : rc; dl = lo ? d1 : dc; r_l = lo ? r_1 : r_c;
                    mr = hi ? (lo ? m2 : m1) : mc;
                    rr = hi ? (lo ? r2 : r1) : rc;
                    dr = hi ? (lo ? d2 : d1) : dc;
                    r_r = hi ? (lo ? r_2 : r_1) : r_c;
                } else {
                    res = project(XSG_MODE_NEGATIVE, ml, rl, dl);
                    r_l = int(res) * (int(ud > u_pi) + 1);
                    res = project(XSG_MODE_POSITIVE, mr, rr, dr);
                    r_r = int(res) * (int(ud > u_pi) + 1);
                }
                if (r_l == 1 && r_r == 1) {
                    flag = 2; r_out = rl; m_out = ml; d_out = dl;
                } else if (r_c == 1) {
                    flag = 1; r_out = rc; m_out = mc; d_out = dc;
                } else if (r_l == 1 || r_r == 1) {
                    // ut_phm_kernels.h:417-421 selects the side whose result is *not* 1
                    const bool use_left = r_l != 1;
                    flag = 1;
                    r_out = use_left ? rl : rr;
                    m_out = use_left ? ml : mr;
                    d_out = use_left ? dl : dr;
                }
            }
        }
        flags[i] = flag;
        radii[i] = make_float2(r_out.x, r_out.y);
        means2d[i] = make_float2(m_out.x, m_out.y);
        depths[i] = d_out;
    }
}

// Workgroups of the moving-pose phase-modelled kernel: enough to fill every CU at that kernel's
// occupancy (four waves per SIMD), striding over the Gaussians; a static pose's launch of it returns
// after one camera load per workgroup.
constexpr int kPhmMovingBlocks = 1024;

// camera_projection_fwd (include/cameras/projection_kernels.h:259-309)
template <int KIND>
__global__ __launch_bounds__(kBlock) void project_points_kernel(
    int64_t n, const float* __restrict__ pack, ProjParams pp, int mode, int no_jac,
    const float* __restrict__ pts, const float* __restrict__ vel, float4* __restrict__ uvdt,
    uint8_t* __restrict__ mask) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const Camera c = load_camera(pack, KIND);
    const f3 pw = ld3(pts + 3 * i);
    const f3 pv = vel ? ld3(vel + 3 * i) : mk3(0.f, 0.f, 0.f);
    float4 r;
    bool valid = true;
    if (!no_jac) {
        camera_projection<KIND>(c, pw, pv, pp, mode, false, r, valid);
    } else {
        // camera_projection_iteration (projection_kernels.h:177-198): plain fixed-point update
        f3 uvd = mk3(0.f, 0.f, 0.f);
        float p_time = 0.f, residual = 0.f;
        if (mode == XSG_MODE_NEGATIVE) p_time = -fabsf(c.roll_u) * 0.5f;
        else if (mode == XSG_MODE_POSITIVE) p_time = fabsf(c.roll_u) * 0.5f;
        bool bad = false;
        for (int it = 0; it < 5; ++it) {
            f3 pc, jpc;
            world_to_camera_jac(c, pw, pv, p_time, pc, jpc);
            uvd = point_to_uvd<KIND>(c, mode, pc);
            residual = (c.pose_time + p_time) - pixel_time(c, uvd.x, uvd.y);
            p_time -= residual;
            if ((uvd.z <= 0.0f) || (uvd.x < -pp.margin) || (uvd.x > 1.0f + pp.margin) ||
                (uvd.y < -pp.margin) || (uvd.y > 1.0f + pp.margin)) {
                bad = true;
                break;
            }
            if (fabsf(residual) < pp.thr) break;
        }
        if (bad) {
            valid = false;
            r = make_float4(0.f, 0.f, 0.f, 0.f);
        } else {
            r = make_float4(uvd.x, uvd.y, uvd.z, p_time);
            valid = (fabsf(residual) < pp.max_res) && (uvd.z > 0.0f);
        }
    }
    r.w += c.pose_time;
    uvdt[i] = r;
    valid = valid && (r.x >= 0.0f && r.y >= 0.0f) && (r.x <= 1.0f && r.y <= 1.0f);
    mask[i] = valid;
}

template <int KIND>
XSG_DEV f2 pixel_uv(const Camera& c, int px, int py, int width, int height) {
    // base_camera_impl.h:9-14; LidarCameraImpl::pixel_to_uv (csrc/cameras/spherical.h:73-79)
    const float u = (static_cast<float>(px) + 0.5f) / static_cast<float>(width);
    if constexpr (KIND == XSG_CAM_LIDAR) return mk2(u, c.beam_v[py]);
    return mk2(u, (static_cast<float>(py) + 0.5f) / static_cast<float>(height));
}

// Image kernels run on 64 x 4 pixel workgroups: lane = column within a 64-wide strip, wavefront =
// row, grid (ceil(width / 64), ceil(height / 4)); no integer division per pixel.
constexpr int kStrip = 64, kStripRows = kBlock / 64;
inline dim3 image_grid(int width, int height, int rows_per_thread = 1) {
    return dim3((unsigned)((width + kStrip - 1) / kStrip),
                (unsigned)((height + kStripRows * rows_per_thread - 1) / (kStripRows * rows_per_thread)));
}

template <int KIND>
XSG_DEV f3 pixel_to_camera_ray(const Camera& c, f2 uv) {
    if constexpr (KIND == XSG_CAM_PINHOLE) {  // perspective.cu:13-16
        return mk3((uv.x - c.i2) / c.i0, (uv.y - c.i3) / c.i1, 1.0f);
    } else if constexpr (KIND == XSG_CAM_DISTORTED) {  // distorted_perspective.cu:100-105
        DistState st;
        const f2 uc = undistort_uv(c, mk2((uv.x - c.i2) / c.i0, (uv.y - c.i3) / c.i1), st);
        return mk3(uc.x, uc.y, 1.0f);
    } else if constexpr (KIND == XSG_CAM_FISHEYE) {  // fisheye_opencv.cu:48-62
        const float x = (uv.x - c.i2) / c.i0, y = (uv.y - c.i3) / c.i1;
        const float delta = sqrtf(x * x + y * y);
        float residual;
        const float th = fisheye_solve_theta(c, delta, residual);
        if (th <= 0.0f) return mk3(0.f, 0.f, 1.0f);
        float st, ct;
        sincosf(th, &st, &ct);
        const float sf = st / delta;
        return mk3(sf * x, sf * y, ct);
    } else {  // spherical.h:9-22, 121-127
        const float az = c.i0 + uv.x * c.i1;
        const float el = c.i2 + uv.y * c.i3;
        float se, ce, sa, ca;
        sincosf(el, &se, &ce);
        sincosf(az, &sa, &ca);
        const float xy = 1.0f * ce;
        return mk3(xy * sa, xy * ca, 1.0f * se);
    }
}

// ray_valid (camera.h:114-120): the distorted model's undistortion converged to 1e-5 inside
// max_radius (distorted_perspective.cu:107-117), the fisheye solve converged on the rising branch of
// the polynomial (fisheye_opencv.cu:64-72); the other models are valid everywhere
template <int KIND>
XSG_DEV bool ray_valid(const Camera& c, f2 uv) {
    if constexpr (KIND == XSG_CAM_DISTORTED) {
        DistState st;
        const f2 ud = mk2((uv.x - c.i2) / c.i0, (uv.y - c.i3) / c.i1);
        const f2 uc = undistort_uv(c, ud, st);
        const float rx = uc.x * st.scale + st.dx - ud.x, ry = uc.y * st.scale + st.dy - ud.y;
        const float r2 = uc.x * uc.x + uc.y * uc.y;
        return (r2 <= c.max_r2) && (fabsf(rx) < 1e-5f) && (fabsf(ry) < 1e-5f);
    } else if constexpr (KIND == XSG_CAM_FISHEYE) {
        const float x = (uv.x - c.i2) / c.i0, y = (uv.y - c.i3) / c.i1;
        const float delta = sqrtf(x * x + y * y);
        if (delta <= 1e-8f) return true;
        float residual;
        const float th = fisheye_solve_theta(c, delta, residual);
        return (fabsf(residual) < 1e-5f) && (fisheye_distortion_deriv(c, th) > 0.0f);
    } else {
        return true;
    }
}

// launch_camera_ray_fwd (include/cameras/ray_kernels.h:7-59) with Camera::camera_ray
// (camera.h:101-131): pose at the pixel's time delta, q = exp(w dt) * q0, t = t0 + v dt.
// Each thread covers kRayRows rows of one column. A static pinhole camera (no v, no w) maps every
// pixel by the one rotation M of q0 (quat_apply as a matrix, exact for any quaternion); its
// camera-space ray is ((u - cx) / fx, (v - cy) / fy, 1), where x is fixed per thread and y per row.
constexpr int kRayRows = 4;

template <int KIND>
XSG_DEV void camera_ray_pixel(const Camera& c, int px, int py, int width, int height, int world_space,
                              int normalized, float* __restrict__ ray_o, float* __restrict__ ray_d,
                              uint8_t* __restrict__ valid) {
    const int64_t idx = (int64_t)py * width + px;
    const f2 uv = pixel_uv<KIND>(c, px, py, width, height);
    f3 ray = pixel_to_camera_ray<KIND>(c, uv);
    if (normalized) ray = ray * (1.0f / sqrtf(dot(ray, ray)));
    f3 o = mk3(0.f, 0.f, 0.f);
    if (world_space) {
        const float dt = pixel_time(c, uv.x, uv.y) - c.pose_time;
        float w1, dw1; f3 xyz1, dxyz1;
        jac_quat_from_axis_angle(c.w, dt, w1, xyz1, dw1, dxyz1);
        const float qw = w1 * c.qw - dot(xyz1, c.qv);
        const f3 qv = c.qw * xyz1 + w1 * c.qv + cross(xyz1, c.qv);
        o = c.t0 + c.v * dt;
        ray = quat_apply(qw, qv, ray);
    }
    if (ray_o) st3(ray_o + 3 * idx, o);
    st3(ray_d + 3 * idx, ray);
    if (valid) valid[idx] = ray_valid<KIND>(c, uv) ? 1 : 0;
}

template <int KIND>
__global__ __launch_bounds__(kBlock) void camera_rays_kernel(
    const float* __restrict__ pack, int width, int height, int world_space, int normalized,
    float* __restrict__ ray_o, float* __restrict__ ray_d, uint8_t* __restrict__ valid) {
    const int px = (int)blockIdx.x * kStrip + (int)(threadIdx.x & 63);
    const int py0 = ((int)blockIdx.y * kStripRows + (int)(threadIdx.x >> 6)) * kRayRows;
    if (px >= width || py0 >= height) return;
    const int py1 = min(height, py0 + kRayRows);
    const Camera c = load_camera(pack, KIND);
    if (KIND == XSG_CAM_PINHOLE && camera_is_static(c, false)) {
        Mat3 m;
        m.r0 = mk3(1.f, 0.f, 0.f); m.r1 = mk3(0.f, 1.f, 0.f); m.r2 = mk3(0.f, 0.f, 1.f);
        if (world_space) {
            const float w = c.qw, x = c.qv.x, y = c.qv.y, z = c.qv.z;
            m.r0 = mk3(1.f - 2.f * (y * y + z * z), 2.f * (x * y - w * z), 2.f * (x * z + w * y));
            m.r1 = mk3(2.f * (x * y + w * z), 1.f - 2.f * (x * x + z * z), 2.f * (y * z - w * x));
            m.r2 = mk3(2.f * (x * z - w * y), 2.f * (y * z + w * x), 1.f - 2.f * (x * x + y * y));
        }
        const f3 o = world_space ? c.t0 : mk3(0.f, 0.f, 0.f);
        const float rx = ((static_cast<float>(px) + 0.5f) / static_cast<float>(width) - c.i2) / c.i0;
        for (int py = py0; py < py1; ++py) {
            const int64_t idx = (int64_t)py * width + px;
            const float ry = ((static_cast<float>(py) + 0.5f) / static_cast<float>(height) - c.i3) / c.i1;
            f3 ray = mk3(rx, ry, 1.0f);
            if (normalized) ray = ray * __builtin_amdgcn_rsqf(rx * rx + ry * ry + 1.0f);
            ray = mul(m, ray);
            if (ray_o) st3(ray_o + 3 * idx, o);
            st3(ray_d + 3 * idx, ray);
            if (valid) valid[idx] = 1;
        }
        return;
    }
    for (int py = py0; py < py1; ++py)
        camera_ray_pixel<KIND>(c, px, py, width, height, world_space, normalized, ray_o, ray_d, valid);
}

// uv_in given: one thread per uv (1D grid); else one thread per pixel (image grid)
template <int KIND>
__global__ __launch_bounds__(kBlock) void pixel_time_kernel(
    const float* __restrict__ pack, int width, int height, const float2* __restrict__ uv_in,
    int64_t n, int delta, float* __restrict__ out) {
    const Camera c = load_camera(pack, KIND);
    int64_t idx;
    f2 uv;
    if (uv_in) {
        idx = (int64_t)blockIdx.x * kBlock + threadIdx.x;
        if (idx >= n) return;
        uv = mk2(uv_in[idx].x, uv_in[idx].y);
    } else {
        const int px = (int)blockIdx.x * kStrip + (int)(threadIdx.x & 63);
        const int py = (int)blockIdx.y * kStripRows + (int)(threadIdx.x >> 6);
        if (px >= width || py >= height) return;
        idx = (int64_t)py * width + px;
        uv = pixel_uv<KIND>(c, px, py, width, height);
    }
    float t = pixel_time(c, uv.x, uv.y);
    if (delta) t = t - c.pose_time;
    out[idx] = t;
}

// undistort_map (distortion.h:33-56) with distort_uv (distorted_perspective.cu:199-203,
// fisheye_opencv.cu:150-156): the distorted position of each pixel's undistorted uv, in [0, 1] with
// normalized_range, else mapped to [-1, 1]
template <int KIND>
__global__ __launch_bounds__(kBlock) void undistort_map_kernel(const float* __restrict__ pack, int width, int height,
                                                               int normalized_range, float2* __restrict__ out) {
    const int px = (int)blockIdx.x * kStrip + (int)(threadIdx.x & 63);
    const int py = (int)blockIdx.y * kStripRows + (int)(threadIdx.x >> 6);
    if (px >= width || py >= height) return;
    const int64_t idx = (int64_t)py * width + px;
    const Camera c = load_camera(pack, KIND);
    const f2 uv = pixel_uv<KIND>(c, px, py, width, height);
    const float x = (uv.x - c.i2) / c.i0, y = (uv.y - c.i3) / c.i1;
    float ru, rv;
    if constexpr (KIND == XSG_CAM_DISTORTED) {
        float scale, du, dv;
        uv_distortion(c, x, y, scale, du, dv);
        ru = (x * scale + du) * c.i0 + c.i2;
        rv = (y * scale + dv) * c.i1 + c.i3;
    } else {
        const float th = sqrtf(x * x + y * y);
        const float scale = (th > 1e-8f) ? fisheye_distortion(c, th) / th : 1.0f;
        ru = x * scale * c.i0 + c.i2;
        rv = y * scale * c.i1 + c.i3;
    }
    out[idx] = normalized_range ? make_float2(ru, rv) : make_float2(ru * 2.0f - 1.0f, rv * 2.0f - 1.0f);
}

// --------------------------------------------------------------------------------------------
// Camera gradients. Per thread the gradient w.r.t. the camera's parameters in pack order (q0, t0,
// v, w, rolling_time, trigger_time, pose_time, then the model's tensors, camera.h:144), reduced per
// block into partials; grad_final_kernel sums the partials in a fixed order and writes the whole
// pack gradient (0 for the lidar beam address and the distorted model's max_radius^2).
template <int KIND>
constexpr int cam_grad_count() {
    return KIND == XSG_CAM_DISTORTED ? 29 : KIND == XSG_CAM_FISHEYE ? 25 : 21;
}
constexpr int kCamGradMax = 29;

template <int NV>
XSG_DEV void block_partials(const float (&g)[NV], float* __restrict__ part, int64_t block) {
    __shared__ float s_w[kBlock / 64][NV];
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const float t = wave_sum(g[k]);
        if (__lane_id() == 0) s_w[wave][k] = t;
    }
    __syncthreads();
    if ((int)threadIdx.x < NV) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < kBlock / 64; ++w) t += s_w[w][threadIdx.x];
        part[block * NV + threadIdx.x] = t;
    }
}

// camera_ray_backward_kernel_cuda (ray_kernels.h:61-161) for this build's pose model: ray_o =
// t0 + v dt, ray_d = q (x) n, q = (cos(theta/2), w dt sigma) (x) q0 with theta = |w| |dt| and
// sigma = sin(theta/2) / theta (jac_quat_from_axis_angle), dt = pixel_time - pose_time.
// Each thread sums kGradRows pixels of its column (rows wave, wave + 4, ...) in registers before the
// workgroup reduction, so a 1080p frame leaves about a thousand partial rows.
constexpr int kGradRows = 8;

template <int KIND>
__global__ __launch_bounds__(kBlock) void camera_rays_bwd_kernel(const float* __restrict__ pack, int width,
                                                                 int height, int world_space, int normalized,
                                                                 const float* __restrict__ d_ray_o,
                                                                 const float* __restrict__ d_ray_d,
                                                                 float* __restrict__ part) {
    constexpr int NG = cam_grad_count<KIND>();
    const Camera c = load_camera(pack, KIND);
    float g[NG];
#pragma unroll
    for (int k = 0; k < NG; ++k) g[k] = 0.f;
    const int px = (int)blockIdx.x * kStrip + (int)(threadIdx.x & 63);
    const int py0 = (int)blockIdx.y * kStripRows * kGradRows + (int)(threadIdx.x >> 6);
    for (int rr = 0; rr < kGradRows; ++rr) {
        const int py = py0 + rr * kStripRows;
        if (px >= width || py >= height) continue;  // every thread takes part in the reduction below
        const int64_t idx = (int64_t)py * width + px;
        const f2 uv = pixel_uv<KIND>(c, px, py, width, height);
        const f3 r = pixel_to_camera_ray<KIND>(c, uv);
        const float il = 1.0f / sqrtf(dot(r, r));
        const f3 n = normalized ? r * il : r;
        const f3 gd = ld3(d_ray_d + 3 * idx);
        const f3 go = d_ray_o ? ld3(d_ray_o + 3 * idx) : mk3(0.f, 0.f, 0.f);
        f3 dn = gd;
        if (world_space) {
            const float dt = pixel_time(c, uv.x, uv.y) - c.pose_time;
            float w1, dw1; f3 xyz1, dxyz1;
            jac_quat_from_axis_angle(c.w, dt, w1, xyz1, dw1, dxyz1);
            const float w2 = c.qw; const f3 xyz2 = c.qv;
            const float qw = w1 * w2 - dot(xyz1, xyz2);
            const f3 qv = w2 * xyz1 + w1 * xyz2 + cross(xyz1, xyz2);
            float d_dt = dot(go, c.v);  // ray_o = t0 + v dt
            g[4] += go.x; g[5] += go.y; g[6] += go.z;
            g[7] += dt * go.x; g[8] += dt * go.y; g[9] += dt * go.z;
            // ray_d = n + 2 (qw (qv x n) + qv x (qv x n))
            dn = gd + 2.0f * (cross(qv, cross(qv, gd)) - qw * cross(qv, gd));
            const float d_qw = 2.0f * dot(gd, cross(qv, n));
            const f3 d_qv = (2.0f * qw) * cross(n, gd) + (2.0f * dot(gd, qv)) * n + (2.0f * dot(qv, n)) * gd -
                            (4.0f * dot(gd, n)) * qv;
            // q = (w1, xyz1) (x) (w2, xyz2)
            const float d_w1 = d_qw * w2 + dot(d_qv, xyz2);
            const f3 d_xyz1 = w2 * d_qv - d_qw * xyz2 + cross(xyz2, d_qv);
            const float d_w2 = d_qw * w1 + dot(d_qv, xyz1);
            const f3 d_xyz2 = w1 * d_qv - d_qw * xyz1 + cross(d_qv, xyz1);
            g[0] += d_w2; g[1] += d_xyz2.x; g[2] += d_xyz2.y; g[3] += d_xyz2.z;
            // (w1, xyz1) = (cos(theta/2), w dt sigma); kappa = dt |dt| sigma'(theta) / |w|
            d_dt += d_w1 * dw1 + dot(d_xyz1, dxyz1);
            const float wn = sqrtf(dot(c.w, c.w));
            const float theta = wn * fabsf(dt);
            float sigma, kappa;
            if (theta < 1e-2f) {
                sigma = 0.5f - theta * theta * (1.0f / 48.0f);
                kappa = -dt * dt * dt * (1.0f / 24.0f);
            } else {
                float sh, ch;
                sincosf(0.5f * theta, &sh, &ch);
                sigma = sh / theta;
                kappa = dt * fabsf(dt) * (0.5f * theta * ch - sh) / (theta * theta * wn);
            }
            const f3 d_w = (-d_w1 * dt * dt * sigma * 0.5f + kappa * dot(d_xyz1, c.w)) * c.w + (dt * sigma) * d_xyz1;
            g[10] += d_w.x; g[11] += d_w.y; g[12] += d_w.z;
            // dt = trigger_time + uv . rolling_time - pose_time
            g[13] += d_dt * uv.x; g[14] += d_dt * uv.y; g[15] += d_dt; g[16] += -d_dt;
        }
        const f3 dr = normalized ? (dn - dot(n, dn) * n) * il : dn;
        if constexpr (KIND == XSG_CAM_PINHOLE) {  // perspective.cu:19-33
            const float ifx = 1.0f / c.i0, ify = 1.0f / c.i1;
            g[17] += -dr.x * (uv.x - c.i2) * ifx * ifx;
            g[18] += -dr.y * (uv.y - c.i3) * ify * ify;
            g[19] += -dr.x * ifx;
            g[20] += -dr.y * ify;
        } else if constexpr (KIND == XSG_CAM_DISTORTED) {
            // distorted_perspective.cu:121-188: re-solve, then at the solution g_d = J^-T dr.xy (J is
            // symmetric; dr.xy / scale where J is nearly singular) and dL/dk = -g_d . dD/dk
            const float ifx = 1.0f / c.i0, ify = 1.0f / c.i1;
            const f2 ud = mk2((uv.x - c.i2) * ifx, (uv.y - c.i3) * ify);
            DistState st;
            const f2 uc = undistort_uv(c, ud, st);
            st = distortion_state(c, uc.x, uc.y);
            const float det = st.juu * st.jvv - st.juv * st.juv;
            float gx, gy;
            if (fabsf(det) <= kDistMinDet) {
                gx = dr.x / st.scale; gy = dr.y / st.scale;
            } else {
                gx = (st.jvv * dr.x - st.juv * dr.y) / det;
                gy = (st.juu * dr.y - st.juv * dr.x) / det;
            }
            g[17] += -gx * ud.x * ifx;
            g[18] += -gy * ud.y * ify;
            g[19] += -gx * ifx;
            g[20] += -gy * ify;
            const float r2 = uc.x * uc.x + uc.y * uc.y, r4 = r2 * r2, r6 = r4 * r2;
            const float d_rad = -(gx * uc.x + gy * uc.y) / st.denom;
            const float d_rad_den = -d_rad * st.scale;
            g[21] += d_rad * r2;
            g[22] += d_rad * r4;
            g[23] += -(gx * 2.0f * uc.x * uc.y + gy * (r2 + 2.0f * uc.y * uc.y));
            g[24] += -(gx * (r2 + 2.0f * uc.x * uc.x) + gy * 2.0f * uc.x * uc.y);
            g[25] += d_rad * r6;
            g[26] += d_rad_den * r2;
            g[27] += d_rad_den * r4;
            g[28] += d_rad_den * r6;
        } else if constexpr (KIND == XSG_CAM_FISHEYE) {
            // fisheye_opencv.cu:74-136: theta(delta, k) implicit through theta_d(theta, k) = delta
            const float x = (uv.x - c.i2) / c.i0, y = (uv.y - c.i3) / c.i1;
            const float delta = sqrtf(x * x + y * y);
            float residual;
            const float th = fisheye_solve_theta(c, delta, residual);
            const float deriv = fisheye_distortion_deriv(c, th);
            if (th > 0.0f && delta > 1e-8f && fabsf(residual) < 1e-5f && deriv > 1e-3f) {
                float st, ct;
                sincosf(th, &st, &ct);
                const float inv_delta = 1.0f / delta;
                const float sf = st * inv_delta;
                const float d_s = dr.x * x + dr.y * y;
                const float d_th = d_s * ct * inv_delta - dr.z * st;
                const float dts = d_th / deriv;
                const float t2 = th * th, t3 = t2 * th;
                g[21] += -dts * t3;
                g[22] += -dts * t3 * t2;
                g[23] += -dts * t3 * t2 * t2;
                g[24] += -dts * t3 * t2 * t2 * t2;
                const float d_delta = -d_s * st * inv_delta * inv_delta + dts;
                const float gx = sf * dr.x + d_delta * x * inv_delta;
                const float gy = sf * dr.y + d_delta * y * inv_delta;
                g[17] += -gx * x / c.i0;
                g[18] += -gy * y / c.i1;
                g[19] += -gx / c.i0;
                g[20] += -gy / c.i1;
            }
        }  // the spherical and lidar models carry no intrinsics gradient (base_camera_impl.h:19-22)
    }
    block_partials<NG>(g, part, (int64_t)blockIdx.y * gridDim.x + blockIdx.x);
}

// pixel_time[_delta][_from_uv]_bwd_kernel (time_kernels.h:123-330): partial sums of g u, g v and g;
// with uv given, d_uv = g rolling_time
template <int KIND>
__global__ __launch_bounds__(kBlock) void pixel_time_bwd_kernel(const float* __restrict__ pack, int width,
                                                                int height, const float2* __restrict__ uv_in,
                                                                int64_t n, const float* __restrict__ grad,
                                                                float2* __restrict__ d_uv, float* __restrict__ part) {
    const Camera c = load_camera(pack, KIND);
    float g[3] = {0.f, 0.f, 0.f};
    for (int rr = 0; rr < kGradRows; ++rr) {
        int64_t idx;
        f2 uv;
        if (uv_in) {  // 1D: element blockIdx.x * kBlock * kGradRows + rr * kBlock + thread
            idx = ((int64_t)blockIdx.x * kGradRows + rr) * kBlock + threadIdx.x;
            if (idx >= n) continue;
            uv = mk2(uv_in[idx].x, uv_in[idx].y);
        } else {
            const int px = (int)blockIdx.x * kStrip + (int)(threadIdx.x & 63);
            const int py = (int)blockIdx.y * kStripRows * kGradRows + (int)(threadIdx.x >> 6) + rr * kStripRows;
            if (px >= width || py >= height) continue;
            idx = (int64_t)py * width + px;
            uv = pixel_uv<KIND>(c, px, py, width, height);
        }
        const float gr = grad[idx];
        if (d_uv) d_uv[idx] = make_float2(gr * c.roll_u, gr * c.roll_v);
        g[0] += gr * uv.x; g[1] += gr * uv.y; g[2] += gr;
    }
    block_partials<3>(g, part, (int64_t)blockIdx.y * gridDim.x + blockIdx.x);
}

// one workgroup: out[e] = sum over blocks of part[b][k] for the nv partial values, placed at the pack
// positions: rays (`rays`) with k = e for the first nv elements; times (nv = 3) at rolling_time,
// trigger_time and, for the delta variants, minus the trigger sum at pose_time; every other pack
// element 0.
constexpr int kFinalBlock = 1024;
__global__ __launch_bounds__(kFinalBlock) void grad_final_kernel(const float* __restrict__ part, int nb, int nv,
                                                                 int rays, int delta, int pack_elems,
                                                                 float* __restrict__ out) {
    const int wave = threadIdx.x >> 6, lane = __lane_id();
    for (int e = wave; e < pack_elems; e += kFinalBlock / 64) {
        const int k = rays ? e : (e == 13 ? 0 : e == 14 ? 1 : (e == 15 || (e == 16 && delta)) ? 2 : -1);
        float t = 0.f;
        if (k >= 0 && k < nv) {
            float t4[4] = {0.f, 0.f, 0.f, 0.f};  // four independent load chains
            int b = lane;
            for (; b + 192 < nb; b += 256) {
#pragma unroll
                for (int u = 0; u < 4; ++u) t4[u] += part[(int64_t)(b + 64 * u) * nv + k];
            }
            for (; b < nb; b += 64) t4[0] += part[(int64_t)b * nv + k];
            t = (t4[0] + t4[1]) + (t4[2] + t4[3]);
        }
        t = wave_sum(t);
        if (lane == 0) out[e] = (!rays && delta && e == 16) ? -t : t;
    }
}

UtWeights ut_weights(float a, float b, float k) {  // ut_kernels.h:17-36 (host, float32)
    const float lam = a * a * (3 + k) - 3;
    UtWeights w;
    w.wm0 = lam / (3 + lam);
    w.wc0 = lam / (3 + lam) + (1 - a * a + b);
    w.wi = 1 / (2 * (3 + lam));
    w.sqrt_dl = sqrtf(lam + 3);
    return w;
}

}  // namespace

// shared with tiling.hip (seam re-projection)
UtWeights xsg_ut_weights(float a, float b, float k) { return ut_weights(a, b, k); }

extern "C" int xsg_ut_project(int kind, int phm, const float* pack, int64_t n, const float* means,
                              const float* velocity, const float* scales, const float* quats,
                              const float* opacity, float width, float height, float ut_alpha,
                              float ut_beta, float ut_kappa, float residual_thr, float max_residual,
                              float max_margin, uint8_t* flags, float* radii, float* means2d,
                              float* depths, xsg_stream_t stream) {
    if (n < 0 || !pack) return xsg_fail(XSG_ERR_INVALID, "xsg_ut_project: bad arguments");
    if (xsg_camera_pack_elements(kind) <= 0) return XSG_ERR_INVALID;
    if (phm && kind != XSG_CAM_SPHERICAL && kind != XSG_CAM_LIDAR)
        return xsg_fail(XSG_ERR_UNSUPPORTED, "projection_utgs_phm needs a spherical or lidar camera");
    if (n == 0) return XSG_OK;
    if (!means || !scales || !quats || !flags || !radii || !means2d || !depths)
        return xsg_fail(XSG_ERR_INVALID, "xsg_ut_project: null tensor");
    const ProjParams pp{residual_thr, max_residual, max_margin};
    const UtWeights ut = ut_weights(ut_alpha, ut_beta, ut_kappa);
    const f2 img = mk2(width, height);
    const dim3 grid(xsg_blocks(n, kBlock)), block(kBlock);
    const hipStream_t s = (hipStream_t)stream;
    auto q4 = reinterpret_cast<const float4*>(quats);
    auto r2 = reinterpret_cast<float2*>(radii);
    auto m2 = reinterpret_cast<float2*>(means2d);
    const int rc = xsg_with_camera_kind(kind, [&](auto k) {
        constexpr int KIND = decltype(k)::value;
        if constexpr (KIND == XSG_CAM_SPHERICAL || KIND == XSG_CAM_LIDAR) {
            if (phm) {
                // a point velocity makes every pose a moving one
                if (!velocity)
                    ut_project_phm_kernel<KIND, true><<<grid, block, 0, s>>>(n, pack, pp, ut, img, means, velocity,
                                                                             scales, q4, opacity, flags, r2, m2,
                                                                             depths);
                const dim3 grid_m(std::min<unsigned>(grid.x, kPhmMovingBlocks));
                ut_project_phm_kernel<KIND, false><<<grid_m, block, 0, s>>>(n, pack, pp, ut, img, means, velocity,
                                                                            scales, q4, opacity, flags, r2, m2,
                                                                            depths);
                return;
            }
        }
        ut_project_kernel<KIND><<<grid, block, 0, s>>>(1, n, pack, xsg_camera_pack_elements(kind), pp, ut, img, means,
                                                       velocity, scales, q4, opacity, flags, r2, m2, depths);
    });
    if (rc != XSG_OK) return rc;
    XSG_TRY_LAUNCH("ut_project");
    return XSG_OK;
}

extern "C" int xsg_ut_project_rig(int kind, int n_cams, const float* packs, int64_t pack_stride, int64_t n,
                                  const float* means, const float* velocity, const float* scales, const float* quats,
                                  const float* opacity, float width, float height, float ut_alpha, float ut_beta,
                                  float ut_kappa, float residual_thr, float max_residual, float max_margin,
                                  uint8_t* flags, float* radii, float* means2d, float* depths, xsg_stream_t stream) {
    const int pe = xsg_camera_pack_elements(kind);
    if (pe <= 0) return XSG_ERR_INVALID;
    if (kind == XSG_CAM_SPHERICAL || kind == XSG_CAM_LIDAR)
        return xsg_fail(XSG_ERR_UNSUPPORTED, "xsg_ut_project_rig takes pinhole, distorted or fisheye cameras");
    if (n < 0 || n_cams < 0 || pack_stride < pe)
        return xsg_fail(XSG_ERR_INVALID, "xsg_ut_project_rig: bad arguments (pack stride %lld for %d elements)",
                        (long long)pack_stride, pe);
    if (n == 0 || n_cams == 0) return XSG_OK;
    if (!packs || !means || !scales || !quats || !flags || !radii || !means2d || !depths)
        return xsg_fail(XSG_ERR_INVALID, "xsg_ut_project_rig: null tensor");
    const ProjParams pp{residual_thr, max_residual, max_margin};
    const UtWeights ut = ut_weights(ut_alpha, ut_beta, ut_kappa);
    const f2 img = mk2(width, height);
    const hipStream_t s = (hipStream_t)stream;
    const int rc = xsg_with_camera_kind(kind, [&](auto k) {
        constexpr int KIND = decltype(k)::value;
        if constexpr (KIND != XSG_CAM_SPHERICAL && KIND != XSG_CAM_LIDAR)
            ut_project_kernel<KIND><<<xsg_blocks(n, kBlock), kBlock, 0, s>>>(
                n_cams, n, packs, pack_stride, pp, ut, img, means, velocity, scales,
                reinterpret_cast<const float4*>(quats), opacity, flags, reinterpret_cast<float2*>(radii),
                reinterpret_cast<float2*>(means2d), depths);
    });
    if (rc != XSG_OK) return rc;
    XSG_TRY_LAUNCH("ut_project_rig");
    return XSG_OK;
}

extern "C" int xsg_project_points(int kind, const float* pack, int64_t n, const float* points,
                                  const float* velocity, float residual_thr, float max_residual,
                                  float max_margin, int mode, int no_jacobian, float* uvdt,
                                  uint8_t* mask, xsg_stream_t stream) {
    if (n < 0 || !pack) return xsg_fail(XSG_ERR_INVALID, "xsg_project_points: bad arguments");
    if (xsg_camera_pack_elements(kind) <= 0) return XSG_ERR_INVALID;
    if (n == 0) return XSG_OK;
    const ProjParams pp{residual_thr, max_residual, max_margin};
    const dim3 grid(xsg_blocks(n, kBlock)), block(kBlock);
    const hipStream_t s = (hipStream_t)stream;
    auto u4 = reinterpret_cast<float4*>(uvdt);
    const int rc = xsg_with_camera_kind(kind, [&](auto k) {
        project_points_kernel<decltype(k)::value><<<grid, block, 0, s>>>(n, pack, pp, mode, no_jacobian, points,
                                                                         velocity, u4, mask);
    });
    if (rc != XSG_OK) return rc;
    XSG_TRY_LAUNCH("project_points");
    return XSG_OK;
}

extern "C" int xsg_camera_rays(int kind, const float* pack, int width, int height, int world_space,
                               int normalized, float* ray_o, float* ray_d, uint8_t* valid,
                               xsg_stream_t stream) {
    if (width < 0 || height < 0 || !pack || !ray_d)
        return xsg_fail(XSG_ERR_INVALID, "xsg_camera_rays: bad arguments");
    if (xsg_camera_pack_elements(kind) <= 0) return XSG_ERR_INVALID;
    const int64_t n = (int64_t)width * height;
    if (n == 0) return XSG_OK;
    const dim3 grid = image_grid(width, height, kRayRows), block(kBlock);
    const hipStream_t s = (hipStream_t)stream;
    const int rc = xsg_with_camera_kind(kind, [&](auto k) {
        camera_rays_kernel<decltype(k)::value><<<grid, block, 0, s>>>(pack, width, height, world_space, normalized,
                                                                      ray_o, ray_d, valid);
    });
    if (rc != XSG_OK) return rc;
    XSG_TRY_LAUNCH("camera_rays");
    return XSG_OK;
}

extern "C" int xsg_pixel_time(int kind, const float* pack, int width, int height, const float* uv,
                              int64_t n_uv, int delta, float* out, xsg_stream_t stream) {
    const int64_t n = uv ? n_uv : (int64_t)width * height;
    if (n < 0 || !pack || !out) return xsg_fail(XSG_ERR_INVALID, "xsg_pixel_time: bad arguments");
    if (xsg_camera_pack_elements(kind) <= 0) return XSG_ERR_INVALID;
    if (n == 0) return XSG_OK;
    const dim3 grid = uv ? dim3(xsg_blocks(n, kBlock)) : image_grid(width, height), block(kBlock);
    const hipStream_t s = (hipStream_t)stream;
    auto uv2 = reinterpret_cast<const float2*>(uv);
    const int rc = xsg_with_camera_kind(kind, [&](auto k) {
        pixel_time_kernel<decltype(k)::value><<<grid, block, 0, s>>>(pack, width, height, uv2, n, delta, out);
    });
    if (rc != XSG_OK) return rc;
    XSG_TRY_LAUNCH("pixel_time");
    return XSG_OK;
}

extern "C" int xsg_undistort_map(int kind, const float* pack, int width, int height, int normalized_range,
                                 float* out, xsg_stream_t stream) {
    if (kind != XSG_CAM_DISTORTED && kind != XSG_CAM_FISHEYE)
        return xsg_fail(XSG_ERR_INVALID, "undistort_map needs a distorted perspective or fisheye camera");
    if (width < 0 || height < 0 || !pack || !out) return xsg_fail(XSG_ERR_INVALID, "xsg_undistort_map: bad arguments");
    const int64_t n = (int64_t)width * height;
    if (n == 0) return XSG_OK;
    const dim3 grid = image_grid(width, height), block(kBlock);
    const hipStream_t s = (hipStream_t)stream;
    auto o2 = reinterpret_cast<float2*>(out);
    if (kind == XSG_CAM_DISTORTED)
        undistort_map_kernel<XSG_CAM_DISTORTED><<<grid, block, 0, s>>>(pack, width, height, normalized_range, o2);
    else
        undistort_map_kernel<XSG_CAM_FISHEYE><<<grid, block, 0, s>>>(pack, width, height, normalized_range, o2);
    XSG_TRY_LAUNCH("undistort_map");
    return XSG_OK;
}

extern "C" size_t xsg_camera_rays_bwd_workspace_bytes(int width, int height) {
    const dim3 g = image_grid(width > 0 ? width : 1, height > 0 ? height : 1, kGradRows);
    return sizeof(float) * (size_t)kCamGradMax * g.x * g.y;
}

extern "C" int xsg_camera_rays_bwd(int kind, const float* pack, int width, int height, int world_space,
                                   int normalized, const float* d_ray_o, const float* d_ray_d, float* grad_pack,
                                   void* workspace, xsg_stream_t stream) {
    const int pe = xsg_camera_pack_elements(kind);
    if (pe <= 0) return XSG_ERR_INVALID;
    if (width < 0 || height < 0) return xsg_fail(XSG_ERR_INVALID, "camera_rays_bwd: negative size");
    if (!pack || !grad_pack || !workspace || (!d_ray_d && (int64_t)width * height > 0))
        return xsg_fail(XSG_ERR_INVALID, "camera_rays_bwd: null pointer");
    if (const int rc = xsg_check_workspace(workspace, "camera_rays_bwd")) return rc;
    const dim3 grid = image_grid(width > 0 ? width : 1, height > 0 ? height : 1, kGradRows);
    const int nb = (int)(grid.x * grid.y);
    float* part = (float*)workspace;
    const hipStream_t s = (hipStream_t)stream;
    int ng = 0;
    const int rc = xsg_with_camera_kind(kind, [&](auto k) {
        constexpr int KIND = decltype(k)::value;
        ng = cam_grad_count<KIND>();
        camera_rays_bwd_kernel<KIND><<<grid, kBlock, 0, s>>>(pack, width, height, world_space, normalized, d_ray_o,
                                                             d_ray_d, part);
    });
    if (rc != XSG_OK) return rc;
    grad_final_kernel<<<1, kFinalBlock, 0, s>>>(part, nb, ng, 1, 0, pe, grad_pack);
    XSG_TRY_LAUNCH("camera_rays_bwd");
    return XSG_OK;
}

// pixel_time_bwd's workgroups: an image grid of kGradRows rows per thread for pixels, else
// kBlock * kGradRows uvs per workgroup
inline dim3 time_bwd_grid(int width, int height, bool from_uv, int64_t n) {
    if (from_uv) return dim3(xsg_blocks(n > 0 ? n : 1, (int64_t)kBlock * kGradRows));
    return image_grid(width > 0 ? width : 1, height > 0 ? height : 1, kGradRows);
}

extern "C" size_t xsg_pixel_time_bwd_workspace_bytes(int width, int height, int64_t n_uv) {
    // enough for either layout: the image grid of width x height and the 1D grid of n_uv
    const dim3 gi = time_bwd_grid(width, height, false, 0), gu = time_bwd_grid(0, 0, true, n_uv);
    const size_t nb = std::max<size_t>((size_t)gi.x * gi.y, (size_t)gu.x * gu.y);
    return sizeof(float) * 3 * nb;
}

extern "C" int xsg_pixel_time_bwd(int kind, const float* pack, int width, int height, const float* uv,
                                  int64_t n_uv, int delta, const float* grad, float* grad_pack, float* d_uv,
                                  void* workspace, xsg_stream_t stream) {
    const int pe = xsg_camera_pack_elements(kind);
    if (pe <= 0) return XSG_ERR_INVALID;
    const int64_t n = uv ? n_uv : (int64_t)width * height;
    if (n < 0 || (!uv && (width < 0 || height < 0))) return xsg_fail(XSG_ERR_INVALID, "pixel_time_bwd: bad size");
    if (!pack || !grad_pack || !workspace || (n > 0 && !grad))
        return xsg_fail(XSG_ERR_INVALID, "pixel_time_bwd: null pointer");
    if (const int rc = xsg_check_workspace(workspace, "pixel_time_bwd")) return rc;
    const dim3 grid = time_bwd_grid(width, height, uv != nullptr, n);
    const int nb = (int)(grid.x * grid.y);
    float* part = (float*)workspace;
    const hipStream_t s = (hipStream_t)stream;
    const float2* uv2 = (const float2*)uv;
    float2* duv2 = uv ? (float2*)d_uv : nullptr;
    const int rc = xsg_with_camera_kind(kind, [&](auto k) {
        pixel_time_bwd_kernel<decltype(k)::value><<<grid, kBlock, 0, s>>>(pack, width, height, uv2, n, grad, duv2,
                                                                          part);
    });
    if (rc != XSG_OK) return rc;
    grad_final_kernel<<<1, kFinalBlock, 0, s>>>(part, nb, 3, 0, delta ? 1 : 0, pe, grad_pack);
    XSG_TRY_LAUNCH("pixel_time_bwd");
    return XSG_OK;
}
