// Camera kernels: unscented-transform projection (plain and phase-modelled), point projection,
// per-pixel rays and pixel times. One thread per Gaussian / point / pixel, 256-thread blocks.
#include "xsg_common.h"

namespace {

constexpr int kBlock = 256;

// unscented_transform_kernel (include/cameras/ut_kernels.h:187-246). Every output element is
// written (zeros for culled Gaussians), which replaces the reference's zero-initialised
// allocations (ut_kernels.h:276-280) with a single pass.
template <int KIND>
__global__ __launch_bounds__(kBlock) void ut_project_kernel(
    int64_t n, const float* __restrict__ pack, ProjParams pp, UtWeights ut, f2 img,
    const float* __restrict__ means, const float* __restrict__ vel, const float* __restrict__ scales,
    const float4* __restrict__ quats, const float* __restrict__ opacity, uint8_t* __restrict__ flags,
    float2* __restrict__ radii, float2* __restrict__ means2d, float* __restrict__ depths) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const Camera cam = load_camera(pack, KIND);
    const bool is_static = camera_is_static(cam, vel != nullptr);
    const float op = opacity ? opacity[i] : 1.0f;
    uint8_t flag = 0;
    f2 m2 = mk2(0.f, 0.f), r2 = mk2(0.f, 0.f);
    float depth = 0.f;
    if (op >= 1.0f / 255.0f) {
        f3 d[3];
        ut_deltas(ut.sqrt_dl, quats[i], ld3(scales + 3 * i), d);
        const f3 pv = vel ? ld3(vel + 3 * i) : mk3(0.f, 0.f, 0.f);
        float udist = 0.f, dep = 0.f;
        f2 mm = mk2(0.f, 0.f), rr = mk2(0.f, 0.f);
        if (ut_projection<KIND>(cam, XSG_MODE_CENTRAL, ut, img, pp, ld3(means + 3 * i), pv, op, d,
                                is_static, mm, rr, dep, udist)) {
            flag = 1; m2 = mm; r2 = rr; depth = dep;
        }
    }
    flags[i] = flag;
    radii[i] = make_float2(r2.x, r2.y);
    means2d[i] = make_float2(m2.x, m2.y);
    depths[i] = depth;
}

// unscented_transform_phm_kernel (include/cameras/ut_phm_kernels.h:13-114)
template <int KIND>
__global__ __launch_bounds__(kBlock) void ut_project_phm_kernel(
    int64_t n, const float* __restrict__ pack, ProjParams pp, UtWeights ut, f2 img,
    const float* __restrict__ means, const float* __restrict__ vel, const float* __restrict__ scales,
    const float4* __restrict__ quats, const float* __restrict__ opacity, uint8_t* __restrict__ flags,
    float2* __restrict__ radii, float2* __restrict__ means2d, float* __restrict__ depths) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const Camera cam = load_camera(pack, KIND);
    const bool is_static = camera_is_static(cam, vel != nullptr);
    const float op = opacity ? opacity[i] : 1.0f;
    uint8_t flag = 0;
    f2 m_out = mk2(0.f, 0.f), r_out = mk2(0.f, 0.f);
    float d_out = 0.f;
    if (op >= 1.0f / 255.0f) {
        f3 d[3];
        ut_deltas(ut.sqrt_dl, quats[i], ld3(scales + 3 * i), d);
        const f3 pw = ld3(means + 3 * i);
        const f3 pv = vel ? ld3(vel + 3 * i) : mk3(0.f, 0.f, 0.f);
        f2 rc = mk2(0.f, 0.f), rl = rc, rr = rc, mc = rc, ml = rc, mr = rc;
        float dc = 0.f, dl = 0.f, dr = 0.f, ud = 0.f;
        bool res = ut_projection<KIND>(cam, XSG_MODE_CENTRAL, ut, img, pp, pw, pv, op, d, is_static,
                                       mc, rc, dc, ud);
        if (res) {
            const float u_pi = float(M_PI) * img.x / fabsf(cam.i1);
            const int r_c = int(res) * (int(ud > u_pi) + 1);
            res = ut_projection<KIND>(cam, XSG_MODE_NEGATIVE, ut, img, pp, pw, pv, op, d, is_static,
                                      ml, rl, dl, ud);
            const int r_l = int(res) * (int(ud > u_pi) + 1);
            res = ut_projection<KIND>(cam, XSG_MODE_POSITIVE, ut, img, pp, pw, pv, op, d, is_static,
                                      mr, rr, dr, ud);
            const int r_r = int(res) * (int(ud > u_pi) + 1);
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

template <int KIND>
XSG_DEV f3 pixel_to_camera_ray(const Camera& c, f2 uv) {
    if constexpr (KIND == XSG_CAM_PINHOLE) {  // perspective.cu:13-16
        return mk3((uv.x - c.i2) / c.i0, (uv.y - c.i3) / c.i1, 1.0f);
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

// launch_camera_ray_fwd (include/cameras/ray_kernels.h:7-59) with Camera::camera_ray
// (camera.h:101-131): pose at the pixel's time delta, q = exp(w dt) * q0, t = t0 + v dt.
template <int KIND>
__global__ __launch_bounds__(kBlock) void camera_rays_kernel(
    const float* __restrict__ pack, int width, int height, int world_space, int normalized,
    float* __restrict__ ray_o, float* __restrict__ ray_d, uint8_t* __restrict__ valid) {
    const int64_t idx = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (idx >= (int64_t)width * height) return;
    const Camera c = load_camera(pack, KIND);
    const int px = (int)(idx % width), py = (int)(idx / width);
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
    if (valid) valid[idx] = 1;  // no ray_valid on pinhole / spherical / lidar impls (camera.h:117-123)
}

template <int KIND>
__global__ __launch_bounds__(kBlock) void pixel_time_kernel(
    const float* __restrict__ pack, int width, int height, const float2* __restrict__ uv_in,
    int64_t n, int delta, float* __restrict__ out) {
    const int64_t idx = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (idx >= n) return;
    const Camera c = load_camera(pack, KIND);
    f2 uv;
    if (uv_in) {
        uv = mk2(uv_in[idx].x, uv_in[idx].y);
    } else {
        uv = pixel_uv<KIND>(c, (int)(idx % width), (int)(idx / width), width, height);
    }
    float t = pixel_time(c, uv.x, uv.y);
    if (delta) t = t - c.pose_time;
    out[idx] = t;
}

// --------------------------------------------------------------------------------------------
// Camera gradients. Per thread the gradient w.r.t. the camera's 21 parameters (q0, t0, v, w,
// rolling_time, trigger_time, pose_time, intrinsics: the camera's tensors in order, camera.h:144),
// reduced per block into partials; grad_final_kernel sums the partials in a fixed order and writes
// the whole pack gradient (the lidar beam address gets 0).
constexpr int kCamGrad = 21;

XSG_DEV float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <int NV>
XSG_DEV void block_partials(const float (&g)[NV], float* __restrict__ part) {
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
        part[(int64_t)blockIdx.x * NV + threadIdx.x] = t;
    }
}

// camera_ray_backward_kernel_cuda (ray_kernels.h:61-161) for this build's pose model: ray_o =
// t0 + v dt, ray_d = q (x) n, q = (cos(theta/2), w dt sigma) (x) q0 with theta = |w| |dt| and
// sigma = sin(theta/2) / theta (jac_quat_from_axis_angle), dt = pixel_time - pose_time.
template <int KIND>
__global__ __launch_bounds__(kBlock) void camera_rays_bwd_kernel(const float* __restrict__ pack, int width,
                                                                 int height, int world_space, int normalized,
                                                                 const float* __restrict__ d_ray_o,
                                                                 const float* __restrict__ d_ray_d,
                                                                 float* __restrict__ part) {
    const int64_t idx = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const Camera c = load_camera(pack, KIND);
    float g[kCamGrad];
#pragma unroll
    for (int k = 0; k < kCamGrad; ++k) g[k] = 0.f;
    if (idx < (int64_t)width * height) {  // every thread takes part in the reduction below
        const f2 uv = pixel_uv<KIND>(c, (int)(idx % width), (int)(idx / width), width, height);
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
            g[4] = go.x; g[5] = go.y; g[6] = go.z;
            g[7] = dt * go.x; g[8] = dt * go.y; g[9] = dt * go.z;
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
            g[0] = d_w2; g[1] = d_xyz2.x; g[2] = d_xyz2.y; g[3] = d_xyz2.z;
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
            g[10] = d_w.x; g[11] = d_w.y; g[12] = d_w.z;
            // dt = trigger_time + uv . rolling_time - pose_time
            g[13] = d_dt * uv.x; g[14] = d_dt * uv.y; g[15] = d_dt; g[16] = -d_dt;
        }
        const f3 dr = normalized ? (dn - dot(n, dn) * n) * il : dn;
        if constexpr (KIND == XSG_CAM_PINHOLE) {  // perspective.cu:19-33
            const float ifx = 1.0f / c.i0, ify = 1.0f / c.i1;
            g[17] = -dr.x * (uv.x - c.i2) * ifx * ifx;
            g[18] = -dr.y * (uv.y - c.i3) * ify * ify;
            g[19] = -dr.x * ifx;
            g[20] = -dr.y * ify;
        }  // the spherical and lidar models carry no intrinsics gradient (base_camera_impl.h:19-22)
    }
    block_partials<kCamGrad>(g, part);
}

// pixel_time[_delta][_from_uv]_bwd_kernel (time_kernels.h:123-330): partial sums of g u, g v and g;
// with uv given, d_uv = g rolling_time
template <int KIND>
__global__ __launch_bounds__(kBlock) void pixel_time_bwd_kernel(const float* __restrict__ pack, int width,
                                                                int height, const float2* __restrict__ uv_in,
                                                                int64_t n, const float* __restrict__ grad,
                                                                float2* __restrict__ d_uv, float* __restrict__ part) {
    const int64_t idx = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const Camera c = load_camera(pack, KIND);
    float g[3] = {0.f, 0.f, 0.f};
    if (idx < n) {
        f2 uv;
        if (uv_in) {
            uv = mk2(uv_in[idx].x, uv_in[idx].y);
        } else {
            uv = pixel_uv<KIND>(c, (int)(idx % width), (int)(idx / width), width, height);
        }
        const float gr = grad[idx];
        if (d_uv) d_uv[idx] = make_float2(gr * c.roll_u, gr * c.roll_v);
        g[0] = gr * uv.x; g[1] = gr * uv.y; g[2] = gr;
    }
    block_partials<3>(g, part);
}

// one workgroup: out[k] = sum over blocks of part[b][k] for the nv partial values, placed at the pack
// positions: rays (nv = kCamGrad) at 0..20; times (nv = 3) at rolling_time, trigger_time and, for
// the delta variants, -trigger at pose_time; every other pack element 0.
__global__ __launch_bounds__(kBlock) void grad_final_kernel(const float* __restrict__ part, int nb, int nv, int delta,
                                                            int pack_elems, float* __restrict__ out) {
    const int wave = threadIdx.x >> 6, lane = __lane_id();
    for (int e = wave; e < pack_elems; e += kBlock / 64) {
        const int k = (nv == kCamGrad) ? e : (e == 13 ? 0 : e == 14 ? 1 : (e == 15 || (e == 16 && delta)) ? 2 : -1);
        float t = 0.f;
        if (k >= 0 && k < nv)
            for (int b = lane; b < nb; b += 64) t += part[(int64_t)b * nv + k];
        t = wave_sum(t);
        if (lane == 0) out[e] = (nv != kCamGrad && delta && e == 16) ? -t : t;
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
    if (n == 0) return XSG_OK;
    if (!means || !scales || !quats || !flags || !radii || !means2d || !depths)
        return xsg_fail(XSG_ERR_INVALID, "xsg_ut_project: null tensor");
    if (phm && kind == XSG_CAM_PINHOLE)
        return xsg_fail(XSG_ERR_UNSUPPORTED, "projection_utgs_phm needs a spherical or lidar camera");
    const ProjParams pp{residual_thr, max_residual, max_margin};
    const UtWeights ut = ut_weights(ut_alpha, ut_beta, ut_kappa);
    const f2 img = mk2(width, height);
    const dim3 grid(xsg_blocks(n, kBlock)), block(kBlock);
    auto q4 = reinterpret_cast<const float4*>(quats);
    auto r2 = reinterpret_cast<float2*>(radii);
    auto m2 = reinterpret_cast<float2*>(means2d);
#define XSG_UT_ARGS n, pack, pp, ut, img, means, velocity, scales, q4, opacity, flags, r2, m2, depths
    switch (kind) {
        case XSG_CAM_PINHOLE:
            ut_project_kernel<XSG_CAM_PINHOLE><<<grid, block, 0, (hipStream_t)stream>>>(XSG_UT_ARGS);
            break;
        case XSG_CAM_SPHERICAL:
            if (phm) ut_project_phm_kernel<XSG_CAM_SPHERICAL><<<grid, block, 0, (hipStream_t)stream>>>(XSG_UT_ARGS);
            else ut_project_kernel<XSG_CAM_SPHERICAL><<<grid, block, 0, (hipStream_t)stream>>>(XSG_UT_ARGS);
            break;
        case XSG_CAM_LIDAR:
            if (phm) ut_project_phm_kernel<XSG_CAM_LIDAR><<<grid, block, 0, (hipStream_t)stream>>>(XSG_UT_ARGS);
            else ut_project_kernel<XSG_CAM_LIDAR><<<grid, block, 0, (hipStream_t)stream>>>(XSG_UT_ARGS);
            break;
        default: return xsg_fail(XSG_ERR_INVALID, "unknown camera kind %d", kind);
    }
#undef XSG_UT_ARGS
    XSG_TRY_LAUNCH("ut_project");
    return XSG_OK;
}

extern "C" int xsg_project_points(int kind, const float* pack, int64_t n, const float* points,
                                  const float* velocity, float residual_thr, float max_residual,
                                  float max_margin, int mode, int no_jacobian, float* uvdt,
                                  uint8_t* mask, xsg_stream_t stream) {
    if (n < 0 || !pack) return xsg_fail(XSG_ERR_INVALID, "xsg_project_points: bad arguments");
    if (n == 0) return XSG_OK;
    const ProjParams pp{residual_thr, max_residual, max_margin};
    const dim3 grid(xsg_blocks(n, kBlock)), block(kBlock);
    auto u4 = reinterpret_cast<float4*>(uvdt);
    switch (kind) {
        case XSG_CAM_PINHOLE:
            project_points_kernel<XSG_CAM_PINHOLE><<<grid, block, 0, (hipStream_t)stream>>>(
                n, pack, pp, mode, no_jacobian, points, velocity, u4, mask);
            break;
        case XSG_CAM_SPHERICAL:
            project_points_kernel<XSG_CAM_SPHERICAL><<<grid, block, 0, (hipStream_t)stream>>>(
                n, pack, pp, mode, no_jacobian, points, velocity, u4, mask);
            break;
        case XSG_CAM_LIDAR:
            project_points_kernel<XSG_CAM_LIDAR><<<grid, block, 0, (hipStream_t)stream>>>(
                n, pack, pp, mode, no_jacobian, points, velocity, u4, mask);
            break;
        default: return xsg_fail(XSG_ERR_INVALID, "unknown camera kind %d", kind);
    }
    XSG_TRY_LAUNCH("project_points");
    return XSG_OK;
}

extern "C" int xsg_camera_rays(int kind, const float* pack, int width, int height, int world_space,
                               int normalized, float* ray_o, float* ray_d, uint8_t* valid,
                               xsg_stream_t stream) {
    if (width < 0 || height < 0 || !pack || !ray_d)
        return xsg_fail(XSG_ERR_INVALID, "xsg_camera_rays: bad arguments");
    const int64_t n = (int64_t)width * height;
    if (n == 0) return XSG_OK;
    const dim3 grid(xsg_blocks(n, kBlock)), block(kBlock);
    switch (kind) {
        case XSG_CAM_PINHOLE:
            camera_rays_kernel<XSG_CAM_PINHOLE><<<grid, block, 0, (hipStream_t)stream>>>(
                pack, width, height, world_space, normalized, ray_o, ray_d, valid);
            break;
        case XSG_CAM_SPHERICAL:
            camera_rays_kernel<XSG_CAM_SPHERICAL><<<grid, block, 0, (hipStream_t)stream>>>(
                pack, width, height, world_space, normalized, ray_o, ray_d, valid);
            break;
        case XSG_CAM_LIDAR:
            camera_rays_kernel<XSG_CAM_LIDAR><<<grid, block, 0, (hipStream_t)stream>>>(
                pack, width, height, world_space, normalized, ray_o, ray_d, valid);
            break;
        default: return xsg_fail(XSG_ERR_INVALID, "unknown camera kind %d", kind);
    }
    XSG_TRY_LAUNCH("camera_rays");
    return XSG_OK;
}

extern "C" int xsg_pixel_time(int kind, const float* pack, int width, int height, const float* uv,
                              int64_t n_uv, int delta, float* out, xsg_stream_t stream) {
    const int64_t n = uv ? n_uv : (int64_t)width * height;
    if (n < 0 || !pack || !out) return xsg_fail(XSG_ERR_INVALID, "xsg_pixel_time: bad arguments");
    if (n == 0) return XSG_OK;
    const dim3 grid(xsg_blocks(n, kBlock)), block(kBlock);
    auto uv2 = reinterpret_cast<const float2*>(uv);
    switch (kind) {
        case XSG_CAM_PINHOLE:
            pixel_time_kernel<XSG_CAM_PINHOLE><<<grid, block, 0, (hipStream_t)stream>>>(pack, width, height, uv2, n, delta, out);
            break;
        case XSG_CAM_SPHERICAL:
            pixel_time_kernel<XSG_CAM_SPHERICAL><<<grid, block, 0, (hipStream_t)stream>>>(pack, width, height, uv2, n, delta, out);
            break;
        case XSG_CAM_LIDAR:
            pixel_time_kernel<XSG_CAM_LIDAR><<<grid, block, 0, (hipStream_t)stream>>>(pack, width, height, uv2, n, delta, out);
            break;
        default: return xsg_fail(XSG_ERR_INVALID, "unknown camera kind %d", kind);
    }
    XSG_TRY_LAUNCH("pixel_time");
    return XSG_OK;
}

extern "C" size_t xsg_camera_rays_bwd_workspace_bytes(int width, int height) {
    const int64_t n = (int64_t)(width > 0 ? width : 0) * (height > 0 ? height : 0);
    return sizeof(float) * (size_t)kCamGrad * xsg_blocks(n > 0 ? n : 1, kBlock);
}

extern "C" int xsg_camera_rays_bwd(int kind, const float* pack, int width, int height, int world_space,
                                   int normalized, const float* d_ray_o, const float* d_ray_d, float* grad_pack,
                                   void* workspace, xsg_stream_t stream) {
    const int pe = xsg_camera_pack_elements(kind);
    if (pe <= 0) return xsg_fail(XSG_ERR_INVALID, "unknown camera kind %d", kind);
    if (width < 0 || height < 0) return xsg_fail(XSG_ERR_INVALID, "camera_rays_bwd: negative size");
    if (!pack || !grad_pack || !workspace || (!d_ray_d && (int64_t)width * height > 0))
        return xsg_fail(XSG_ERR_INVALID, "camera_rays_bwd: null pointer");
    const int64_t n = (int64_t)width * height;
    const unsigned nb = xsg_blocks(n > 0 ? n : 1, kBlock);
    float* part = (float*)workspace;
    const hipStream_t s = (hipStream_t)stream;
    switch (kind) {
        case XSG_CAM_PINHOLE:
            camera_rays_bwd_kernel<XSG_CAM_PINHOLE><<<nb, kBlock, 0, s>>>(pack, width, height, world_space,
                                                                          normalized, d_ray_o, d_ray_d, part);
            break;
        case XSG_CAM_SPHERICAL:
            camera_rays_bwd_kernel<XSG_CAM_SPHERICAL><<<nb, kBlock, 0, s>>>(pack, width, height, world_space,
                                                                            normalized, d_ray_o, d_ray_d, part);
            break;
        default:
            camera_rays_bwd_kernel<XSG_CAM_LIDAR><<<nb, kBlock, 0, s>>>(pack, width, height, world_space,
                                                                        normalized, d_ray_o, d_ray_d, part);
            break;
    }
    grad_final_kernel<<<1, kBlock, 0, s>>>(part, (int)nb, kCamGrad, 0, pe, grad_pack);
    XSG_TRY_LAUNCH("camera_rays_bwd");
    return XSG_OK;
}

extern "C" size_t xsg_pixel_time_bwd_workspace_bytes(int64_t n) {
    return sizeof(float) * 3 * (size_t)xsg_blocks(n > 0 ? n : 1, kBlock);
}

extern "C" int xsg_pixel_time_bwd(int kind, const float* pack, int width, int height, const float* uv,
                                  int64_t n_uv, int delta, const float* grad, float* grad_pack, float* d_uv,
                                  void* workspace, xsg_stream_t stream) {
    const int pe = xsg_camera_pack_elements(kind);
    if (pe <= 0) return xsg_fail(XSG_ERR_INVALID, "unknown camera kind %d", kind);
    const int64_t n = uv ? n_uv : (int64_t)width * height;
    if (n < 0 || (!uv && (width < 0 || height < 0))) return xsg_fail(XSG_ERR_INVALID, "pixel_time_bwd: bad size");
    if (!pack || !grad_pack || !workspace || (n > 0 && !grad))
        return xsg_fail(XSG_ERR_INVALID, "pixel_time_bwd: null pointer");
    const unsigned nb = xsg_blocks(n > 0 ? n : 1, kBlock);
    float* part = (float*)workspace;
    const hipStream_t s = (hipStream_t)stream;
    const float2* uv2 = (const float2*)uv;
    float2* duv2 = uv ? (float2*)d_uv : nullptr;
    switch (kind) {
        case XSG_CAM_PINHOLE:
            pixel_time_bwd_kernel<XSG_CAM_PINHOLE><<<nb, kBlock, 0, s>>>(pack, width, height, uv2, n, grad, duv2, part);
            break;
        case XSG_CAM_SPHERICAL:
            pixel_time_bwd_kernel<XSG_CAM_SPHERICAL><<<nb, kBlock, 0, s>>>(pack, width, height, uv2, n, grad, duv2,
                                                                           part);
            break;
        default:
            pixel_time_bwd_kernel<XSG_CAM_LIDAR><<<nb, kBlock, 0, s>>>(pack, width, height, uv2, n, grad, duv2, part);
            break;
    }
    grad_final_kernel<<<1, kBlock, 0, s>>>(part, (int)nb, 3, delta ? 1 : 0, pe, grad_pack);
    XSG_TRY_LAUNCH("pixel_time_bwd");
    return XSG_OK;
}
