// Shared device helpers for the xsimgs_amd HIP kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <type_traits>

#include "../../include/xsimgs_amd.h"

#define XSG_DEV __device__ __forceinline__
#define XSG_HD __host__ __device__ __forceinline__

// Error reporting shared by every C-ABI entry point (defined in capi.hip).
int xsg_fail(int code, const char* fmt, ...);

// Workspaces are 256-byte aligned (as hipMalloc and torch's allocator return them): the kernels'
// vector accesses into them rely on it.
constexpr uintptr_t kWorkspaceAlign = 256;
inline int xsg_check_workspace(const void* ws, const char* who) {
    if (((uintptr_t)ws & (kWorkspaceAlign - 1)) != 0)
        return xsg_fail(XSG_ERR_INVALID, "%s: workspace must be %d-byte aligned", who, (int)kWorkspaceAlign);
    return XSG_OK;
}

// Host-side dispatch over the camera models: calls f(std::integral_constant<int, KIND>{}).
template <typename F>
int xsg_with_camera_kind(int kind, F&& f) {
    switch (kind) {
        case XSG_CAM_PINHOLE: f(std::integral_constant<int, XSG_CAM_PINHOLE>{}); return XSG_OK;
        case XSG_CAM_SPHERICAL: f(std::integral_constant<int, XSG_CAM_SPHERICAL>{}); return XSG_OK;
        case XSG_CAM_LIDAR: f(std::integral_constant<int, XSG_CAM_LIDAR>{}); return XSG_OK;
        case XSG_CAM_DISTORTED: f(std::integral_constant<int, XSG_CAM_DISTORTED>{}); return XSG_OK;
        case XSG_CAM_FISHEYE: f(std::integral_constant<int, XSG_CAM_FISHEYE>{}); return XSG_OK;
        default: return xsg_fail(XSG_ERR_INVALID, "unknown camera kind %d", kind);
    }
}
int xsg_launch_status(const char* what);

#define XSG_TRY_LAUNCH(what)                                  \
    do {                                                      \
        int _rc = xsg_launch_status(what);                    \
        if (_rc != XSG_OK) return _rc;                        \
    } while (0)

static inline unsigned xsg_blocks(long n, int block) { return (unsigned)((n + block - 1) / block); }

// --------------------------------------------------------------------------
// small vector types (plain structs: no reliance on HIP vector operators)
// --------------------------------------------------------------------------
struct f2 { float x, y; };
struct f3 { float x, y, z; };

XSG_HD f2 mk2(float x, float y) { return f2{x, y}; }
XSG_HD f3 mk3(float x, float y, float z) { return f3{x, y, z}; }
XSG_HD f3 operator+(f3 a, f3 b) { return mk3(a.x + b.x, a.y + b.y, a.z + b.z); }
XSG_HD f3 operator-(f3 a, f3 b) { return mk3(a.x - b.x, a.y - b.y, a.z - b.z); }
XSG_HD f3 operator-(f3 a) { return mk3(-a.x, -a.y, -a.z); }
XSG_HD f3 operator*(f3 a, float s) { return mk3(a.x * s, a.y * s, a.z * s); }
XSG_HD f3 operator*(float s, f3 a) { return mk3(a.x * s, a.y * s, a.z * s); }
XSG_HD float dot(f3 a, f3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
XSG_HD f3 cross(f3 a, f3 b) {
    return mk3(a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x);
}
XSG_DEV f3 ld3(const float* p) { return mk3(p[0], p[1], p[2]); }
XSG_DEV void st3(float* p, f3 v) { p[0] = v.x; p[1] = v.y; p[2] = v.z; }

// --------------------------------------------------------------------------
// Camera pack. Flat float layout (elements):
//   [0..3] q0 (w,x,y,z) camera-to-world   [4..6] t0   [7..9] v   [10..12] w
//   [13..14] rolling duration (u, v)  [15] trigger time  [16] pose time
//   [17..20] impl: pinhole, distorted, fisheye f.x f.y c.x c.y |
//            spherical, lidar phi_min phi_range theta_min theta_range
//   [21..22] lidar: device address of beam_v (two 32-bit words, low first)
//   [21..28] distorted: k1 k2 p1 p2 k3 k4 k5 k6, [29] max_radius^2
//   [21..24] fisheye: k1 k2 k3 k4
// Mirrors Camera<Impl> (reference include/cameras/camera.h:67-79) field by field.
// --------------------------------------------------------------------------
struct Camera {
    float qw; f3 qv;
    f3 t0, v, w;
    float roll_u, roll_v;
    float trigger_time, pose_time;
    float i0, i1, i2, i3;
    const float* beam_v;
    float k[8];   // distortion coefficients (distorted: k1 k2 p1 p2 k3 k4 k5 k6; fisheye: k1..k4)
    float max_r2; // distorted: largest squared camera-space radius that projects
};

XSG_DEV Camera load_camera(const float* __restrict__ p, int kind) {
    Camera c;
    c.qw = p[0]; c.qv = mk3(p[1], p[2], p[3]);
    c.t0 = mk3(p[4], p[5], p[6]);
    c.v = mk3(p[7], p[8], p[9]);
    c.w = mk3(p[10], p[11], p[12]);
    c.roll_u = p[13]; c.roll_v = p[14];
    c.trigger_time = p[15]; c.pose_time = p[16];
    c.i0 = p[17]; c.i1 = p[18]; c.i2 = p[19]; c.i3 = p[20];
    c.beam_v = nullptr;
#pragma unroll
    for (int i = 0; i < 8; ++i) c.k[i] = 0.f;
    c.max_r2 = 0.f;
    if (kind == XSG_CAM_LIDAR) {
        const uint32_t lo = __float_as_uint(p[21]), hi = __float_as_uint(p[22]);
        c.beam_v = reinterpret_cast<const float*>(((uint64_t)hi << 32) | lo);
    } else if (kind == XSG_CAM_DISTORTED) {
#pragma unroll
        for (int i = 0; i < 8; ++i) c.k[i] = p[21 + i];
        c.max_r2 = p[29];
    } else if (kind == XSG_CAM_FISHEYE) {
#pragma unroll
        for (int i = 0; i < 4; ++i) c.k[i] = p[21 + i];
    }
    return c;
}

// --------------------------------------------------------------------------
// Distorted perspective (OpenCV rational radial + tangential) and OpenCV fisheye models
// (reference csrc/cameras/distorted_perspective.cu, fisheye_opencv.cu, include/cameras/distortion.h)
// --------------------------------------------------------------------------
constexpr float kDistMinDet = 1e-3f;  // distorted_perspective.cu:9

// uv_distortion (distortion.h:8-30): radial scale and tangential offset at a camera-space uv
XSG_DEV void uv_distortion(const Camera& c, float u, float v, float& scale, float& du, float& dv) {
    const float uu = u * u, vv = v * v;
    const float r2 = uu + vv;
    const float num = 1.0f + r2 * (c.k[0] + r2 * (c.k[1] + r2 * c.k[4]));
    const float den = 1.0f + r2 * (c.k[5] + r2 * (c.k[6] + r2 * c.k[7]));
    scale = num / den;
    const float uv2 = 2.0f * u * v;
    du = c.k[2] * uv2 + c.k[3] * (r2 + 2.0f * uu);
    dv = c.k[2] * (r2 + 2.0f * vv) + c.k[3] * uv2;
}

// DistortionState (distorted_perspective.cu:11-36, 44-78): distortion at uv and its symmetric Jacobian
struct DistState { float scale, denom, dx, dy, juu, juv, jvv; };

XSG_DEV DistState distortion_state(const Camera& c, float u, float v) {
    const float k1 = c.k[0], k2 = c.k[1], p1 = c.k[2], p2 = c.k[3];
    const float k3 = c.k[4], k4 = c.k[5], k5 = c.k[6], k6 = c.k[7];
    const float r2 = u * u + v * v;
    const float num = 1.0f + r2 * (k1 + r2 * (k2 + r2 * k3));
    const float den = 1.0f + r2 * (k4 + r2 * (k5 + r2 * k6));
    const float scale = num / den;
    const float d_num = k1 + r2 * (2.0f * k2 + 3.0f * k3 * r2);
    const float d_den = k4 + r2 * (2.0f * k5 + 3.0f * k6 * r2);
    const float d_scale = (d_num * den - num * d_den) / (den * den);
    DistState s;
    s.scale = scale;
    s.denom = den;
    s.dx = 2.0f * p1 * u * v + p2 * (r2 + 2.0f * u * u);
    s.dy = p1 * (r2 + 2.0f * v * v) + 2.0f * p2 * u * v;
    s.juu = scale + 2.0f * u * u * d_scale + 2.0f * p1 * v + 6.0f * p2 * u;
    s.juv = 2.0f * u * v * d_scale + 2.0f * p1 * u + 2.0f * p2 * v;
    s.jvv = scale + 2.0f * v * v * d_scale + 6.0f * p1 * v + 2.0f * p2 * u;
    return s;
}

// undistort_uv (distorted_perspective.cu:80-98): five Newton steps on uv * scale + delta = ud, a
// fixed-point step where the Jacobian is nearly singular; `st` keeps the last step's state (taken
// before that step's update)
XSG_DEV f2 undistort_uv(const Camera& c, f2 ud, DistState& st) {
    f2 uv = ud;
#pragma unroll
    for (int j = 0; j < 5; ++j) {
        st = distortion_state(c, uv.x, uv.y);
        const float rx = uv.x * st.scale + st.dx - ud.x;
        const float ry = uv.y * st.scale + st.dy - ud.y;
        const float det = st.juu * st.jvv - st.juv * st.juv;
        if (fabsf(det) > kDistMinDet) {
            uv.x -= (st.jvv * rx - st.juv * ry) / det;
            uv.y -= (st.juu * ry - st.juv * rx) / det;
        } else {
            uv.x = (ud.x - st.dx) / st.scale;
            uv.y = (ud.y - st.dy) / st.scale;
        }
    }
    return uv;
}

// Kannala-Brandt polynomial theta_d(theta) and its derivative (fisheye_opencv.cu:14-32)
XSG_DEV float fisheye_distortion(const Camera& c, float th) {
    const float t2 = th * th;
    float d = t2 * c.k[3] + c.k[2];
    d = t2 * d + c.k[1];
    d = t2 * d + c.k[0];
    d = t2 * d + 1.0f;
    return th * d;
}

XSG_DEV float fisheye_distortion_deriv(const Camera& c, float th) {
    const float t2 = th * th;
    float d = t2 * 9.0f * c.k[3] + 7.0f * c.k[2];
    d = t2 * d + 5.0f * c.k[1];
    d = t2 * d + 3.0f * c.k[0];
    d = t2 * d + 1.0f;
    return d;
}

// solve_theta (fisheye_opencv.cu:34-46): at most 20 Newton steps, derivative clamped at 0.1,
// theta kept in [0, pi]
XSG_DEV float fisheye_solve_theta(const Camera& c, float delta, float& residual) {
    float th = delta;
    residual = 0.0f;
    for (int i = 0; i < 20; ++i) {
        residual = fisheye_distortion(c, th) - delta;
        th -= residual / fmaxf(fisheye_distortion_deriv(c, th), 0.1f);
        th = fminf(fmaxf(th, 0.0f), float(M_PI));
        if (fabsf(residual) < 1e-6f) break;
    }
    return th;
}

XSG_DEV float pixel_time(const Camera& c, float u, float v) {  // camera.h:89-91
    return c.trigger_time + (u * c.roll_u + v * c.roll_v);
}

XSG_DEV float u_pose_of(const Camera& c) {  // spherical.h:113-114
    return (fabsf(c.roll_u) > 0.0f) ? (c.pose_time - c.trigger_time) / c.roll_u : 0.5f;
}

// --------------------------------------------------------------------------
// Rolling-shutter projection (reference include/cameras/projection_kernels.h)
// --------------------------------------------------------------------------
XSG_DEV void jac_quat_from_axis_angle(f3 w, float t, float& qw, f3& qxyz, float& dqw, f3& dqxyz) {
    // projection_kernels.h:12-36. sin/cos of an exactly-zero angle are 0 and 1, so the
    // common t == 0 / w == 0 case skips sincosf with bit-identical results.
    const float w_norm = sqrtf(dot(w, w));
    const float theta = w_norm * fabsf(t);
    float s = 0.0f, c = 1.0f;
    if (theta != 0.0f) sincosf(0.5f * theta, &s, &c);
    const float scale = (theta < 1e-2f) ? 0.5f - theta * theta * (1.0f / 48.0f) : s / theta;
    qw = c;
    qxyz = (w * scale) * t;
    dqw = -0.5f * copysignf(1.0f, t) * s * w_norm;
    dqxyz = w * (0.5f * c);
}

XSG_DEV f3 quat_apply(float w, f3 xyz, f3 p) {  // projection_kernels.h:67-71
    const f3 uv = cross(xyz, p);
    const f3 uuv = cross(xyz, uv);
    return p + 2.0f * (w * uv + uuv);
}

XSG_DEV void world_to_camera_jac(const Camera& c, f3 point, f3 pvel, float time, f3& res, f3& dres) {
    // projection_kernels.h:74-113
    float w1, dw1; f3 xyz1, dxyz1;
    jac_quat_from_axis_angle(c.w, time, w1, xyz1, dw1, dxyz1);
    const float w2 = c.qw; const f3 xyz2 = c.qv;
    const float w = w1 * w2 - dot(xyz1, xyz2);
    f3 xyz = w2 * xyz1 + w1 * xyz2 + cross(xyz1, xyz2);
    const float dw = dw1 * w2 - dot(dxyz1, xyz2);
    f3 dxyz = dw1 * xyz2 + w2 * dxyz1 + cross(dxyz1, xyz2);
    xyz = -xyz; dxyz = -dxyz;
    const f3 vdiff = pvel - c.v;
    const f3 p = point - c.t0 + vdiff * time;
    const f3 uv = cross(xyz, p);
    const f3 uuv = cross(xyz, uv);
    res = p + 2.0f * (w * uv + uuv);
    const f3 duv = cross(dxyz, p);
    const f3 dp = 2.0f * (dw * uv + w * duv + cross(dxyz, uv) + cross(xyz, duv));
    dres = dp + quat_apply(w, xyz, vdiff);
}

// The phase unwrapping of SphericalCamera's angles_to_uv (csrc/cameras/spherical.h:109-125): u from the
// azimuth, shifted by one turn towards the pose's side in the negative / positive modes. The pose's u
// and the turn depend on the camera only.
struct PhaseUnwrap { float u_pose, u_offset; bool forward; };

XSG_DEV PhaseUnwrap phase_unwrap(const Camera& c) {
    return {u_pose_of(c), 2.0f * float(M_PI) / fabsf(c.i1), c.roll_u > 0};
}

XSG_DEV float unwrap_u(const PhaseUnwrap& w, int mode, float u) {
    if (w.forward) {
        if ((mode == XSG_MODE_NEGATIVE) && (u > w.u_pose)) u = u - w.u_offset;
        if ((mode == XSG_MODE_POSITIVE) && (u < w.u_pose)) u = u + w.u_offset;
    } else {
        if ((mode == XSG_MODE_NEGATIVE) && (u < w.u_pose)) u = u + w.u_offset;
        if ((mode == XSG_MODE_POSITIVE) && (u > w.u_pose)) u = u - w.u_offset;
    }
    return u;
}

// angles_to_uv (spherical.h:109-125)
XSG_DEV f2 angles_to_uv(const Camera& c, int mode, float phi, float theta) {
    return mk2(unwrap_u(phase_unwrap(c), mode, (phi - c.i0) / c.i1), (theta - c.i2) / c.i3);
}

// Camera models with a projection Jacobian take Newton steps on the pixel time; the others the
// fixed-point step (projection_kernels.h:116-198, selected at :224-236)
template <int KIND>
constexpr bool has_projection_jacobian() {
    return KIND == XSG_CAM_PINHOLE || KIND == XSG_CAM_SPHERICAL || KIND == XSG_CAM_LIDAR;
}

template <int KIND>
XSG_DEV f3 point_to_uvd(const Camera& c, int mode, f3 p) {
    if constexpr (KIND == XSG_CAM_PINHOLE) {  // perspective.cu:36-42
        return mk3(p.x * c.i0 / p.z + c.i2, p.y * c.i1 / p.z + c.i3, p.z);
    } else if constexpr (KIND == XSG_CAM_DISTORTED) {  // distorted_perspective.cu:190-197
        const float x = p.x / p.z, y = p.y / p.z;
        float scale, du, dv;
        uv_distortion(c, x, y, scale, du, dv);
        const float r2 = x * x + y * y;
        return mk3((x * scale + du) * c.i0 + c.i2, (y * scale + dv) * c.i1 + c.i3, (r2 <= c.max_r2) ? p.z : 0.0f);
    } else if constexpr (KIND == XSG_CAM_FISHEYE) {  // fisheye_opencv.cu:138-148
        const float norm = fmaxf(1e-6f, hypotf(p.x, p.y));
        const float th = atan2f(norm, p.z);
        const bool valid = fisheye_distortion_deriv(c, th) > 0.0f;
        const float delta = fisheye_distortion(c, th) / norm;
        const float depth = (valid && (delta > 0.0f)) ? sqrtf(dot(p, p)) : 0.0f;
        return mk3(c.i0 * delta * p.x + c.i2, c.i1 * delta * p.y + c.i3, depth);
    } else {  // spherical.h:133-142
        const float x2y2 = p.x * p.x + p.y * p.y;
        const float r = sqrtf(x2y2 + p.z * p.z);
        const float phi = atan2f(-p.x, -p.y) + float(M_PI);
        const float theta = asinf(p.z / r);
        const f2 uv = angles_to_uv(c, mode, phi, theta);
        return mk3(uv.x, uv.y, r);
    }
}

template <int KIND>
XSG_DEV void point_to_uvd_jacob(const Camera& c, int mode, f3 p, f3 dp, f3& uvd, f2& du_dv) {
    if constexpr (KIND == XSG_CAM_PINHOLE) {  // perspective.cu:44-52
        uvd = point_to_uvd<KIND>(c, mode, p);
        du_dv.x = c.i0 * (dp.x - uvd.x * dp.z) / uvd.z;
        du_dv.y = c.i1 * (dp.y - uvd.y * dp.z) / uvd.z;
    } else {  // spherical.h:133-153
        const float x2y2 = p.x * p.x + p.y * p.y;
        const float r = sqrtf(x2y2 + p.z * p.z);
        const float phi = atan2f(-p.x, -p.y) + float(M_PI);
        const float theta = asinf(p.z / r);
        const f2 uv = angles_to_uv(c, mode, phi, theta);
        uvd = mk3(uv.x, uv.y, r);
        const float x2y2_sqrt = sqrtf(x2y2);
        const float r2 = r * r;
        const float mul = p.z / (r2 * x2y2_sqrt);
        du_dv.x = ((-p.x * dp.y + p.y * dp.x) / x2y2) / c.i1;
        du_dv.y = ((x2y2_sqrt * dp.z) / r2 - mul * (p.x * dp.x + p.y * dp.y)) / c.i3;
    }
}

struct ProjParams {
    float thr, max_res, margin;
};

// camera_projection: projection_kernels.h:201-256 (Newton solve of the pixel time).
// `is_static` (no camera motion, no point velocity) lets the camera-space point be computed
// once: the pose is then independent of the time, so every iteration sees the same point.
template <int KIND>
XSG_DEV void camera_projection(const Camera& c, f3 pw, f3 pv, const ProjParams& pp, int mode,
                               bool is_static, float4& uvdt, bool& valid) {
    f3 uvd = mk3(0.f, 0.f, 0.f);
    float p_time = 0.0f;
    if (mode == XSG_MODE_NEGATIVE) p_time = -fabsf(c.roll_u) * 0.5f;
    else if (mode == XSG_MODE_POSITIVE) p_time = fabsf(c.roll_u) * 0.5f;
    float residual = 0.0f;
    f3 pc = mk3(0.f, 0.f, 0.f), jpc = mk3(0.f, 0.f, 0.f);
    f2 du_dv = mk2(0.f, 0.f);
    constexpr bool newton = has_projection_jacobian<KIND>();
    if (is_static) {
        // static pose: world_to_camera(p, t) == quat_apply(q0.w, -q0.xyz, p - t0) for every t
        f3 r, dr;
        world_to_camera_jac(c, pw, pv, p_time, r, dr);
        pc = r; jpc = dr;
        if constexpr (newton) point_to_uvd_jacob<KIND>(c, mode, pc, jpc, uvd, du_dv);
        else uvd = point_to_uvd<KIND>(c, mode, pc);
    }
#pragma unroll 1
    for (int i = 0; i < 5; ++i) {
        if (!is_static) {
            world_to_camera_jac(c, pw, pv, p_time, pc, jpc);
            if constexpr (newton) point_to_uvd_jacob<KIND>(c, mode, pc, jpc, uvd, du_dv);
            else uvd = point_to_uvd<KIND>(c, mode, pc);
        }
        const float assumed = c.pose_time + p_time;
        const float real_time = pixel_time(c, uvd.x, uvd.y);
        residual = assumed - real_time;
        if constexpr (newton) {
            const float d_res = 1.0f - (du_dv.x * c.roll_u + du_dv.y * c.roll_v);
            p_time -= residual / d_res;
        } else {
            p_time -= residual;  // camera_projection_iteration (projection_kernels.h:177-198)
        }
        if ((uvd.z <= 0.0f) || (uvd.x < -pp.margin) || (uvd.x > 1.0f + pp.margin) ||
            (uvd.y < -pp.margin) || (uvd.y > 1.0f + pp.margin)) {
            valid = false;
            uvdt = make_float4(0.f, 0.f, 0.f, 0.f);
            return;
        }
        if (fabsf(residual) < pp.thr) break;
    }
    uvdt = make_float4(uvd.x, uvd.y, uvd.z, p_time);
    valid = valid && (fabsf(residual) < pp.max_res) && (uvd.z > 0.0f);
}

XSG_DEV bool camera_is_static(const Camera& c, bool has_vel) {
    return !has_vel && c.w.x == 0.f && c.w.y == 0.f && c.w.z == 0.f && c.v.x == 0.f &&
           c.v.y == 0.f && c.v.z == 0.f;
}

// unscented_transform_deltas (ut_kernels.h:38-49): columns of R(q) scaled by s_i * sqrt(3+lambda),
// from the normalised quaternion (w, x, y, z).
XSG_DEV void ut_deltas(float sqrt_dl, float4 q, f3 s, f3 d[3]) {
    float w = q.x, x = q.y, y = q.z, z = q.w;
    const float inv = 1.0f / sqrtf(w * w + x * x + y * y + z * z);
    w *= inv; x *= inv; y *= inv; z *= inv;
    d[0] = mk3(1.f - 2.f * (y * y + z * z), 2.f * (x * y + w * z), 2.f * (x * z - w * y)) * (s.x * sqrt_dl);
    d[1] = mk3(2.f * (x * y - w * z), 1.f - 2.f * (x * x + z * z), 2.f * (y * z + w * x)) * (s.y * sqrt_dl);
    d[2] = mk3(2.f * (x * z + w * y), 2.f * (y * z - w * x), 1.f - 2.f * (x * x + y * y)) * (s.z * sqrt_dl);
}

// ut_deltas with the quaternion's inverse norm as one reciprocal square root (1 ulp)
XSG_DEV void ut_deltas_rsq(float sqrt_dl, float4 q, f3 s, f3 d[3]) {
    float w = q.x, x = q.y, y = q.z, z = q.w;
    const float inv = __builtin_amdgcn_rsqf(w * w + x * x + y * y + z * z);
    w *= inv; x *= inv; y *= inv; z *= inv;
    d[0] = mk3(1.f - 2.f * (y * y + z * z), 2.f * (x * y + w * z), 2.f * (x * z - w * y)) * (s.x * sqrt_dl);
    d[1] = mk3(2.f * (x * y - w * z), 1.f - 2.f * (x * x + z * z), 2.f * (y * z + w * x)) * (s.y * sqrt_dl);
    d[2] = mk3(2.f * (x * z + w * y), 2.f * (y * z - w * x), 1.f - 2.f * (x * x + y * y)) * (s.z * sqrt_dl);
}

struct UtWeights { float wm0, wc0, wi, sqrt_dl; };

// A camera whose pose does not move maps world to camera space by one linear map: quat_apply with
// the conjugate of q0 (world_to_camera_jac at any time), p -> p + 2 (w (u x p) + u x (u x p)) with
// u = -q0.xyz, i.e. M = I + 2 w [u]x + 2 (u u^T - |u|^2 I) (exact for any quaternion).
struct Mat3 { f3 r0, r1, r2; };

XSG_DEV Mat3 static_world_to_camera(const Camera& c) {
    const float w = c.qw, x = -c.qv.x, y = -c.qv.y, z = -c.qv.z;
    Mat3 m;
    m.r0 = mk3(1.f - 2.f * (y * y + z * z), 2.f * (x * y - w * z), 2.f * (x * z + w * y));
    m.r1 = mk3(2.f * (x * y + w * z), 1.f - 2.f * (x * x + z * z), 2.f * (y * z - w * x));
    m.r2 = mk3(2.f * (x * z - w * y), 2.f * (y * z + w * x), 1.f - 2.f * (x * x + y * y));
    return m;
}

XSG_DEV f3 mul(const Mat3& m, f3 v) { return mk3(dot(m.r0, v), dot(m.r1, v), dot(m.r2, v)); }

// The time steps of camera_projection for a static pose, from the projected point: the point does not
// depend on the time, so the projection's time Jacobian is 0 and the Newton step of the Jacobian
// models reduces to the fixed-point step p_time -= residual, as for the other models
// (projection_kernels.h:116-198).
XSG_DEV void static_projection_tail(const Camera& c, f3 uvd, const ProjParams& pp, int mode, float4& uvdt,
                                    bool& valid) {
    float p_time = 0.0f;
    if (mode == XSG_MODE_NEGATIVE) p_time = -fabsf(c.roll_u) * 0.5f;
    else if (mode == XSG_MODE_POSITIVE) p_time = fabsf(c.roll_u) * 0.5f;
    float residual = 0.0f;
    if ((uvd.z <= 0.0f) || (uvd.x < -pp.margin) || (uvd.x > 1.0f + pp.margin) || (uvd.y < -pp.margin) ||
        (uvd.y > 1.0f + pp.margin)) {
        valid = false;
        uvdt = make_float4(0.f, 0.f, 0.f, 0.f);
        return;
    }
    const float real_time = pixel_time(c, uvd.x, uvd.y);
#pragma unroll 1
    for (int i = 0; i < 5; ++i) {
        residual = (c.pose_time + p_time) - real_time;
        p_time -= residual;
        if (fabsf(residual) < pp.thr) break;
    }
    uvdt = make_float4(uvd.x, uvd.y, uvd.z, p_time);
    valid = valid && (fabsf(residual) < pp.max_res) && (uvd.z > 0.0f);
}

// camera_projection for a static pose from the camera-space point. The pinhole projection takes one
// reciprocal of z.
template <int KIND>
XSG_DEV void static_camera_projection(const Camera& c, f3 pc, const ProjParams& pp, int mode, float4& uvdt,
                                      bool& valid) {
    f3 uvd;
    if constexpr (KIND == XSG_CAM_PINHOLE) {
        const float iz = 1.0f / pc.z;
        uvd = mk3(pc.x * c.i0 * iz + c.i2, pc.y * c.i1 * iz + c.i3, pc.z);
    } else {
        uvd = point_to_uvd<KIND>(c, mode, pc);
    }
    static_projection_tail(c, uvd, pp, mode, uvdt, valid);
}

// unscented_transform (ut_kernels.h:52-137) + the radii / on-screen test of
// unscented_transform_projection (ut_kernels.h:140-184) over the seven sigma points that
// proj(i, uvdt, valid) projects (0: the centre; 2k + 1 and 2k + 2: the centre plus and minus delta k).
// On failure mean2d / depth keep what the reference leaves in them (untouched if the centre point
// fails, the accumulated mean if a sigma point fails) and radii come from a zero covariance, because the
// phase-modelled selection (ut_phm_kernels.h:417-421) can pick a failed side.
// The opacity-aware extent of the radii (ut_kernels.h:175-177): one per Gaussian, whatever the mode.
XSG_DEV float ut_extend(float opac) { return fminf(3.33f, sqrtf(2.0f * logf(opac / (1.0f / 255.0f)))); }

// sqrt by the hardware instruction (v_sqrt_f32, within 1 ulp) where the UT's float32 noise is far larger
// than an ulp: the sigma points' ranges and the radii. sqrtf's correctly rounded expansion costs about
// fourteen instructions instead of one.
XSG_DEV float hw_sqrt(float x) { return __builtin_amdgcn_sqrtf(x); }

template <typename Proj>
XSG_DEV bool ut_projection_core(const UtWeights& ut, f2 img, float extend, Proj&& proj, f2& mean2d, f2& radii,
                                float& depth, float& u_distance) {
    float4 uvdt;
    bool valid = true;
    f2 pts[7];
    bool result = true;
    proj(0, uvdt, valid);
    f2 cov_xx_xy = mk2(0.f, 0.f);
    float cov_yy = 0.f;
    if (!valid) {
        result = false;
    } else {
        pts[0] = mk2(uvdt.x * img.x, uvdt.y * img.y);
        mean2d = mk2(ut.wm0 * pts[0].x, ut.wm0 * pts[0].y);
        depth = uvdt.z;
        float u_min = pts[0].x, u_max = pts[0].x;
#pragma unroll
        for (int i = 0; i < 6; ++i) {
            proj(i + 1, uvdt, valid);
            pts[i + 1] = mk2(uvdt.x * img.x, uvdt.y * img.y);
            mean2d.x += ut.wi * pts[i + 1].x;
            mean2d.y += ut.wi * pts[i + 1].y;
            u_min = fminf(u_min, pts[i + 1].x);
            u_max = fmaxf(u_max, pts[i + 1].x);
        }
        if (!valid) {
            result = false;
        } else {
            u_distance = u_max - u_min;
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
    radii = mk2(extend * hw_sqrt(fmaxf(0.0f, cov_xx_xy.x)), extend * hw_sqrt(fmaxf(0.0f, cov_yy)));
    const bool ix = !(((mean2d.x + radii.x) < 0) || (img.x < (mean2d.x - radii.x)));
    const bool iy = !(((mean2d.y + radii.y) < 0) || (img.y < (mean2d.y - radii.y)));
    return result && ix && iy;
}

// One Gaussian in one phase mode. A static pose maps world to camera space by one linear map, so the
// seven camera-space points are M (pw - t0) and that plus and minus M d_k; a moving one solves each
// point's pixel time (camera_projection).
template <int KIND>
XSG_DEV bool ut_projection(const Camera& c, int mode, const UtWeights& ut, f2 img, const ProjParams& pp,
                           f3 pw, f3 pv, float opac, const f3 d[3], bool is_static, f2& mean2d,
                           f2& radii, float& depth, float& u_distance) {
    if (is_static) {
        const Mat3 m = static_world_to_camera(c);
        const f3 pc0 = mul(m, pw - c.t0);
        f3 e[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) e[k] = mul(m, d[k]);
        auto proj = [&](int i, float4& uvdt, bool& valid) {
            const f3 pc = i == 0 ? pc0 : ((i & 1) ? pc0 + e[(i - 1) >> 1] : pc0 - e[(i - 1) >> 1]);
            static_camera_projection<KIND>(c, pc, pp, mode, uvdt, valid);
        };
        return ut_projection_core(ut, img, ut_extend(opac), proj, mean2d, radii, depth, u_distance);
    }
    auto proj = [&](int i, float4& uvdt, bool& valid) {
        const f3 pw_i = i == 0 ? pw : ((i & 1) ? pw + d[(i - 1) >> 1] : pw - d[(i - 1) >> 1]);
        camera_projection<KIND>(c, pw_i, pv, pp, mode, false, uvdt, valid);
    };
    return ut_projection_core(ut, img, ut_extend(opac), proj, mean2d, radii, depth, u_distance);
}

// A static spherical / lidar camera's sigma points before phase unwrapping: each camera-space point's
// u = (azimuth - u0) / du, v and range (point_to_uvd's spherical branch, spherical.h:133-142). None of
// them depends on the phase mode, which only shifts u by one turn (unwrap_u), so the three modes of
// the phase-modelled projection share them, and the binning's seam re-projection of a static pose
// computes them the same way (its depth, the centre's range, is then the stored depth bit for bit).
struct SigmaUv { float u[7], v[7], r[7]; };

// atan(y / x) for 0 <= |y| <= x / 4: the Taylor series of atan t to t^11 (the first term left out,
// t^13 / 13, is below 2^-27 of atan t for |t| <= 1/4).
XSG_DEV float atan_small(float y, float x) {
    const float t = y * __builtin_amdgcn_rcpf(x);
    const float t2 = t * t;
    float q = -1.0f / 11.0f;
    q = fmaf(q, t2, 1.0f / 9.0f);
    q = fmaf(q, t2, -1.0f / 7.0f);
    q = fmaf(q, t2, 1.0f / 5.0f);
    q = fmaf(q, t2, -1.0f / 3.0f);
    return fmaf(q * t2, t, t);
}

// The sigma points p = p0 +- e_k lie close to the centre p0 (0.17 of the Gaussian's scale), so their
// azimuth and elevation are the centre's plus a small angle: the azimuth difference is
// atan2(y0 ex - x0 ey, rho0^2 + x0 ex + y0 ey) (times the sign of the delta), the elevation difference
// atan2(dz rho0 - z0 drho, rho rho0 + z z0) with rho - rho0 = (rho^2 - rho0^2) / (rho + rho0), both
// formed from the deltas without cancellation and evaluated by atan_small; only the centre takes
// atan2 / asin. A point whose angle difference is not small (a Gaussian near the camera or a pole), or
// whose azimuth lands within 1e-4 of the image seam (where atan2's branch decides between 0 and 2 pi),
// takes atan2 / asin of its own coordinates, as the centre does.
XSG_DEV void sigma_uv(const Camera& c, f3 pw, const f3 d[3], SigmaUv& a) {
    const Mat3 m = static_world_to_camera(c);
    const f3 p0 = mul(m, pw - c.t0);
    f3 e[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) e[k] = mul(m, d[k]);
    const float rho0_sq = p0.x * p0.x + p0.y * p0.y;
    const float r0 = hw_sqrt(rho0_sq + p0.z * p0.z);
    const float phi0 = atan2f(-p0.x, -p0.y) + float(M_PI);
    const float theta0 = asinf(p0.z / r0);
    const float rho0 = hw_sqrt(rho0_sq);
    const float two_pi = 2.0f * float(M_PI);
    // u and v by reciprocal multiplies (1 ulp): far below the float32 noise of the UT's weighted sums
    const float inv_du = __builtin_amdgcn_rcpf(c.i1), inv_dv = __builtin_amdgcn_rcpf(c.i3);
    a.u[0] = (phi0 - c.i0) * inv_du;
    a.v[0] = (theta0 - c.i2) * inv_dv;
    a.r[0] = r0;
#pragma unroll
    for (int i = 1; i < 7; ++i) {
        const f3 ek = e[(i - 1) >> 1];
        const float sg = (i & 1) ? 1.0f : -1.0f;
        const f3 p = (i & 1) ? p0 + ek : p0 - ek;
        const float cross_xy = sg * (p0.y * ek.x - p0.x * ek.y);   // y0 x - x0 y
        const float dot_xy = rho0_sq + sg * (p0.x * ek.x + p0.y * ek.y);  // x0 x + y0 y
        const float drho_sq = sg * 2.0f * (p0.x * ek.x + p0.y * ek.y) + (ek.x * ek.x + ek.y * ek.y);
        const float rho_sq = p.x * p.x + p.y * p.y;
        const float rho = hw_sqrt(rho_sq);
        const float r = hw_sqrt(rho_sq + p.z * p.z);
        float phi = phi0 + atan_small(cross_xy, dot_xy);
        phi = phi <= 0.0f ? phi + two_pi : (phi > two_pi ? phi - two_pi : phi);
        const bool phi_small = dot_xy > 0.0f && fabsf(cross_xy) <= 0.25f * dot_xy && phi > 1e-4f &&
                               phi < two_pi - 1e-4f;
        if (!phi_small) phi = atan2f(-p.x, -p.y) + float(M_PI);
        const float drho = drho_sq * __builtin_amdgcn_rcpf(rho + rho0);
        const float num = sg * ek.z * rho0 - p0.z * drho;
        const float den = rho * rho0 + p.z * p0.z;
        float theta;
        if (den > 0.0f && fabsf(num) <= 0.25f * den) theta = theta0 + atan_small(num, den);
        else theta = asinf(p.z / r);
        a.u[i] = (phi - c.i0) * inv_du;
        a.v[i] = (theta - c.i2) * inv_dv;
        a.r[i] = r;
    }
}

// extend: ut_extend of the Gaussian's opacity (computed once for all its modes)
XSG_DEV bool ut_projection_sigma_uv(const Camera& c, const PhaseUnwrap& w, int mode, const UtWeights& ut, f2 img,
                                    const ProjParams& pp, float extend, const SigmaUv& a, f2& mean2d, f2& radii,
                                    float& depth, float& u_distance) {
    auto proj = [&](int i, float4& uvdt, bool& valid) {
        static_projection_tail(c, mk3(unwrap_u(w, mode, a.u[i]), a.v[i], a.r[i]), pp, mode, uvdt, valid);
    };
    return ut_projection_core(ut, img, extend, proj, mean2d, radii, depth, u_distance);
}

// Workgroups are dispatched round-robin over the 8 XCDs; xcd_tile gives each XCD a contiguous run of
// logical blocks, so that neighbouring blocks (tiles that share most of their Gaussians, writer
// segments that share the cache lines at their boundaries) share an L2.
XSG_DEV int xcd_tile(int b, int nblocks) {
    const int x = b & 7, q = nblocks >> 3, r = nblocks & 7;
    return x * q + min(x, r) + (b >> 3);
}

// --------------------------------------------------------------------------
// wave64 helpers
// --------------------------------------------------------------------------
XSG_DEV int lane_id() { return __lane_id(); }

// Sum over the 64 lanes of a wavefront; every lane receives the total.
XSG_DEV float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
