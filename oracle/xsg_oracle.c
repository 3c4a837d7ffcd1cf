/*
 * CPU oracle for the xsimgs Gaussian-splatting hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates the reference algorithm (whesense/xsimgs) on the CPU, one function per
 * reference kernel, each citing the reference file:line it follows. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library, and
 * only as the checker or the timed CPU baseline; the product path never does.
 *
 * Parity pins (what checks each function against something other than itself):
 *   orc_ut_weights            closed form (tests/test_oracle_pins.py)
 *   orc_project_utgs          on-axis closed form, EWA small-scale limit,
 *                             rolling-shutter residual invariant
 *   orc_project_utgs_phm      a float64 restatement of each phase mode from the geometry on
 *                             hand-placed Gaussians covering every branch of the seam
 *                             selection, three shutter timings (tests/test_oracle_phm.py)
 *   orc_camera_rays           closed form pinhole / spherical / lidar rays
 *   orc_camera_rays_bwd       fp64 central differences of orc_camera_rays w.r.t. every camera
 *                             parameter (pinhole, spherical, lidar; world / camera space)
 *   orc_pixel_time_bwd        closed form (pixel time is linear in the camera's timing)
 *   orc_packed_mask_from_instances  numpy packbits (little bit order) of the element mask
 *   orc_rigid_fwd / _bwd      scipy Rotation for the rotations and products; fp64 central
 *                             differences of orc_rigid_fwd for the backward
 *   distorted / fisheye       rays -> projection round trip, zero-coefficient limits (pinhole,
 *   models                    equidistant fisheye), the published OpenCV polynomials evaluated
 *                             independently, undistort map = projection of the pinhole ray,
 *                             fp64 central differences for their intrinsics / coefficient
 *                             gradients; projection_nojac: fixed point = landing pixel's time
 *   orc_sh_fwd / orc_sh_bwd   scipy.special.sph_harm basis, fp64 finite differences
 *   orc_isect_*               brute-force tile enumeration in Python, numpy stable sort;
 *                             the seam spans of orc_isect_spherical_family: exact first- and
 *                             second-span tile sets from a float64 restatement of the
 *                             re-projection and the span bounds, every shutter branch
 *                             (tests/test_oracle_seam.py)
 *   orc_sort_pairs            numpy argsort(kind="stable")
 *   orc_offset_encode         numpy searchsorted
 *   orc_eval3d_fwd            one-Gaussian closed form, two-Gaussian analytic
 *                             composite, depth-sorted brute force without tiles
 *   orc_eval3d_bwd            fp64 finite differences of orc_eval3d_fwd (no-clamp
 *                             regime); the 0.99 clamp band by a hand-derived closed
 *                             form (tests/test_oracle_bwd_band.py)
 */
#include "xsg_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define K(x) ((real)(x))
#ifdef ORC_DOUBLE
#define SQRT sqrt
#define EXP exp
#define LOG log
#define FLOOR floor
#define CEIL ceil
#define ATAN2 atan2
#define ASIN asin
#define SIN sin
#define COS cos
#define FABS fabs
#define COPYSIGN copysign
#define FMIN fmin
#define FMAX fmax
#define HYPOT hypot
#define ORC_PI 3.14159265358979323846
#else
#define SQRT sqrtf
#define EXP expf
#define LOG logf
#define FLOOR floorf
#define CEIL ceilf
#define ATAN2 atan2f
#define ASIN asinf
#define SIN sinf
#define COS cosf
#define FABS fabsf
#define COPYSIGN copysignf
#define FMIN fminf
#define FMAX fmaxf
#define HYPOT hypotf
#define ORC_PI ((float)3.14159265358979323846)
#endif

#define ALPHA_THR_MIN (K(1.0) / K(255.0))

typedef struct { real x, y; } v2;
typedef struct { real x, y, z; } v3;
/* glm-style 3x3 matrix: m[col][row] */
typedef struct { real m[3][3]; } m3;

static inline v3 V3(real x, real y, real z) { v3 r = {x, y, z}; return r; }
static inline v3 add3(v3 a, v3 b) { return V3(a.x + b.x, a.y + b.y, a.z + b.z); }
static inline v3 sub3(v3 a, v3 b) { return V3(a.x - b.x, a.y - b.y, a.z - b.z); }
static inline v3 scl3(v3 a, real s) { return V3(a.x * s, a.y * s, a.z * s); }
static inline real dot3(v3 a, v3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
static inline v3 cross3(v3 a, v3 b) {
    return V3(a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x);
}
static inline v3 ld3(const real *p) { return V3(p[0], p[1], p[2]); }
static inline v3 mv(const m3 *M, v3 v) { /* glm M * v */
    return V3(M->m[0][0] * v.x + M->m[1][0] * v.y + M->m[2][0] * v.z,
              M->m[0][1] * v.x + M->m[1][1] * v.y + M->m[2][1] * v.z,
              M->m[0][2] * v.x + M->m[1][2] * v.y + M->m[2][2] * v.z);
}
static inline m3 transpose3(const m3 *A) {
    m3 r;
    for (int c = 0; c < 3; ++c) for (int k = 0; k < 3; ++k) r.m[c][k] = A->m[k][c];
    return r;
}
static inline v3 normalize3(v3 v) { real l = SQRT(dot3(v, v)); return scl3(v, K(1.0) / l); }

/* ------------------------------------------------------------------------- */
/* UT weights: include/cameras/ut_kernels.h:17-36                           */
/* ------------------------------------------------------------------------- */
void orc_ut_weights(real ut_alpha, real ut_beta, real ut_kappa, real *out4) {
    const real lam = ut_alpha * ut_alpha * (K(3) + ut_kappa) - K(3);
    out4[0] = lam / (K(3) + lam);
    out4[1] = lam / (K(3) + lam) + (K(1) - ut_alpha * ut_alpha + ut_beta);
    out4[2] = K(1) / (K(2) * (K(3) + lam));
    out4[3] = SQRT(lam + K(3));
}

/* ------------------------------------------------------------------------- */
/* Rolling-shutter projection: include/cameras/projection_kernels.h:12-256   */
/* ------------------------------------------------------------------------- */
static void jac_quat_from_axis_angle(v3 w, real t, real *qw, v3 *qxyz, real *dqw, v3 *dqxyz) {
    /* projection_kernels.h:12-36 */
    const real w_norm2 = dot3(w, w);
    const real w_norm = SQRT(w_norm2);
    const real theta = w_norm * FABS(t);
    const real sin_half = SIN(K(0.5) * theta), cos_half = COS(K(0.5) * theta);
    const real scale = (theta < K(1e-2)) ? K(0.5) - theta * theta * (K(1.0) / K(48.0))
                                         : sin_half / theta;
    *qw = cos_half;
    *qxyz = scl3(scl3(w, scale), t);
    *dqw = K(-0.5) * COPYSIGN(K(1.0), t) * sin_half * w_norm;
    *dqxyz = scl3(w, K(0.5) * cos_half);
}

static v3 quat_apply(real w, v3 xyz, v3 p) { /* projection_kernels.h:67-71 */
    const v3 uv = cross3(xyz, p);
    const v3 uuv = cross3(xyz, uv);
    return add3(p, scl3(add3(scl3(uv, w), uuv), K(2.0)));
}

static void jac_world_to_camera(const orc_camera *c, v3 point, v3 pvel, real time,
                                v3 *result, v3 *d_result) {
    /* projection_kernels.h:74-113 (quat_mul :38-51, quat_apply jac :53-65) */
    real w1, dw1; v3 xyz1, dxyz1;
    jac_quat_from_axis_angle(ld3(c->w), time, &w1, &xyz1, &dw1, &dxyz1);
    const real w2 = c->q[0];
    const v3 xyz2 = V3(c->q[1], c->q[2], c->q[3]);
    real w = w1 * w2 - dot3(xyz1, xyz2);
    v3 xyz = add3(add3(scl3(xyz2, w1), scl3(xyz1, w2)), cross3(xyz1, xyz2));
    real dw = dw1 * w2 - dot3(dxyz1, xyz2);
    v3 dxyz = add3(add3(scl3(xyz2, dw1), scl3(dxyz1, w2)), cross3(dxyz1, xyz2));
    xyz = scl3(xyz, K(-1));
    dxyz = scl3(dxyz, K(-1));
    const v3 vdiff = sub3(pvel, ld3(c->v));
    const v3 p = add3(sub3(point, ld3(c->t)), scl3(vdiff, time));
    const v3 uv = cross3(xyz, p);
    const v3 uuv = cross3(xyz, uv);
    *result = add3(p, scl3(add3(scl3(uv, w), uuv), K(2.0)));
    const v3 duv = cross3(dxyz, p);
    const v3 dp = scl3(add3(add3(scl3(uv, dw), scl3(duv, w)), add3(cross3(dxyz, uv), cross3(xyz, duv))),
                       K(2.0));
    *d_result = add3(dp, quat_apply(w, xyz, vdiff));
}

static real u_pose_of(const orc_camera *c) { /* spherical.h:113-114 */
    return (FABS(c->rolling[0]) > K(0)) ? (c->pose_time - c->trigger_time) / c->rolling[0] : K(0.5);
}

static v2 angles_to_uv(const orc_camera *c, int mode, real phi, real theta) {
    /* csrc/cameras/spherical.h:109-125 */
    real u = (phi - c->impl[0]) / c->impl[1];
    const real u_pose = u_pose_of(c);
    const real u_offset = (K(2.0) * ORC_PI / FABS(c->impl[1]));
    if (c->rolling[0] > 0) {
        if (mode == ORC_MODE_NEG && u > u_pose) u = u - u_offset;
        if (mode == ORC_MODE_POS && u < u_pose) u = u + u_offset;
    } else {
        if (mode == ORC_MODE_NEG && u < u_pose) u = u + u_offset;
        if (mode == ORC_MODE_POS && u > u_pose) u = u - u_offset;
    }
    const real v = (theta - c->impl[2]) / c->impl[3];
    v2 r = {u, v};
    return r;
}

/* ------------------------------------------------------------------------- */
/* Distorted perspective (OpenCV rational + tangential) and OpenCV fisheye    */
/* camera models: csrc/cameras/distorted_perspective.cu, fisheye_opencv.cu,   */
/* include/cameras/distortion.h                                               */
/* ------------------------------------------------------------------------- */
#define DIST_MIN_DET K(1e-3)

/* uv_distortion (distortion.h:8-30): radial scale and tangential offset of a camera-space uv */
static void uv_distortion(const real *k, real u, real v, real *scale, real *du, real *dv) {
    const real uu = u * u, vv = v * v;
    const real r2 = uu + vv;
    const real num = K(1.0) + r2 * (k[0] + r2 * (k[1] + r2 * k[4]));
    const real den = K(1.0) + r2 * (k[5] + r2 * (k[6] + r2 * k[7]));
    *scale = num / den;
    const real uv2 = K(2.0) * u * v;
    *du = k[2] * uv2 + k[3] * (r2 + K(2.0) * uu);
    *dv = k[2] * (r2 + K(2.0) * vv) + k[3] * uv2;
}

/* DistortionState (distorted_perspective.cu:11-36, :44-78): the distortion at uv with its
 * (symmetric) Jacobian */
typedef struct { real scale, denom, dx, dy, juu, juv, jvv; } dist_state;

static dist_state distortion_state(const real *k, real u, real v) {
    const real k1 = k[0], k2 = k[1], p1 = k[2], p2 = k[3], k3 = k[4], k4 = k[5], k5 = k[6], k6 = k[7];
    const real r2 = u * u + v * v;
    const real num = K(1.0) + r2 * (k1 + r2 * (k2 + r2 * k3));
    const real den = K(1.0) + r2 * (k4 + r2 * (k5 + r2 * k6));
    const real scale = num / den;
    const real d_num = k1 + r2 * (K(2.0) * k2 + K(3.0) * k3 * r2);
    const real d_den = k4 + r2 * (K(2.0) * k5 + K(3.0) * k6 * r2);
    const real d_scale = (d_num * den - num * d_den) / (den * den);
    dist_state s;
    s.scale = scale;
    s.denom = den;
    s.dx = K(2.0) * p1 * u * v + p2 * (r2 + K(2.0) * u * u);
    s.dy = p1 * (r2 + K(2.0) * v * v) + K(2.0) * p2 * u * v;
    s.juu = scale + K(2.0) * u * u * d_scale + K(2.0) * p1 * v + K(6.0) * p2 * u;
    s.juv = K(2.0) * u * v * d_scale + K(2.0) * p1 * u + K(2.0) * p2 * v;
    s.jvv = scale + K(2.0) * v * v * d_scale + K(6.0) * p1 * v + K(2.0) * p2 * u;
    return s;
}

/* undistort_uv (distorted_perspective.cu:80-98): five Newton steps on uv * scale + delta = uv_d,
 * a fixed-point step where the Jacobian is nearly singular. `st` keeps the state of the last step
 * (taken before that step's update). */
static v2 undistort_uv(const real *k, v2 ud, dist_state *st) {
    v2 uv = ud;
    for (int j = 0; j < 5; ++j) {
        *st = distortion_state(k, uv.x, uv.y);
        const real rx = uv.x * st->scale + st->dx - ud.x;
        const real ry = uv.y * st->scale + st->dy - ud.y;
        const real det = st->juu * st->jvv - st->juv * st->juv;
        if (FABS(det) > DIST_MIN_DET) {
            uv.x -= (st->jvv * rx - st->juv * ry) / det;
            uv.y -= (st->juu * ry - st->juv * rx) / det;
        } else {
            uv.x = (ud.x - st->dx) / st->scale;
            uv.y = (ud.y - st->dy) / st->scale;
        }
    }
    return uv;
}

/* Kannala-Brandt polynomial and its derivative (fisheye_opencv.cu:14-32) */
static real fisheye_distortion(const real *k, real theta) {
    const real t2 = theta * theta;
    real d = t2 * k[3] + k[2];
    d = t2 * d + k[1];
    d = t2 * d + k[0];
    d = t2 * d + K(1.0);
    return theta * d;
}

static real fisheye_distortion_deriv(const real *k, real theta) {
    const real t2 = theta * theta;
    real d = t2 * K(9.0) * k[3] + K(7.0) * k[2];
    d = t2 * d + K(5.0) * k[1];
    d = t2 * d + K(3.0) * k[0];
    d = t2 * d + K(1.0);
    return d;
}

/* solve_theta (fisheye_opencv.cu:34-46): at most 20 Newton steps with the derivative clamped at 0.1
 * and theta kept in [0, pi] */
static real fisheye_solve_theta(const real *k, real delta, real *residual) {
    real theta = delta;
    *residual = 0;
    for (int i = 0; i < 20; ++i) {
        *residual = fisheye_distortion(k, theta) - delta;
        theta -= *residual / FMAX(fisheye_distortion_deriv(k, theta), K(0.1));
        theta = FMIN(FMAX(theta, K(0.0)), ORC_PI);
        if (FABS(*residual) < K(1e-6)) break;
    }
    return theta;
}

/* camera_point_to_uvd of every camera model (perspective.cu:36-42, spherical.h:133-142,
 * distorted_perspective.cu:190-197, fisheye_opencv.cu:138-148) */
static v3 point_to_uvd(const orc_camera *c, int mode, v3 p) {
    const real fx = c->impl[0], fy = c->impl[1], cx = c->impl[2], cy = c->impl[3];
    if (c->kind == ORC_PINHOLE) return V3(p.x * fx / p.z + cx, p.y * fy / p.z + cy, p.z);
    if (c->kind == ORC_DISTORTED) {
        const real x = p.x / p.z, y = p.y / p.z;
        real scale, du, dv;
        uv_distortion(c->dist, x, y, &scale, &du, &dv);
        const real r2 = x * x + y * y;
        return V3((x * scale + du) * fx + cx, (y * scale + dv) * fy + cy, (r2 <= c->max_radius_sq) ? p.z : K(0));
    }
    if (c->kind == ORC_FISHEYE) {
        const real norm = FMAX(K(1e-6), HYPOT(p.x, p.y));
        const real theta = ATAN2(norm, p.z);
        const int valid = fisheye_distortion_deriv(c->dist, theta) > K(0);
        const real delta = fisheye_distortion(c->dist, theta) / norm;
        const real depth = (valid && delta > K(0)) ? SQRT(dot3(p, p)) : K(0);
        return V3(fx * delta * p.x + cx, fy * delta * p.y + cy, depth);
    }
    const real r = SQRT(p.x * p.x + p.y * p.y + p.z * p.z);
    const real phi = ATAN2(-p.x, -p.y) + ORC_PI;
    const real theta = ASIN(p.z / r);
    const v2 uv = angles_to_uv(c, mode, phi, theta);
    return V3(uv.x, uv.y, r);
}

static int has_projection_jacobian(const orc_camera *c) {
    return c->kind == ORC_PINHOLE || c->kind == ORC_SPHERICAL || c->kind == ORC_LIDAR;
}

static void point_to_uvd_jacob(const orc_camera *c, int mode, v3 p, v3 dp, v3 *uvd, v2 *du_dv) {
    if (c->kind == ORC_PINHOLE) {
        /* csrc/cameras/perspective.cu:36-52 */
        const real fx = c->impl[0], fy = c->impl[1], cx = c->impl[2], cy = c->impl[3];
        *uvd = V3(p.x * fx / p.z + cx, p.y * fy / p.z + cy, p.z);
        du_dv->x = fx * (dp.x - uvd->x * dp.z) / uvd->z;
        du_dv->y = fy * (dp.y - uvd->y * dp.z) / uvd->z;
    } else {
        /* csrc/cameras/spherical.h:133-153 */
        const real x2y2 = p.x * p.x + p.y * p.y;
        const real r = SQRT(x2y2 + p.z * p.z);
        const real phi = ATAN2(-p.x, -p.y) + ORC_PI;
        const real theta = ASIN(p.z / r);
        const v2 uv = angles_to_uv(c, mode, phi, theta);
        *uvd = V3(uv.x, uv.y, r);
        const real x2y2_sqrt = SQRT(x2y2);
        const real r2 = r * r;
        const real mul = p.z / (r2 * x2y2_sqrt);
        du_dv->x = ((-p.x * dp.y + p.y * dp.x) / x2y2) / c->impl[1];
        du_dv->y = ((x2y2_sqrt * dp.z) / r2 - mul * (p.x * dp.x + p.y * dp.y)) / c->impl[3];
    }
}

/* Float32 decision margins (test diagnostics only; they change no result). While tl_mg is set, the
 * UT helpers lower *tl_mg to the smallest ratio |x - threshold| / e(x) over the threshold decisions
 * they take, e(x) being a bound on the error a float32 evaluation of x carries (F32_U = 2^-24, the
 * float32 unit roundoff, whatever precision this build computes in). A ratio below 1 marks an
 * outcome that float32 rounding can decide either way. tl_ut_err carries the error bounds of the
 * last unscented_transform to ut_projection and the phase-modelled selection. */
#define F32_U K(5.9604644775390625e-8)
static _Thread_local real *tl_mg;
typedef struct { real em, erx, ery, ep_max, rx_err, ry_err; } ut_err_t;
static _Thread_local ut_err_t tl_ut_err;
static void mg_note(real dist, real bound) {
    if (!tl_mg) return;
    const real r = FABS(dist) / (bound > 0 ? bound : (real)1e-30);
    if (r < *tl_mg) *tl_mg = r;
}

static void camera_projection(const orc_camera *c, v3 p_world, v3 p_vel, real thr, real max_res,
                              real margin, int mode, int no_jac, real uvdt[4], int *valid) {
    /* projection_kernels.h:201-256 with jac_camera_projection_iteration :116-174 for the models
     * that have a projection Jacobian, else (and for projection_nojac) the fixed-point
     * camera_projection_iteration :177-198 */
    const int newton = has_projection_jacobian(c) && !no_jac;
    v3 uvd = V3(0, 0, 0);
    real p_time = 0;
    if (mode == ORC_MODE_NEG) p_time = -FABS(c->rolling[0]) * K(0.5);
    else if (mode == ORC_MODE_POS) p_time = FABS(c->rolling[0]) * K(0.5);
    real residual = 0;
    for (int i = 0; i < 5; ++i) {
        v3 pc, jpc; v2 du_dv = {0, 0};
        jac_world_to_camera(c, p_world, p_vel, p_time, &pc, &jpc);
        if (newton) point_to_uvd_jacob(c, mode, pc, jpc, &uvd, &du_dv);
        else uvd = point_to_uvd(c, mode, pc);
        const real assumed = c->pose_time + p_time;
        const real real_time = c->trigger_time + (uvd.x * c->rolling[0] + uvd.y * c->rolling[1]);
        residual = assumed - real_time;
        if (newton) {
            const real d_res = K(1.0) - (du_dv.x * c->rolling[0] + du_dv.y * c->rolling[1]);
            p_time -= residual / d_res;
        } else {
            p_time -= residual;
        }
        if (tl_mg) {  /* uvd carries a few roundings of the camera point and the projection */
            const real ez = K(8) * F32_U * (FABS(pc.x) + FABS(pc.y) + FABS(pc.z) + FABS(uvd.z));
            const real eu = K(16) * F32_U * (FABS(uvd.x) + K(1)), ev = K(16) * F32_U * (FABS(uvd.y) + K(1));
            mg_note(uvd.z, ez);
            mg_note(uvd.x + margin, eu); mg_note(uvd.x - K(1) - margin, eu);
            mg_note(uvd.y + margin, ev); mg_note(uvd.y - K(1) - margin, ev);
        }
        if ((uvd.z <= K(0)) || (uvd.x < -margin) || (uvd.x > K(1) + margin) ||
            (uvd.y < -margin) || (uvd.y > K(1) + margin)) {
            *valid = 0;
            uvdt[0] = uvdt[1] = uvdt[2] = uvdt[3] = 0;
            return;
        }
        if (FABS(residual) < thr) break;
    }
    uvdt[0] = uvd.x; uvdt[1] = uvd.y; uvdt[2] = uvd.z; uvdt[3] = p_time;
    *valid = *valid && (FABS(residual) < max_res) && (uvd.z > K(0));
}

/* unscented_transform_deltas: ut_kernels.h:38-49. deltas[i] = column i of R(q) * s_i * sqrt(3+lambda).
 * The quaternion is normalised first (unit-quaternion assumption; toast's to_matrix is not in the tree). */
static void ut_deltas(real sqrt_dl, const real *q, const real *s, v3 d[3]) {
    real w = q[0], x = q[1], y = q[2], z = q[3];
    const real inv = K(1.0) / SQRT(w * w + x * x + y * y + z * z);
    w *= inv; x *= inv; y *= inv; z *= inv;
    const v3 c0 = V3(K(1) - K(2) * (y * y + z * z), K(2) * (x * y + w * z), K(2) * (x * z - w * y));
    const v3 c1 = V3(K(2) * (x * y - w * z), K(1) - K(2) * (x * x + z * z), K(2) * (y * z + w * x));
    const v3 c2 = V3(K(2) * (x * z + w * y), K(2) * (y * z - w * x), K(1) - K(2) * (x * x + y * y));
    d[0] = scl3(c0, s[0] * sqrt_dl);
    d[1] = scl3(c1, s[1] * sqrt_dl);
    d[2] = scl3(c2, s[2] * sqrt_dl);
}

static int unscented_transform(const orc_camera *c, const real ut[4], v2 img, int mode, real thr,
                               real max_res, real margin, v3 p_world, v3 p_vel, const v3 d[3],
                               v2 *mean2d, real *depth, real *u_distance, v3 *cov2d) {
    /* ut_kernels.h:52-137 */
    real uvdt[4]; int valid = 1;
    v2 pts[7];
    camera_projection(c, p_world, p_vel, thr, max_res, margin, mode, 0, uvdt, &valid);
    if (!valid) return 0;
    pts[0].x = uvdt[0] * img.x; pts[0].y = uvdt[1] * img.y;
    mean2d->x = ut[0] * pts[0].x; mean2d->y = ut[0] * pts[0].y;
    *depth = uvdt[2];
    real u_min = pts[0].x, u_max = pts[0].x;
    real sign = K(1.0);
    for (int i = 0; i < 6; ++i) {
        camera_projection(c, add3(p_world, scl3(d[i / 2], sign)), p_vel, thr, max_res, margin, mode, 0,
                          uvdt, &valid);
        pts[i + 1].x = uvdt[0] * img.x; pts[i + 1].y = uvdt[1] * img.y;
        mean2d->x += ut[2] * pts[i + 1].x; mean2d->y += ut[2] * pts[i + 1].y;
        u_min = FMIN(u_min, pts[i + 1].x);
        u_max = FMAX(u_max, pts[i + 1].x);
        sign *= K(-1.0);
    }
    if (!valid) return 0;
    *u_distance = u_max - u_min;
    real vx = pts[0].x - mean2d->x, vy = pts[0].y - mean2d->y;
    *cov2d = V3(ut[1] * (vx * vx), ut[1] * (vx * vy), ut[1] * (vy * vy));
    for (int i = 1; i < 7; ++i) {
        vx = pts[i].x - mean2d->x; vy = pts[i].y - mean2d->y;
        cov2d->x += ut[2] * (vx * vx); cov2d->y += ut[2] * (vx * vy); cov2d->z += ut[2] * (vy * vy);
    }
    const real det = cov2d->x * cov2d->z - cov2d->y * cov2d->y;
    if (tl_mg) {
        /* each sigma point in pixels carries a few roundings of its own size (and of the principal
         * point added to it); the weighted sums cancel terms |w| times larger than the mean
         * (ut_kernels.h:17-36) */
        const real u = F32_U;
        real ep[7], em = 0, epm = 0;
        for (int i = 0; i < 7; ++i) {
            ep[i] = u * (K(3) * (FABS(pts[i].x) + FABS(pts[i].y)) + K(0.5) * (img.x + img.y));
            const real w = FABS(i ? ut[2] : ut[0]);
            em += w * (ep[i] + K(4) * u * (FABS(pts[i].x) + FABS(pts[i].y)));
            epm = FMAX(epm, ep[i]);
        }
        /* each point's own error enters through 2 w v_i; an error d of the mean shifts every v_i by
         * the same d and moves the covariance by 2 d sum(w_c v) + d^2 sum(w_c) only: the mean weights
         * sum to 1, so sum(w_c v) = (w_c0 - w_m0) v_0 */
        real dcx = 0, dcy = 0, dcz = 0, s1x = 0, s1y = 0, sw = 0;
        for (int i = 0; i < 7; ++i) {
            const real wc = i ? ut[2] : ut[1], w = FABS(wc);
            const real vx = pts[i].x - mean2d->x, vy = pts[i].y - mean2d->y;
            const real ax = FABS(vx), ay = FABS(vy);
            dcx += w * (K(2) * ax * ep[i] + K(4) * u * ax * ax);
            dcz += w * (K(2) * ay * ep[i] + K(4) * u * ay * ay);
            dcy += w * ((ax + ay) * ep[i] + K(4) * u * ax * ay);
            s1x += wc * vx; s1y += wc * vy; sw += wc;
        }
        dcx += K(2) * FABS(s1x) * em + FABS(sw) * em * em;
        dcz += K(2) * FABS(s1y) * em + FABS(sw) * em * em;
        dcy += (FABS(s1x) + FABS(s1y)) * em + FABS(sw) * em * em;
        const real edet = dcx * FABS(cov2d->z) + dcz * FABS(cov2d->x) + K(2) * FABS(cov2d->y) * dcy +
                          K(4) * u * (FABS(cov2d->x * cov2d->z) + cov2d->y * cov2d->y);
        mg_note(det, edet);
        mg_note(cov2d->x, dcx);
        mg_note(cov2d->z, dcz);
        tl_ut_err.em = em;
        tl_ut_err.erx = cov2d->x > 0 ? dcx / (K(2) * SQRT(cov2d->x)) : K(1e30);
        tl_ut_err.ery = cov2d->z > 0 ? dcz / (K(2) * SQRT(cov2d->z)) : K(1e30);
        tl_ut_err.ep_max = epm;
    }
    if (det <= K(0) || cov2d->x < 0 || cov2d->z < 0) return 0;
    return 1;
}

static int ut_projection(const orc_camera *c, int mode, const real ut[4], v2 img, real thr,
                         real max_res, real margin, v3 p_world, v3 p_vel, real opac,
                         const v3 d[3], v2 *mean2d, v2 *radii, real *depth, real *u_distance) {
    /* ut_kernels.h:140-184 */
    v3 cov2d = V3(0, 0, 0);
    const int result = unscented_transform(c, ut, img, mode, thr, max_res, margin, p_world, p_vel, d,
                                           mean2d, depth, u_distance, &cov2d);
    const real extend = FMIN(K(3.33), SQRT(K(2.0) * LOG(opac / ALPHA_THR_MIN)));
    radii->x = extend * SQRT(FMAX(K(0), cov2d.x));
    radii->y = extend * SQRT(FMAX(K(0), cov2d.z));
    const int ix = !(((mean2d->x + radii->x) < 0) || (img.x < (mean2d->x - radii->x)));
    const int iy = !(((mean2d->y + radii->y) < 0) || (img.y < (mean2d->y - radii->y)));
    if (tl_mg && result) {
        tl_ut_err.rx_err = extend * tl_ut_err.erx + K(4) * F32_U * radii->x;
        tl_ut_err.ry_err = extend * tl_ut_err.ery + K(4) * F32_U * radii->y;
        const real ex = tl_ut_err.em + tl_ut_err.rx_err + K(4) * F32_U * FABS(mean2d->x);
        const real ey = tl_ut_err.em + tl_ut_err.ry_err + K(4) * F32_U * FABS(mean2d->y);
        mg_note(mean2d->x + radii->x, ex); mg_note(mean2d->x - radii->x - img.x, ex);
        mg_note(mean2d->y + radii->y, ey); mg_note(mean2d->y - radii->y - img.y, ey);
    }
    return result && ix && iy;
}

/* Projection of points (uvdt + mask): projection_kernels.h:259-309 (jacobian variant). */
void orc_projection(const orc_camera *c, int n, const real *pts, const real *vel, real thr,
                    real max_res, real margin, int mode, int no_jac, real *uvdt_out, uint8_t *mask_out) {
    for (int i = 0; i < n; ++i) {
        int valid = 1; real uvdt[4];
        const v3 pv = vel ? ld3(vel + 3 * i) : V3(0, 0, 0);
        camera_projection(c, ld3(pts + 3 * i), pv, thr, max_res, margin, mode, no_jac, uvdt, &valid);
        uvdt[3] += c->pose_time;
        memcpy(uvdt_out + 4 * i, uvdt, sizeof(uvdt));
        valid = valid && (uvdt[0] >= 0 && uvdt[1] >= 0) && (uvdt[0] <= 1 && uvdt[1] <= 1);
        mask_out[i] = (uint8_t)valid;
    }
}

/* UT projection: unscented_transform_kernel ut_kernels.h:187-246 + launcher :249-305.
 * Outputs are zero for culled Gaussians (the reference zero-initialises, :276-280). */
void orc_project_utgs(const orc_camera *c, int n, const real *means, const real *vel,
                      const real *scales, const real *quats, const real *opacity, real width,
                      real height, const real ut[4], real thr, real max_res, real margin,
                      uint8_t *flags, real *radii, real *means2d, real *depths, real *fmargin) {
    const v2 img = {width, height};
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i) {
        real mg = K(1e30);
        flags[i] = 0; radii[2 * i] = radii[2 * i + 1] = 0;
        means2d[2 * i] = means2d[2 * i + 1] = 0; depths[i] = 0;
        if (fmargin) fmargin[i] = mg;
        const real op = opacity ? opacity[i] : K(1.0);
        if (op < ALPHA_THR_MIN) continue;
        v3 d[3];
        ut_deltas(ut[3], quats + 4 * i, scales + 3 * i, d);
        v2 m2, r2; real depth = 0, udist = 0;
        const v3 pv = vel ? ld3(vel + 3 * i) : V3(0, 0, 0);
        /* the margin pointer lives only around the one call that notes into mg */
        tl_mg = fmargin ? &mg : NULL;
        const int ok = ut_projection(c, ORC_MODE_CENTRAL, ut, img, thr, max_res, margin,
                                     ld3(means + 3 * i), pv, op, d, &m2, &r2, &depth, &udist);
        if (fmargin) fmargin[i] = mg;
        tl_mg = NULL;
        if (!ok) continue;
        radii[2 * i] = r2.x; radii[2 * i + 1] = r2.y;
        flags[i] = 1;
        means2d[2 * i] = m2.x; means2d[2 * i + 1] = m2.y;
        depths[i] = depth;
    }
}

/* Phase-modelled UT: unscented_transform_phm_kernel ut_phm_kernels.h:13-114. */
void orc_project_utgs_phm(const orc_camera *c, int n, const real *means, const real *vel,
                          const real *scales, const real *quats, const real *opacity, real width,
                          real height, const real ut[4], real thr, real max_res, real margin,
                          uint8_t *flags, real *radii, real *means2d, real *depths, real *fmargin) {
    const v2 img = {width, height};
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i) {
        real mg = K(1e30);
        tl_mg = fmargin ? &mg : NULL;
        flags[i] = 0; radii[2 * i] = radii[2 * i + 1] = 0;
        means2d[2 * i] = means2d[2 * i + 1] = 0; depths[i] = 0;
        if (fmargin) fmargin[i] = mg;
        const real op = opacity ? opacity[i] : K(1.0);
        if (op < ALPHA_THR_MIN) { tl_mg = NULL; continue; }
        v3 d[3];
        ut_deltas(ut[3], quats + 4 * i, scales + 3 * i, d);
        const v3 pw = ld3(means + 3 * i);
        const v3 pv = vel ? ld3(vel + 3 * i) : V3(0, 0, 0);
        v2 rc = {0, 0}, rl = {0, 0}, rr = {0, 0}, mc = {0, 0}, ml = {0, 0}, mr = {0, 0};
        real dc = 0, dl = 0, dr = 0, ud = 0;
        const real u_pi = ORC_PI * img.x / FABS(c->impl[1]);
        /* u_distance = u_max - u_min over the sigma points: two sigma points' errors */
#define PHM_NOTE(res_) do { if (tl_mg && (res_)) mg_note(ud - u_pi, K(2) * tl_ut_err.ep_max + K(4) * F32_U * u_pi); } while (0)
        int res = ut_projection(c, ORC_MODE_CENTRAL, ut, img, thr, max_res, margin, pw, pv, op, d,
                                &mc, &rc, &dc, &ud);
        PHM_NOTE(res);
        if (!res) { if (fmargin) fmargin[i] = mg; tl_mg = NULL; continue; }
        const int r_c = res * ((ud > u_pi) + 1);
        res = ut_projection(c, ORC_MODE_NEG, ut, img, thr, max_res, margin, pw, pv, op, d, &ml, &rl,
                            &dl, &ud);
        PHM_NOTE(res);
        const int r_l = res * ((ud > u_pi) + 1);
        res = ut_projection(c, ORC_MODE_POS, ut, img, thr, max_res, margin, pw, pv, op, d, &mr, &rr,
                            &dr, &ud);
        PHM_NOTE(res);
#undef PHM_NOTE
        if (fmargin) fmargin[i] = mg;
        tl_mg = NULL;
        const int r_r = res * ((ud > u_pi) + 1);
        if (r_l == 1 && r_r == 1) {
            flags[i] = 2; radii[2 * i] = rl.x; radii[2 * i + 1] = rl.y;
            means2d[2 * i] = ml.x; means2d[2 * i + 1] = ml.y; depths[i] = dl;
            continue;
        }
        if (r_c == 1) {
            flags[i] = 1; radii[2 * i] = rc.x; radii[2 * i + 1] = rc.y;
            means2d[2 * i] = mc.x; means2d[2 * i + 1] = mc.y; depths[i] = dc;
            continue;
        }
        if (r_l != 1 && r_r != 1) continue;
        const int use_left = r_l != 1;  /* reference selects the non-compact side's partner */
        flags[i] = 1;
        radii[2 * i] = use_left ? rl.x : rr.x; radii[2 * i + 1] = use_left ? rl.y : rr.y;
        means2d[2 * i] = use_left ? ml.x : mr.x; means2d[2 * i + 1] = use_left ? ml.y : mr.y;
        depths[i] = use_left ? dl : dr;
    }
}

/* ------------------------------------------------------------------------- */
/* Camera rays: ray_kernels.h:7-59, camera.h:85-131, base_camera_impl.h:9-14 */
/* ------------------------------------------------------------------------- */
static v3 pixel_to_camera_ray(const orc_camera *c, real u, real v) {
    if (c->kind == ORC_PINHOLE) { /* perspective.cu:13-16 */
        return V3((u - c->impl[2]) / c->impl[0], (v - c->impl[3]) / c->impl[1], K(1.0));
    }
    if (c->kind == ORC_DISTORTED) { /* distorted_perspective.cu:100-105 */
        dist_state st;
        const v2 ud = {(u - c->impl[2]) / c->impl[0], (v - c->impl[3]) / c->impl[1]};
        const v2 uc = undistort_uv(c->dist, ud, &st);
        return V3(uc.x, uc.y, K(1.0));
    }
    if (c->kind == ORC_FISHEYE) { /* fisheye_opencv.cu:48-62 */
        const real x = (u - c->impl[2]) / c->impl[0], y = (v - c->impl[3]) / c->impl[1];
        const real delta = SQRT(x * x + y * y);
        real residual;
        const real theta = fisheye_solve_theta(c->dist, delta, &residual);
        if (theta <= K(0)) return V3(0, 0, K(1.0));
        const real sf = SIN(theta) / delta;
        return V3(sf * x, sf * y, COS(theta));
    }
    /* spherical.h:9-22, 121-127 */
    const real az = c->impl[0] + u * c->impl[1];
    const real el = c->impl[2] + v * c->impl[3];
    const real xy = K(1.0) * COS(el);
    return V3(xy * SIN(az), xy * COS(az), K(1.0) * SIN(el));
}

/* ray_valid (camera.h:114-120): distorted_perspective.cu:107-117 (the undistortion converged
 * to 1e-5, inside max_radius), fisheye_opencv.cu:64-72 (converged, on the rising branch of the
 * polynomial); every other model is valid everywhere */
static int ray_valid(const orc_camera *c, real u, real v) {
    if (c->kind == ORC_DISTORTED) {
        dist_state st;
        const v2 ud = {(u - c->impl[2]) / c->impl[0], (v - c->impl[3]) / c->impl[1]};
        const v2 uc = undistort_uv(c->dist, ud, &st);
        const real rx = uc.x * st.scale + st.dx - ud.x, ry = uc.y * st.scale + st.dy - ud.y;
        const real r2 = uc.x * uc.x + uc.y * uc.y;
        return (r2 <= c->max_radius_sq) && (FABS(rx) < K(1e-5)) && (FABS(ry) < K(1e-5));
    }
    if (c->kind == ORC_FISHEYE) {
        const real x = (u - c->impl[2]) / c->impl[0], y = (v - c->impl[3]) / c->impl[1];
        const real delta = SQRT(x * x + y * y);
        if (delta <= K(1e-8)) return 1;
        real residual;
        const real theta = fisheye_solve_theta(c->dist, delta, &residual);
        return (FABS(residual) < K(1e-5)) && (fisheye_distortion_deriv(c->dist, theta) > K(0));
    }
    return 1;
}

/* undistort_map (distortion.h:33-56) with distort_uv of distorted_perspective.cu:199-203 and
 * fisheye_opencv.cu:150-156: per pixel, the distorted position of the pixel's undistorted uv, in
 * [0, 1] with normalized_range set, else mapped to [-1, 1] */
void orc_undistort_map(const orc_camera *c, int width, int height, int normalized_range, real *out) {
    const real fx = c->impl[0], fy = c->impl[1], cx = c->impl[2], cy = c->impl[3];
    for (int idx = 0; idx < width * height; ++idx) {
        const int px = idx % width, py = idx / width;
        const real u = ((real)px + K(0.5)) / (real)width;
        const real v = ((real)py + K(0.5)) / (real)height;
        const real x = (u - cx) / fx, y = (v - cy) / fy;
        real ru, rv;
        if (c->kind == ORC_DISTORTED) {
            real scale, du, dv;
            uv_distortion(c->dist, x, y, &scale, &du, &dv);
            ru = (x * scale + du) * fx + cx;
            rv = (y * scale + dv) * fy + cy;
        } else {
            const real theta = SQRT(x * x + y * y);
            const real scale = (theta > K(1e-8)) ? fisheye_distortion(c->dist, theta) / theta : K(1.0);
            ru = x * scale * fx + cx;
            rv = y * scale * fy + cy;
        }
        out[2 * idx] = normalized_range ? ru : ru * K(2.0) - K(1.0);
        out[2 * idx + 1] = normalized_range ? rv : rv * K(2.0) - K(1.0);
    }
}

void orc_camera_rays(const orc_camera *c, int width, int height, int world_space, int normalized,
                     real *ray_o, real *ray_d, uint8_t *valid) {
    for (int idx = 0; idx < width * height; ++idx) {
        const int px = idx % width, py = idx / width;
        const real u = ((real)px + K(0.5)) / (real)width;
        const real v = (c->kind == ORC_LIDAR) ? c->beam_v[py] : ((real)py + K(0.5)) / (real)height;
        v3 ray = pixel_to_camera_ray(c, u, v);
        if (normalized) ray = normalize3(ray);
        v3 o = V3(0, 0, 0);
        if (world_space) {
            /* camera.h:101-103,125-131: pose at the pixel's time delta, q = exp(w dt) * q0, t = t0 + v dt */
            const real dt = c->trigger_time + (u * c->rolling[0] + v * c->rolling[1]) - c->pose_time;
            real w1, dw1; v3 xyz1, dxyz1;
            jac_quat_from_axis_angle(ld3(c->w), dt, &w1, &xyz1, &dw1, &dxyz1);
            const real w2 = c->q[0];
            const v3 xyz2 = V3(c->q[1], c->q[2], c->q[3]);
            const real qw = w1 * w2 - dot3(xyz1, xyz2);
            const v3 qv = add3(add3(scl3(xyz2, w1), scl3(xyz1, w2)), cross3(xyz1, xyz2));
            o = add3(ld3(c->t), scl3(ld3(c->v), dt));
            ray = quat_apply(qw, qv, ray);
        }
        ray_o[3 * idx] = o.x; ray_o[3 * idx + 1] = o.y; ray_o[3 * idx + 2] = o.z;
        ray_d[3 * idx] = ray.x; ray_d[3 * idx + 1] = ray.y; ray_d[3 * idx + 2] = ray.z;
        if (valid) valid[idx] = (uint8_t)ray_valid(c, u, v);
    }
}

/* Backward of orc_camera_rays w.r.t. the camera: camera_ray_backward_kernel_cuda
 * (ray_kernels.h:61-161), restated for the pose model of orc_camera_rays. Gradients are summed
 * over pixels (in double) into out[orc_grad_elements(kind)] = q(4) t(3) v(3) w(3) rolling(2)
 * trigger_time pose_time, then the model's tensors: impl(4) for pinhole / spherical / lidar,
 * f c(4) dist(8) max_radius_sq(1) for distorted, f c(4) dist(4) for fisheye -- the camera's tensor
 * order (camera.h:144, perspective.cu:8, spherical.h:35, distorted_perspective.cu:8,
 * fisheye_opencv.cu:7). d_ray_o may
 * be NULL. Only the pinhole model has an intrinsics gradient (perspective.cu:19-33); the spherical
 * and lidar models inherit the empty one (base_camera_impl.h:19-22). */
/* Camera gradient length: the 17 pose / timing values and the model's own tensors
 * (perspective.cu:8, spherical.h:35, distorted_perspective.cu:8, fisheye_opencv.cu:7) */
int orc_grad_elements(int kind) {
    return kind == ORC_DISTORTED ? 30 : kind == ORC_FISHEYE ? 25 : 21;
}

void orc_camera_rays_bwd(const orc_camera *c, int width, int height, int world_space, int normalized,
                         const real *d_ray_o, const real *d_ray_d, real *out) {
    double acc[32];
    for (int k = 0; k < 32; ++k) acc[k] = 0.0;
    for (int idx = 0; idx < width * height; ++idx) {
        const int px = idx % width, py = idx / width;
        const real u = ((real)px + K(0.5)) / (real)width;
        const real v = (c->kind == ORC_LIDAR) ? c->beam_v[py] : ((real)py + K(0.5)) / (real)height;
        const v3 r = pixel_to_camera_ray(c, u, v);
        const v3 n = normalized ? normalize3(r) : r;
        const v3 gd = ld3(d_ray_d + 3 * idx);
        const v3 go = d_ray_o ? ld3(d_ray_o + 3 * idx) : V3(0, 0, 0);
        v3 dn = gd;
        if (world_space) {
            const real dt = c->trigger_time + (u * c->rolling[0] + v * c->rolling[1]) - c->pose_time;
            const v3 w = ld3(c->w);
            real w1, dw1; v3 xyz1, dxyz1;
            jac_quat_from_axis_angle(w, dt, &w1, &xyz1, &dw1, &dxyz1);
            const real w2 = c->q[0];
            const v3 xyz2 = V3(c->q[1], c->q[2], c->q[3]);
            const real qw = w1 * w2 - dot3(xyz1, xyz2);
            const v3 qv = add3(add3(scl3(xyz2, w1), scl3(xyz1, w2)), cross3(xyz1, xyz2));
            /* ray_o = t0 + v dt */
            real d_dt = dot3(go, ld3(c->v));
            acc[4] += go.x; acc[5] += go.y; acc[6] += go.z;
            acc[7] += dt * go.x; acc[8] += dt * go.y; acc[9] += dt * go.z;
            /* ray_d = n + 2 (qw (qv x n) + qv x (qv x n)) */
            dn = add3(gd, scl3(add3(scl3(cross3(qv, gd), -qw), cross3(qv, cross3(qv, gd))), K(2.0)));
            const real d_qw = K(2.0) * dot3(gd, cross3(qv, n));
            const v3 d_qv = add3(add3(scl3(cross3(n, gd), K(2.0) * qw), scl3(n, K(2.0) * dot3(gd, qv))),
                                 sub3(scl3(gd, K(2.0) * dot3(qv, n)), scl3(qv, K(4.0) * dot3(gd, n))));
            /* q = (w1, xyz1) (x) (w2, xyz2) */
            const real d_w1 = d_qw * w2 + dot3(d_qv, xyz2);
            const v3 d_xyz1 = add3(add3(scl3(xyz2, -d_qw), scl3(d_qv, w2)), cross3(xyz2, d_qv));
            const real d_w2 = d_qw * w1 + dot3(d_qv, xyz1);
            const v3 d_xyz2 = add3(add3(scl3(xyz1, -d_qw), scl3(d_qv, w1)), cross3(d_qv, xyz1));
            acc[0] += d_w2; acc[1] += d_xyz2.x; acc[2] += d_xyz2.y; acc[3] += d_xyz2.z;
            /* (w1, xyz1) = (cos(theta/2), w dt sigma), theta = |w| |dt|, sigma = sin(theta/2) / theta */
            d_dt += d_w1 * dw1 + dot3(d_xyz1, dxyz1);
            const real wn = SQRT(dot3(w, w));
            const real theta = wn * FABS(dt);
            real sigma, kappa;  /* kappa = dt |dt| sigma'(theta) / |w| */
            if (theta < K(1e-2)) {
                sigma = K(0.5) - theta * theta * (K(1.0) / K(48.0));
                kappa = -dt * dt * dt / K(24.0);
            } else {
                const real sh = SIN(K(0.5) * theta), ch = COS(K(0.5) * theta);
                sigma = sh / theta;
                kappa = dt * FABS(dt) * (K(0.5) * theta * ch - sh) / (theta * theta * wn);
            }
            const v3 d_w = add3(add3(scl3(w, -d_w1 * dt * dt * sigma * K(0.5)), scl3(d_xyz1, dt * sigma)),
                                scl3(w, kappa * dot3(d_xyz1, w)));
            acc[10] += d_w.x; acc[11] += d_w.y; acc[12] += d_w.z;
            /* dt = trigger_time + u rolling.x + v rolling.y - pose_time */
            acc[13] += d_dt * u; acc[14] += d_dt * v;
            acc[15] += d_dt; acc[16] -= d_dt;
        }
        v3 dr = dn;
        if (normalized) {  /* normalize backward */
            const real il = K(1.0) / SQRT(dot3(r, r));
            dr = scl3(sub3(dn, scl3(n, dot3(n, dn))), il);
        }
        if (c->kind == ORC_PINHOLE) {  /* perspective.cu:19-33 */
            const real ifx = K(1.0) / c->impl[0], ify = K(1.0) / c->impl[1];
            acc[17] += -dr.x * (u - c->impl[2]) * ifx * ifx;
            acc[18] += -dr.y * (v - c->impl[3]) * ify * ify;
            acc[19] += -dr.x * ifx;
            acc[20] += -dr.y * ify;
        } else if (c->kind == ORC_DISTORTED) {
            /* distorted_perspective.cu:121-188: re-solve, then the implicit-function gradient at the
             * solution: g_d = J^-T (dr.x, dr.y) (J symmetric; d / scale where J is nearly singular),
             * dL/dk = -g_d . dD/dk */
            const real ifx = K(1.0) / c->impl[0], ify = K(1.0) / c->impl[1];
            const v2 ud = {(u - c->impl[2]) * ifx, (v - c->impl[3]) * ify};
            dist_state st;
            const v2 uc = undistort_uv(c->dist, ud, &st);
            st = distortion_state(c->dist, uc.x, uc.y);
            const real det = st.juu * st.jvv - st.juv * st.juv;
            real gx, gy;
            if (FABS(det) <= DIST_MIN_DET) {
                gx = dr.x / st.scale; gy = dr.y / st.scale;
            } else {
                gx = (st.jvv * dr.x - st.juv * dr.y) / det;
                gy = (st.juu * dr.y - st.juv * dr.x) / det;
            }
            acc[17] += -gx * ud.x * ifx;
            acc[18] += -gy * ud.y * ify;
            acc[19] += -gx * ifx;
            acc[20] += -gy * ify;
            const real r2 = uc.x * uc.x + uc.y * uc.y, r4 = r2 * r2, r6 = r4 * r2;
            const real d_rad = -(gx * uc.x + gy * uc.y) / st.denom;
            const real d_rad_den = -d_rad * st.scale;
            acc[21] += d_rad * r2;
            acc[22] += d_rad * r4;
            acc[23] += -(gx * K(2.0) * uc.x * uc.y + gy * (r2 + K(2.0) * uc.y * uc.y));
            acc[24] += -(gx * (r2 + K(2.0) * uc.x * uc.x) + gy * K(2.0) * uc.x * uc.y);
            acc[25] += d_rad * r6;
            acc[26] += d_rad_den * r2;
            acc[27] += d_rad_den * r4;
            acc[28] += d_rad_den * r6;
        } else if (c->kind == ORC_FISHEYE) {
            /* fisheye_opencv.cu:74-136: theta(delta, k) implicit through theta_d(theta, k) = delta */
            const real x = (u - c->impl[2]) / c->impl[0], y = (v - c->impl[3]) / c->impl[1];
            const real delta = SQRT(x * x + y * y);
            real residual;
            const real theta = fisheye_solve_theta(c->dist, delta, &residual);
            const real deriv = fisheye_distortion_deriv(c->dist, theta);
            if (theta > K(0) && delta > K(1e-8) && FABS(residual) < K(1e-5) && deriv > K(1e-3)) {
                const real st = SIN(theta), ct = COS(theta);
                const real inv_delta = K(1.0) / delta;
                const real sf = st * inv_delta;
                const real d_s = dr.x * x + dr.y * y;
                const real d_theta = d_s * ct * inv_delta - dr.z * st;
                const real dts = d_theta / deriv;
                const real t2 = theta * theta, t3 = t2 * theta;
                acc[21] += -dts * t3;
                acc[22] += -dts * t3 * t2;
                acc[23] += -dts * t3 * t2 * t2;
                acc[24] += -dts * t3 * t2 * t2 * t2;
                const real d_delta = -d_s * st * inv_delta * inv_delta + dts;
                const real gx = sf * dr.x + d_delta * x * inv_delta;
                const real gy = sf * dr.y + d_delta * y * inv_delta;
                acc[17] += -gx * x / c->impl[0];
                acc[18] += -gy * y / c->impl[1];
                acc[19] += -gx / c->impl[0];
                acc[20] += -gy / c->impl[1];
            }
        }
    }
    const int ne = orc_grad_elements(c->kind);
    for (int k = 0; k < ne; ++k) out[k] = (real)acc[k];
}

/* pixel_time[_delta][_from_uv] backward (time_kernels.h:123-330): with uv NULL the n = width *
 * height pixels' own uv. out as orc_camera_rays_bwd: trigger_time += sum g, rolling += sum g uv,
 * pose_time -= sum g for the delta variants; d_uv[i] = g_i rolling when uv is given. */
void orc_pixel_time_bwd(const orc_camera *c, int width, int height, const real *uv, long n, int delta,
                        const real *grad, real *out, real *d_uv) {
    double g0 = 0.0, gu = 0.0, gv = 0.0;
    if (!uv) n = (long)width * height;
    for (long i = 0; i < n; ++i) {
        real u, v;
        if (uv) {
            u = uv[2 * i]; v = uv[2 * i + 1];
            if (d_uv) { d_uv[2 * i] = grad[i] * c->rolling[0]; d_uv[2 * i + 1] = grad[i] * c->rolling[1]; }
        } else {
            const int px = (int)(i % width), py = (int)(i / width);
            u = ((real)px + K(0.5)) / (real)width;
            v = (c->kind == ORC_LIDAR) ? c->beam_v[py] : ((real)py + K(0.5)) / (real)height;
        }
        g0 += grad[i]; gu += (double)grad[i] * u; gv += (double)grad[i] * v;
    }
    for (int k = 0; k < orc_grad_elements(c->kind); ++k) out[k] = 0;
    out[13] = (real)gu; out[14] = (real)gv; out[15] = (real)g0;
    if (delta) out[16] = (real)-g0;
}

/* ------------------------------------------------------------------------- */
/* Spherical harmonics: csrc/color/sh_fwd.cu:16-159, sh_bwd.cu:20-315         */
/* ------------------------------------------------------------------------- */
static real sh_eval(int deg, v3 dir, const real *cf, const real *dc, long bo) {
    /* sh_fwd.cu:16-115; cf points at band 0 (or band 1 when dc != NULL) of one channel */
    real result;
    const real *c;
    if (dc) { result = K(0.2820947917738781) * dc[0]; c = cf - bo; }
    else { result = K(0.2820947917738781) * cf[0]; c = cf; }
    if (deg >= 1) {
        const real x = dir.x, y = dir.y, z = dir.z;
        result += K(0.48860251190292) * (-y * c[bo] + z * c[2 * bo] - x * c[3 * bo]);
        if (deg >= 2) {
            const real z2 = z * z;
            const real fTmp0B = K(-1.092548430592079) * z;
            const real fC1 = x * x - y * y, fS1 = K(2) * x * y;
            const real p6 = K(0.9461746957575601) * z2 - K(0.3153915652525201);
            const real p7 = fTmp0B * x, p5 = fTmp0B * y;
            const real p8 = K(0.5462742152960395) * fC1, p4 = K(0.5462742152960395) * fS1;
            result += p4 * c[4 * bo] + p5 * c[5 * bo] + p6 * c[6 * bo] + p7 * c[7 * bo] + p8 * c[8 * bo];
            if (deg >= 3) {
                const real fTmp0C = K(-2.285228997322329) * z2 + K(0.4570457994644658);
                const real fTmp1B = K(1.445305721320277) * z;
                const real fC2 = x * fC1 - y * fS1, fS2 = x * fS1 + y * fC1;
                const real p12 = z * (K(1.865881662950577) * z2 - K(1.119528997770346));
                const real p13 = fTmp0C * x, p11 = fTmp0C * y;
                const real p14 = fTmp1B * fC1, p10 = fTmp1B * fS1;
                const real p15 = K(-0.5900435899266435) * fC2, p9 = K(-0.5900435899266435) * fS2;
                result += p9 * c[9 * bo] + p10 * c[10 * bo] + p11 * c[11 * bo] + p12 * c[12 * bo] +
                          p13 * c[13 * bo] + p14 * c[14 * bo] + p15 * c[15 * bo];
                if (deg >= 4) {
                    const real fTmp0D = z * (K(-4.683325804901025) * z2 + K(2.007139630671868));
                    const real fTmp1C = K(3.31161143515146) * z2 - K(0.47308734787878);
                    const real fTmp2B = K(-1.770130769779931) * z;
                    const real fC3 = x * fC2 - y * fS2, fS3 = x * fS2 + y * fC2;
                    const real p20 = K(1.984313483298443) * z * p12 - K(1.006230589874905) * p6;
                    const real p21 = fTmp0D * x, p19 = fTmp0D * y;
                    const real p22 = fTmp1C * fC1, p18 = fTmp1C * fS1;
                    const real p23 = fTmp2B * fC2, p17 = fTmp2B * fS2;
                    const real p24 = K(0.6258357354491763) * fC3, p16 = K(0.6258357354491763) * fS3;
                    result += p16 * c[16 * bo] + p17 * c[17 * bo] + p18 * c[18 * bo] + p19 * c[19 * bo] +
                              p20 * c[20 * bo] + p21 * c[21 * bo] + p22 * c[22 * bo] + p23 * c[23 * bo] +
                              p24 * c[24 * bo];
                }
            }
        }
    }
    return result;
}

static inline int mask_bit(const uint32_t *mask, long idx) {
    return mask ? ((mask[idx / 32] & (1u << (idx % 32))) != 0) : 1;
}

/* spherical_harmonics_fused_fwd: sh_fwd.cu:119-245. out must be zero-initialised by the caller
 * (masked Gaussians keep the caller's values, sh_fwd.cu:136, 212). */
void orc_sh_fwd(int deg, const real *origin, int n, int dim, const real *pos, const real *coeffs,
                const real *dc, const uint32_t *mask, int layout_3kn, real *out) {
    const v3 o = ld3(origin);
#pragma omp parallel for schedule(static)
    for (long i = 0; i < n; ++i) {
        if (!mask_bit(mask, i)) continue;
        const v3 dir = normalize3(sub3(ld3(pos + 3 * i), o));
        for (int ch = 0; ch < 3; ++ch) {
            if (layout_3kn) {
                const real *cf = coeffs + (long)ch * n * dim + i;
                const real *dcp = dc ? dc + (long)ch * n + i : NULL;
                out[3 * i + ch] = sh_eval(deg, dir, cf, dcp, n) + K(0.5);
            } else {
                const real *cf = coeffs + i * dim * 3 + ch;
                const real *dcp = dc ? dc + i * 3 + ch : NULL;
                out[3 * i + ch] = sh_eval(deg, dir, cf, dcp, 3) + K(0.5);
            }
        }
    }
}

static void sh_eval_bwd(int deg, v3 dir, const real *cf, long bo, real d_out, real *dcf, real *ddc,
                        v3 *d_dir) {
    /* sh_bwd.cu:20-247 */
    const real *c; real *dc;
    if (ddc) { ddc[0] = K(0.2820947917738781) * d_out; c = cf - bo; dc = dcf - bo; }
    else { dcf[0] = K(0.2820947917738781) * d_out; c = cf; dc = dcf; }
    if (deg < 1) return;
    const real x = dir.x, y = dir.y, z = dir.z;
    dc[bo] = K(-0.48860251190292) * y * d_out;
    dc[2 * bo] = K(0.48860251190292) * z * d_out;
    dc[3 * bo] = K(-0.48860251190292) * x * d_out;
    d_dir->x += K(-0.48860251190292) * c[3 * bo] * d_out;
    d_dir->y += K(-0.48860251190292) * c[1 * bo] * d_out;
    d_dir->z += K(0.48860251190292) * c[2 * bo] * d_out;
    if (deg < 2) return;
    const real z2 = z * z;
    const real fTmp0B = K(-1.092548430592079) * z;
    const real fC1 = x * x - y * y, fS1 = K(2) * x * y;
    const real p6 = K(0.9461746957575601) * z2 - K(0.3153915652525201);
    const real p7 = fTmp0B * x, p5 = fTmp0B * y;
    const real p8 = K(0.5462742152960395) * fC1, p4 = K(0.5462742152960395) * fS1;
    dc[4 * bo] = p4 * d_out; dc[5 * bo] = p5 * d_out; dc[6 * bo] = p6 * d_out;
    dc[7 * bo] = p7 * d_out; dc[8 * bo] = p8 * d_out;
    const real fTmp0B_z = K(-1.092548430592079);
    const real fC1_x = K(2) * x, fC1_y = K(-2) * y, fS1_x = K(2) * y, fS1_y = K(2) * x;
    const real p6_z = K(2) * K(0.9461746957575601) * z;
    const real p7_x = fTmp0B, p7_z = fTmp0B_z * x, p5_y = fTmp0B, p5_z = fTmp0B_z * y;
    const real p8_x = K(0.5462742152960395) * fC1_x, p8_y = K(0.5462742152960395) * fC1_y;
    const real p4_x = K(0.5462742152960395) * fS1_x, p4_y = K(0.5462742152960395) * fS1_y;
    d_dir->x += d_out * (p4_x * c[4 * bo] + p8_x * c[8 * bo] + p7_x * c[7 * bo]);
    d_dir->y += d_out * (p4_y * c[4 * bo] + p8_y * c[8 * bo] + p5_y * c[5 * bo]);
    d_dir->z += d_out * (p6_z * c[6 * bo] + p7_z * c[7 * bo] + p5_z * c[5 * bo]);
    if (deg < 3) return;
    const real fTmp0C = K(-2.285228997322329) * z2 + K(0.4570457994644658);
    const real fTmp1B = K(1.445305721320277) * z;
    const real fC2 = x * fC1 - y * fS1, fS2 = x * fS1 + y * fC1;
    const real p12 = z * (K(1.865881662950577) * z2 - K(1.119528997770346));
    const real p13 = fTmp0C * x, p11 = fTmp0C * y;
    const real p14 = fTmp1B * fC1, p10 = fTmp1B * fS1;
    const real p15 = K(-0.5900435899266435) * fC2, p9 = K(-0.5900435899266435) * fS2;
    dc[9 * bo] = p9 * d_out; dc[10 * bo] = p10 * d_out; dc[11 * bo] = p11 * d_out;
    dc[12 * bo] = p12 * d_out; dc[13 * bo] = p13 * d_out; dc[14 * bo] = p14 * d_out;
    dc[15 * bo] = p15 * d_out;
    const real fTmp0C_z = K(-2.285228997322329) * K(2) * z;
    const real fTmp1B_z = K(1.445305721320277);
    const real fC2_x = fC1 + x * fC1_x - y * fS1_x;
    const real fC2_y = x * fC1_y - fS1 - y * fS1_y;
    const real fS2_x = fS1 + x * fS1_x + y * fC1_x;
    const real fS2_y = x * fS1_y + fC1 + y * fC1_y;
    const real p12_z = K(3) * K(1.865881662950577) * z2 - K(1.119528997770346);
    const real p13_x = fTmp0C, p13_z = fTmp0C_z * x, p11_y = fTmp0C, p11_z = fTmp0C_z * y;
    const real p14_x = fTmp1B * fC1_x, p14_y = fTmp1B * fC1_y, p14_z = fTmp1B_z * fC1;
    const real p10_x = fTmp1B * fS1_x, p10_y = fTmp1B * fS1_y, p10_z = fTmp1B_z * fS1;
    const real p15_x = K(-0.5900435899266435) * fC2_x, p15_y = K(-0.5900435899266435) * fC2_y;
    const real p9_x = K(-0.5900435899266435) * fS2_x, p9_y = K(-0.5900435899266435) * fS2_y;
    d_dir->x += d_out * (p9_x * c[9 * bo] + p15_x * c[15 * bo] + p10_x * c[10 * bo] +
                         p14_x * c[14 * bo] + p13_x * c[13 * bo]);
    d_dir->y += d_out * (p9_y * c[9 * bo] + p15_y * c[15 * bo] + p10_y * c[10 * bo] +
                         p14_y * c[14 * bo] + p11_y * c[11 * bo]);
    d_dir->z += d_out * (p12_z * c[12 * bo] + p13_z * c[13 * bo] + p11_z * c[11 * bo] +
                         p14_z * c[14 * bo] + p10_z * c[10 * bo]);
    if (deg < 4) return;
    const real fTmp0D = z * (K(-4.683325804901025) * z2 + K(2.007139630671868));
    const real fTmp1C = K(3.31161143515146) * z2 - K(0.47308734787878);
    const real fTmp2B = K(-1.770130769779931) * z;
    const real fC3 = x * fC2 - y * fS2, fS3 = x * fS2 + y * fC2;
    const real p20 = K(1.984313483298443) * z * p12 + K(-1.006230589874905) * p6;
    const real p21 = fTmp0D * x, p19 = fTmp0D * y;
    const real p22 = fTmp1C * fC1, p18 = fTmp1C * fS1;
    const real p23 = fTmp2B * fC2, p17 = fTmp2B * fS2;
    const real p24 = K(0.6258357354491763) * fC3, p16 = K(0.6258357354491763) * fS3;
    dc[16 * bo] = p16 * d_out; dc[17 * bo] = p17 * d_out; dc[18 * bo] = p18 * d_out;
    dc[19 * bo] = p19 * d_out; dc[20 * bo] = p20 * d_out; dc[21 * bo] = p21 * d_out;
    dc[22 * bo] = p22 * d_out; dc[23 * bo] = p23 * d_out; dc[24 * bo] = p24 * d_out;
    const real fTmp0D_z = K(3) * K(-4.683325804901025) * z2 + K(2.007139630671868);
    const real fTmp1C_z = K(2) * K(3.31161143515146) * z;
    const real fTmp2B_z = K(-1.770130769779931);
    const real fC3_x = fC2 + x * fC2_x - y * fS2_x;
    const real fC3_y = x * fC2_y - fS2 - y * fS2_y;
    const real fS3_x = fS2 + y * fC2_x + x * fS2_x;
    const real fS3_y = x * fS2_y + fC2 + y * fC2_y;
    const real p20_z = K(1.984313483298443) * (p12 + z * p12_z) + K(-1.006230589874905) * p6_z;
    const real p21_x = fTmp0D, p21_z = fTmp0D_z * x, p19_y = fTmp0D, p19_z = fTmp0D_z * y;
    const real p22_x = fTmp1C * fC1_x, p22_y = fTmp1C * fC1_y, p22_z = fTmp1C_z * fC1;
    const real p18_x = fTmp1C * fS1_x, p18_y = fTmp1C * fS1_y, p18_z = fTmp1C_z * fS1;
    const real p23_x = fTmp2B * fC2_x, p23_y = fTmp2B * fC2_y, p23_z = fTmp2B_z * fC2;
    const real p17_x = fTmp2B * fS2_x, p17_y = fTmp2B * fS2_y, p17_z = fTmp2B_z * fS2;
    const real p24_x = K(0.6258357354491763) * fC3_x, p24_y = K(0.6258357354491763) * fC3_y;
    const real p16_x = K(0.6258357354491763) * fS3_x, p16_y = K(0.6258357354491763) * fS3_y;
    d_dir->x += d_out * (p16_x * c[16 * bo] + p24_x * c[24 * bo] + p17_x * c[17 * bo] +
                         p23_x * c[23 * bo] + p18_x * c[18 * bo] + p22_x * c[22 * bo] +
                         p21_x * c[21 * bo]);
    d_dir->y += d_out * (p16_y * c[16 * bo] + p24_y * c[24 * bo] + p17_y * c[17 * bo] +
                         p23_y * c[23 * bo] + p18_y * c[18 * bo] + p22_y * c[22 * bo] +
                         p19_y * c[19 * bo]);
    d_dir->z += d_out * (p20_z * c[20 * bo] + p21_z * c[21 * bo] + p19_z * c[19 * bo] +
                         p22_z * c[22 * bo] + p18_z * c[18 * bo] + p23_z * c[23 * bo] +
                         p17_z * c[17 * bo]);
}

/* spherical_harmonics_fused_bwd: sh_bwd.cu:250-376. Outputs must be zero-initialised.
 * d_origin[3] = -sum of d_positions (sh_bwd.cu:306, 375). */
void orc_sh_bwd(int deg, const real *origin, int n, int dim, const real *pos, const real *coeffs,
                const uint32_t *mask, int layout_3kn, const real *d_output, int has_dc,
                real *d_coeffs, real *d_dc, real *d_pos, real *d_origin) {
    const v3 o = ld3(origin);
    double so[3] = {0, 0, 0};
    for (long i = 0; i < n; ++i) {
        if (!mask_bit(mask, i)) continue;
        const v3 diff = sub3(ld3(pos + 3 * i), o);
        const v3 dir = normalize3(diff);
        v3 dsum = V3(0, 0, 0);
        for (int ch = 0; ch < 3; ++ch) {
            const real d_out = d_output[3 * i + ch];
            v3 ddir = V3(0, 0, 0);
            if (layout_3kn) {
                sh_eval_bwd(deg, dir, coeffs + (long)ch * n * dim + i, n, d_out,
                            d_coeffs + (long)ch * n * dim + i, has_dc ? d_dc + (long)ch * n + i : NULL,
                            &ddir);
            } else {
                sh_eval_bwd(deg, dir, coeffs + i * dim * 3 + ch, 3, d_out, d_coeffs + i * dim * 3 + ch,
                            has_dc ? d_dc + i * 3 + ch : NULL, &ddir);
            }
            /* normalize_bwd (toast): d_v = (d_n - (d_n . n) n) / |v| */
            const real il = K(1.0) / SQRT(dot3(diff, diff));
            const real il3 = il * il * il;
            const v3 dd = sub3(scl3(ddir, il), scl3(diff, il3 * dot3(ddir, diff)));
            dsum = add3(dsum, dd);
        }
        d_pos[3 * i] += dsum.x; d_pos[3 * i + 1] += dsum.y; d_pos[3 * i + 2] += dsum.z;
        so[0] -= dsum.x; so[1] -= dsum.y; so[2] -= dsum.z;
    }
    d_origin[0] = (real)so[0]; d_origin[1] = (real)so[1]; d_origin[2] = (real)so[2];
}

/* ------------------------------------------------------------------------- */
/* Tile binning                                                              */
/* ------------------------------------------------------------------------- */
static inline int imin(int a, int b) { return a < b ? a : b; }
static inline int imax(int a, int b) { return a > b ? a : b; }

static void regular_rect(const float *means2d, const float *radii, long i, float tsx, float tsy,
                         int ntx, int nty, int *tmin_x, int *tmin_y, int *tmax_x, int *tmax_y) {
    /* regular_tiling.cu:41-56: float32 division by tile size, floor/ceil, clamp to [0, n] */
    const float mx = means2d[2 * i] / tsx, my = means2d[2 * i + 1] / tsy;
    const float rx = radii[2 * i] / tsx, ry = radii[2 * i + 1] / tsy;
    *tmin_x = imin(ntx, imax(0, (int)floorf(mx - rx)));
    *tmin_y = imin(nty, imax(0, (int)floorf(my - ry)));
    *tmax_x = imin(ntx, imax(0, (int)ceilf(mx + rx)));
    *tmax_y = imin(nty, imax(0, (int)ceilf(my + ry)));
}

/* isect_tiles_kernel<true>: regular_tiling.cu:13-69 (count pass). Binning is always float32,
 * whatever REAL is, because it must be bit-exact with the reference. */
void orc_isect_regular_count(int n, const float *means2d, const float *radii, int width, int height,
                             int tsx, int tsy, int32_t *tiles_per_gauss) {
    const int ntx = (width + tsx - 1) / tsx, nty = (height + tsy - 1) / tsy;
    for (long i = 0; i < n; ++i) {
        if (radii[2 * i] <= 0 || radii[2 * i + 1] <= 0) { tiles_per_gauss[i] = 0; continue; }
        int a, b, c, d;
        regular_rect(means2d, radii, i, (float)tsx, (float)tsy, ntx, nty, &a, &b, &c, &d);
        tiles_per_gauss[i] = (d - b) * (c - a);
    }
}

static inline int64_t make_key(int64_t tile_id, float depth) {
    int32_t bits; memcpy(&bits, &depth, 4);
    return (tile_id << 32) | (int64_t)bits;   /* tiling_common.cuh:37, 62, 68: sign-extended */
}

/* isect_tiles_kernel<false> + fill_tiles_exclusive: regular_tiling.cu:58-64, tiling_common.cuh:50-73 */
void orc_isect_regular_fill(int n, const float *means2d, const float *radii, const float *depths,
                            int width, int height, int tsx, int tsy, const int64_t *cum,
                            int64_t *isect_ids, int32_t *flatten_ids) {
    const int ntx = (width + tsx - 1) / tsx, nty = (height + tsy - 1) / tsy;
    for (long i = 0; i < n; ++i) {
        if (radii[2 * i] <= 0 || radii[2 * i + 1] <= 0) continue;
        int a, b, c, d;
        regular_rect(means2d, radii, i, (float)tsx, (float)tsy, ntx, nty, &a, &b, &c, &d);
        if ((d - b) * (c - a) <= 0) continue;
        int64_t off = i > 0 ? cum[i - 1] : 0;
        for (int y = b; y < d; ++y)
            for (int x = a; x < c; ++x) {
                isect_ids[off] = make_key((int64_t)y * ntx + x, depths[i]);
                flatten_ids[off] = (int32_t)i;
                ++off;
            }
    }
}

/* phm_lidar_tiling.cu:16-91 */
static void find_bounds_increasing(float vmin, float vmax, int n, const float *values, int *tmin, int *tmax) {
    int i = 0;
    while (i < n && values[i] < vmin) ++i;
    *tmin = imin(imax(i - 1, 0), n - 1);
    while (i < n && values[i] < vmax) ++i;
    *tmax = imin(imax(i - 1, 0), n - 1);
}

static void tile_limits_irregular(float mx, float my, float rx, float ry, float u_min, float u_max,
                                  float u_per_tile, int n_elev, const float *elev, int *tmin_x,
                                  int *tmin_y, int *tmax_x, int *tmax_y, int *num) {
    *tmin_x = 0; *tmin_y = 0; *tmax_x = -1; *tmax_y = -1;
    const float lo = fmaxf(mx - rx, u_min), hi = fminf(mx + rx, u_max);
    if (hi <= lo) return;
    *tmin_x = (int)floorf(lo / u_per_tile);
    *tmax_x = (int)ceilf(hi / u_per_tile) - 1;
    find_bounds_increasing(my - ry, my + ry, n_elev, elev, tmin_y, tmax_y);
    *num += (*tmax_y - *tmin_y + 1) * (*tmax_x - *tmin_x + 1);
}

/* phm_spherical_tiling.cu:15-45 */
static void tile_limits_regular(float mx, float my, float rx, float ry, float u_min, float u_max,
                                float u_per_tile, int n_v, float v_per_tile, int *tmin_x, int *tmin_y,
                                int *tmax_x, int *tmax_y, int *num) {
    *tmin_x = 0; *tmin_y = 0; *tmax_x = 0; *tmax_y = 0;
    const float lo = fmaxf(mx - rx, u_min), hi = fminf(mx + rx, u_max);
    if (hi <= lo) return;
    *tmin_x = (int)floorf(lo / u_per_tile);
    *tmin_y = imin(n_v, imax(0, (int)floorf((my - ry) / v_per_tile)));
    *tmax_x = (int)ceilf(hi / u_per_tile);
    *tmax_y = imin(n_v, imax(0, (int)ceilf((my + ry) / v_per_tile)));
    *num += (*tmax_y - *tmin_y) * (*tmax_x - *tmin_x);
}

/* Float32 decision margins of one span's tile range (test diagnostics): lo / hi against u_min /
 * u_max and the nearest azimuth tile boundary, the span's emptiness, and the v extent against the
 * elevation boundaries (lidar) or the nearest v tile boundary. ex / ey bound the float32 error of the
 * normalised centre plus radius. */
static void span_margins(float mx, float my, float rx, float ry, float u_min, float u_max, float u_per_tile,
                         int lidar, int n_el, const float *elev, float v_per_tile, real ex, real ey) {
    if (!tl_mg) return;
    const real xs[2] = {(real)mx - rx, (real)mx + rx}, ys[2] = {(real)my - ry, (real)my + ry};
    const real lo = FMAX(xs[0], u_min), hi = FMIN(xs[1], u_max);
    mg_note(xs[0] - u_min, ex); mg_note(xs[1] - u_max, ex);
    mg_note(hi - lo, K(2) * ex);
    if (hi <= lo) return;
    for (int k = 0; k < 2; ++k) {
        /* an end clamped to u_min / u_max is that bound exactly on every implementation */
        const int clamped = k ? xs[1] >= u_max : xs[0] <= u_min;
        const real t = (k ? hi : lo) / u_per_tile;
        if (!clamped) mg_note((t - FLOOR(t + K(0.5))) * u_per_tile, ex);
        if (lidar) {
            for (int j = 0; j < n_el; ++j) mg_note(ys[k] - elev[j], ey);
        } else {
            const real tv = ys[k] / v_per_tile;
            mg_note((tv - FLOOR(tv + K(0.5))) * v_per_tile, ey);
        }
    }
}

/* The float32 camera for the seam re-projection inside the lidar/spherical binning. */
typedef struct {
    orc_camera cam;
    float ut[4];
} orc_bin_ctx;

/* isect_lidar_tiles_kernel (phm_lidar_tiling.cu:96-234) and isect_spherical_tiles_kernel
 * (phm_spherical_tiling.cu:47-174). kind: 0 = lidar (irregular v grid, inclusive),
 * 1 = spherical (regular grid, exclusive). cum == NULL selects the count pass. */
void orc_isect_spherical_family(int kind, const orc_camera *cam, const real *ut, int n,
                                const real *points, const real *vel, const real *scale,
                                const real *quat, const real *opacity, const uint8_t *flags,
                                const float *means2d, const float *radii, const float *depths,
                                const float *elev, int n_elev, int tsx, int tsy, float img_w,
                                float img_h, const int64_t *cum, int32_t *tiles_per_gauss,
                                int64_t *isect_ids, int32_t *flatten_ids, real *seam_margin) {
    const int lidar = kind == 0;
    int n_az, n_el;
    float u_per_tile, v_per_tile = 0;
    if (lidar) {
        n_az = ((int)img_w + tsx - 1) / tsx;
        n_el = n_elev;
        u_per_tile = (float)tsx / img_w;
    } else {
        n_az = (int)ceilf(img_w / (float)tsx);
        n_el = (int)ceilf(img_h / (float)tsy);
        u_per_tile = (float)tsx / img_w;
        v_per_tile = (float)tsy / img_h;
    }
    const v2 img = {img_w, img_h};
    for (long i = 0; i < n; ++i) {
        const int first = cum == NULL;
        float rx = radii[2 * i], ry = radii[2 * i + 1];
        const int flag = flags[i];
        if (rx <= 0 || ry <= 0 || flag == 0) { if (first) tiles_per_gauss[i] = 0; continue; }
        int a, b, c, d, num = 0;
        int64_t off = 0;
        float u_min = 0.0f, u_max = 1.0f;
        const float u_pose = (float)u_pose_of(cam);
        if (flag == 2) { if (cam->rolling[0] > 0) u_max = u_pose; else u_min = u_pose; }
        float mx = means2d[2 * i] / img_w, my = means2d[2 * i + 1] / img_h;
        rx /= img_w; ry /= img_h;
        if (lidar) tile_limits_irregular(mx, my, rx, ry, u_min, u_max, u_per_tile, n_el, elev, &a, &b, &c, &d, &num);
        else tile_limits_regular(mx, my, rx, ry, u_min, u_max, u_per_tile, n_el, v_per_tile, &a, &b, &c, &d, &num);
        if (!first) {
            off = i > 0 ? cum[i - 1] : 0;
            const int ye = lidar ? d + 1 : d, xe = lidar ? c + 1 : c;
            for (int y = b; y < ye; ++y)
                for (int x = a; x < xe; ++x) {
                    isect_ids[off] = make_key((int64_t)y * n_az + x, depths[i]);
                    flatten_ids[off] = (int32_t)i;
                    ++off;
                }
        }
        if (flag == 2) {
            v3 dl[3];
            ut_deltas(ut[3], quat + 4 * i, scale + 3 * i, dl);
            const real op = opacity ? opacity[i] : K(1.0);
            v2 m2, r2; real depth = 0, udist = 0;
            const v3 pv = vel ? ld3(vel + 3 * i) : V3(0, 0, 0);
            real mg = K(1e30);
            tl_mg = seam_margin ? &mg : NULL;
            const int ok = ut_projection(cam, ORC_MODE_POS, ut, img, K(1e-4), K(0.002), K(1.0),
                                         ld3(points + 3 * i), pv, op, dl, &m2, &r2, &depth, &udist);
            if (ok && tl_mg) {
                const real ex = (tl_ut_err.em + tl_ut_err.rx_err) / img_w + K(4) * F32_U * (FABS(m2.x) / img_w + K(1));
                const real ey = (tl_ut_err.em + tl_ut_err.ry_err) / img_h + K(4) * F32_U * (FABS(m2.y) / img_h + K(1));
                float ulo, uhi;
                if (cam->rolling[0] > 0) { ulo = ceilf(u_pose / u_per_tile) * u_per_tile + 1e-6f; uhi = 1.0f; }
                else { ulo = 0.0f; uhi = floorf(u_pose / u_per_tile) * u_per_tile - 1e-6f; }
                span_margins((float)m2.x / img_w, (float)m2.y / img_h, (float)r2.x / img_w, (float)r2.y / img_h,
                             ulo, uhi, u_per_tile, lidar, n_el, elev, v_per_tile, ex, ey);
            }
            if (seam_margin) seam_margin[i] = mg;
            tl_mg = NULL;
            if (ok) {
                if (cam->rolling[0] > 0) {
                    u_min = ceilf(u_pose / u_per_tile) * u_per_tile + 1e-6f;
                    u_max = 1.0f;
                } else {
                    u_min = 0.0f;
                    u_max = floorf(u_pose / u_per_tile) * u_per_tile - 1e-6f;
                }
                const float m2x = (float)m2.x / img_w, m2y = (float)m2.y / img_h;
                const float r2x = (float)r2.x / img_w, r2y = (float)r2.y / img_h;
                if (lidar) tile_limits_irregular(m2x, m2y, r2x, r2y, u_min, u_max, u_per_tile, n_el, elev, &a, &b, &c, &d, &num);
                else tile_limits_regular(m2x, m2y, r2x, r2y, u_min, u_max, u_per_tile, n_el, v_per_tile, &a, &b, &c, &d, &num);
                if (!first) {
                    const int ye = lidar ? d + 1 : d, xe = lidar ? c + 1 : c;
                    for (int y = b; y < ye; ++y)
                        for (int x = a; x < xe; ++x) {
                            isect_ids[off] = make_key((int64_t)y * n_az + x, (float)depth);
                            flatten_ids[off] = (int32_t)i;
                            ++off;
                        }
                }
            }
        }
        if (first) tiles_per_gauss[i] = num;
    }
}

/* Stable sort of (key, value) pairs by key bits [0, end_bit) -- cub::DeviceRadixSort::SortPairs
 * semantics as used by sort_intersections (tiling_common.cu:102-162). LSD radix, 8-bit digits. */
void orc_sort_pairs(int64_t n, int64_t *keys, int32_t *vals, int end_bit) {
    if (n <= 0) return;
    int64_t *k2 = (int64_t *)malloc(sizeof(int64_t) * n);
    int32_t *v2b = (int32_t *)malloc(sizeof(int32_t) * n);
    int64_t *ks = keys, *kd = k2; int32_t *vs = vals, *vd = v2b;
    const uint64_t mask = end_bit >= 64 ? ~0ull : ((1ull << end_bit) - 1);
    for (int shift = 0; shift < end_bit; shift += 8) {
        int64_t count[257];
        memset(count, 0, sizeof(count));
        for (int64_t i = 0; i < n; ++i) count[(((uint64_t)ks[i] & mask) >> shift & 255) + 1]++;
        for (int b = 0; b < 256; ++b) count[b + 1] += count[b];
        for (int64_t i = 0; i < n; ++i) {
            const int dg = (int)((((uint64_t)ks[i] & mask) >> shift) & 255);
            const int64_t p = count[dg]++;
            kd[p] = ks[i]; vd[p] = vs[i];
        }
        int64_t *tk = ks; ks = kd; kd = tk;
        int32_t *tv = vs; vs = vd; vd = tv;
    }
    if (ks != keys) { memcpy(keys, ks, sizeof(int64_t) * n); memcpy(vals, vs, sizeof(int32_t) * n); }
    free(k2); free(v2b);
}

/* isect_offset_encode_kernel: tiling_common.cu:25-99 (camera id above tile_n_bits, :41-44). */
void orc_offset_encode(int64_t n, const int64_t *isect_ids, int n_tiles, int n_cams, int32_t *offsets) {
    const int total = n_tiles * n_cams;
    if (n == 0) { for (int i = 0; i < total; ++i) offsets[i] = 0; return; }
    const uint32_t tile_n_bits = (uint32_t)floorf(log2f((float)n_tiles)) + 1;
    for (int64_t idx = 0; idx < n; ++idx) {
        const int64_t cur = isect_ids[idx] >> 32;
        const int64_t id_cur = (cur >> tile_n_bits) * n_tiles + (cur & ((1 << tile_n_bits) - 1));
        if (idx == 0) for (int64_t i = 0; i < id_cur + 1; ++i) offsets[i] = 0;
        if (idx == n - 1) for (int64_t i = id_cur + 1; i < total; ++i) offsets[i] = (int32_t)n;
        if (idx > 0) {
            const int64_t prev = isect_ids[idx - 1] >> 32;
            if (prev == cur) continue;
            const int64_t id_prev = (prev >> tile_n_bits) * n_tiles + (prev & ((1 << tile_n_bits) - 1));
            for (int64_t i = id_prev + 1; i < id_cur + 1; ++i) offsets[i] = (int32_t)idx;
        }
    }
}

/* ------------------------------------------------------------------------- */
/* eval3d compositing: csrc/rasterization/eval3d_fwd.cu, eval3d_bwd.cu, utils.h */
/* ------------------------------------------------------------------------- */
static m3 quat_to_rotmat(const real *q) { /* utils.h:61-83 */
    real w = q[0], x = q[1], y = q[2], z = q[3];
    const real inv = K(1.0) / SQRT(x * x + y * y + z * z + w * w);
    x *= inv; y *= inv; z *= inv; w *= inv;
    const real x2 = x * x, y2 = y * y, z2 = z * z, xy = x * y, xz = x * z, yz = y * z;
    const real wx = w * x, wy = w * y, wz = w * z;
    m3 R;
    R.m[0][0] = K(1) - K(2) * (y2 + z2); R.m[0][1] = K(2) * (xy + wz); R.m[0][2] = K(2) * (xz - wy);
    R.m[1][0] = K(2) * (xy - wz); R.m[1][1] = K(1) - K(2) * (x2 + z2); R.m[1][2] = K(2) * (yz + wx);
    R.m[2][0] = K(2) * (xz + wy); R.m[2][1] = K(2) * (yz - wx); R.m[2][2] = K(1) - K(2) * (x2 + y2);
    return R;
}

/* iscl_rot = S^-1 R^T, glm m[col][row]: m[c][r] = R[r][c] / s_r (eval3d_fwd.cu:92-107) */
static m3 iscl_rot_of(const m3 *R, const real *s) {
    m3 M;
    for (int c = 0; c < 3; ++c)
        for (int r = 0; r < 3; ++r) M.m[c][r] = (K(1.0) / s[r]) * R->m[r][c];
    return M;
}

static v3 safe_normalize(v3 v) { /* utils.h:85-88 */
    const real l = dot3(v, v);
    return l > 0 ? scl3(v, K(1.0) / SQRT(l)) : v;
}

typedef struct {
    int width, height, tile_w, tile_h, n_tiles_w, n_tiles_h;
    int64_t n_isects;
} orc_grid;

static void tile_range(const orc_grid *g, const int32_t *offsets, int tile, int64_t *start, int64_t *end) {
    /* utils.h:48-58 */
    *start = offsets[tile];
    *end = (tile == g->n_tiles_w * g->n_tiles_h - 1) ? g->n_isects : offsets[tile + 1];
}

/* rasterize_eval3d_fwd_kernel: eval3d_fwd.cu:34-166 (+ dynamic eval3d_dynamic_fwd.cu:125 when
 * velocity != NULL: mean(t) = mean + dt_pixel * velocity). counters[0] += evaluated pairs,
 * counters[1] += contributing pairs. */
void orc_eval3d_fwd(int cdim, int n, const real *means, const real *quats, const real *scales,
                    const real *colors, const real *opac, const real *velocity,
                    const real *ray_time_delta, int width, int height, int tile_w, int tile_h,
                    const real *ray_o, const real *ray_d, const int32_t *offsets, int n_tiles_w,
                    int n_tiles_h, int64_t n_isects, const int32_t *flatten_ids, real *out_rgb,
                    real *out_depth, real *out_alpha, int32_t *last_ids, int64_t *counters,
                    const uint8_t *tile_mask, real *fmargin) {
    (void)n;
    const orc_grid g = {width, height, tile_w, tile_h, n_tiles_w, n_tiles_h, n_isects};
    const int n_tiles = n_tiles_w * n_tiles_h;
    int64_t evaluated = 0, contributing = 0;
#pragma omp parallel for schedule(dynamic, 4) reduction(+ : evaluated, contributing)
    for (int tile = 0; tile < n_tiles; ++tile) {
        if (tile_mask && !tile_mask[tile]) continue;  /* test subset: tiles left out keep their outputs */
        const int ty = tile / n_tiles_w, tx = tile % n_tiles_w;
        int64_t rs, re;
        tile_range(&g, offsets, tile, &rs, &re);
        const int64_t cnt = re > rs ? re - rs : 0;
        m3 *Ms = (m3 *)malloc(sizeof(m3) * (cnt ? cnt : 1));
        for (int64_t k = 0; k < cnt; ++k) {
            const int32_t gid = flatten_ids[rs + k];
            m3 R = quat_to_rotmat(quats + 4 * gid);
            Ms[k] = iscl_rot_of(&R, scales + 3 * gid);
        }
        real *pix = (real *)malloc(sizeof(real) * (cdim > 0 ? cdim : 1));
        for (int yy = 0; yy < tile_h; ++yy)
            for (int xx = 0; xx < tile_w; ++xx) {
                const int i = ty * tile_h + yy, j = tx * tile_w + xx;
                if (!(i < height && j < width)) continue;
                const long pid = (long)i * width + j;
                const v3 ro = ld3(ray_o + 3 * pid), rd = ld3(ray_d + 3 * pid);
                const real dtp = ray_time_delta ? ray_time_delta[pid] : K(0);
                real T = K(1.0), depth = K(0);
                real mg = K(1e30), relT = 0;  /* decision margins (fmargin) and T's relative error bound */
                int32_t cur = 0;
                for (int k = 0; k < cdim; ++k) pix[k] = 0;
                for (int64_t k = 0; k < cnt; ++k) {
                    const int32_t gid = flatten_ids[rs + k];
                    v3 xyz = ld3(means + 3 * gid);
                    if (velocity) xyz = add3(xyz, scl3(ld3(velocity + 3 * gid), dtp));
                    const v3 gro = mv(&Ms[k], sub3(ro, xyz));
                    const v3 grd = mv(&Ms[k], rd);
                    const v3 gcrod = cross3(safe_normalize(grd), gro);
                    const real power = K(-0.5) * dot3(gcrod, gcrod);
                    const real alpha = FMIN(K(0.999), opac[gid] * EXP(power));
                    ++evaluated;
                    real ea = 0;  /* relative error bound of a float32 alpha */
                    if (fmargin) {
                        /* |n x gro| is off by the error of gro (|M| = 1 / s_min times a few roundings of
                         * the ray origin and the mean) plus |gro| times the direction error (~ the
                         * condition s_max / s_min of M); exp turns the error of the power into a
                         * relative one */
                        const real *s = scales + 3 * gid;
                        const real smin = FMIN(s[0], FMIN(s[1], s[2])), smax = FMAX(s[0], FMAX(s[1], s[2]));
                        const v3 om = sub3(ro, xyz);
                        const real lom = SQRT(dot3(om, om));
                        const real lor = (ro.x != 0 || ro.y != 0 || ro.z != 0) ? SQRT(dot3(ro, ro)) + SQRT(dot3(xyz, xyz)) : 0;
                        const real dist = SQRT(dot3(gcrod, gcrod)), lg = SQRT(dot3(gro, gro));
                        const real e_d = F32_U * (K(3) * (lom / smin + (smax / smin) * lg) + lor / smin);
                        ea = K(4) * F32_U + dist * e_d + K(2) * F32_U * FABS(power);
                        const real araw = opac[gid] * EXP(power);
                        if (araw < K(0.999)) {
                            const real r = FABS(araw - K(1.0) / K(255.0)) / (K(2) * ea * araw + (real)1e-30);
                            if (r < mg) mg = r;
                        }
                    }
                    if (alpha < K(1.0) / K(255.0)) continue;
                    const real hit_t = -dot3(gro, grd) / dot3(grd, grd);
                    const real next_T = T * (K(1.0) - alpha);
                    if (fmargin) {
                        const real e1 = (ea * alpha + F32_U) / (K(1.0) - alpha) + K(2) * F32_U;
                        const real r = FABS(next_T - K(1e-4)) / (K(2) * next_T * (relT + e1) + (real)1e-30);
                        if (r < mg) mg = r;
                        relT += e1;
                    }
                    if (next_T <= K(1e-4)) break;
                    const real vis = alpha * T;
                    depth += vis * hit_t;
                    for (int c = 0; c < cdim; ++c) pix[c] += colors[(long)gid * cdim + c] * vis;
                    cur = (int32_t)(rs + k);
                    T = next_T;
                    ++contributing;
                }
                out_alpha[pid] = K(1.0) - T;
                if (fmargin) fmargin[pid] = mg;
                out_depth[pid] = depth;
                for (int c = 0; c < cdim; ++c) out_rgb[pid * cdim + c] = pix[c];
                last_ids[pid] = cur;
            }
        free(pix);
        free(Ms);
    }
    if (counters) { counters[0] += evaluated; counters[1] += contributing; }
}

static void quat_to_rotmat_vjp(const real *quat, const m3 *v_R, real *v_quat) {
    /* utils.h:208-230, v_R glm-indexed [col][row] */
    real w = quat[0], x = quat[1], y = quat[2], z = quat[3];
    const real inv = K(1.0) / SQRT(x * x + y * y + z * z + w * w);
    x *= inv; y *= inv; z *= inv; w *= inv;
    const real (*V)[3] = v_R->m;
    real vqn[4];
    vqn[0] = K(2) * (x * (V[1][2] - V[2][1]) + y * (V[2][0] - V[0][2]) + z * (V[0][1] - V[1][0]));
    vqn[1] = K(2) * (K(-2) * x * (V[1][1] + V[2][2]) + y * (V[0][1] + V[1][0]) + z * (V[0][2] + V[2][0]) +
                     w * (V[1][2] - V[2][1]));
    vqn[2] = K(2) * (x * (V[0][1] + V[1][0]) - K(2) * y * (V[0][0] + V[2][2]) + z * (V[1][2] + V[2][1]) +
                     w * (V[2][0] - V[0][2]));
    vqn[3] = K(2) * (x * (V[0][2] + V[2][0]) + y * (V[1][2] + V[2][1]) - K(2) * z * (V[0][0] + V[1][1]) +
                     w * (V[0][1] - V[1][0]));
    const real qn[4] = {w, x, y, z};
    const real dp = vqn[0] * qn[0] + vqn[1] * qn[1] + vqn[2] * qn[2] + vqn[3] * qn[3];
    for (int k = 0; k < 4; ++k) v_quat[k] += (vqn[k] - dp * qn[k]) * inv;
}

static void quat_scale_to_preci_half_vjp(const real *quat, const real *scale, const m3 *R,
                                         const m3 *v_M, real *v_quat, real *v_scale) {
    /* utils.h:232-263: M = R S, S = diag(1/scale) */
    const real s[3] = {K(1.0) / scale[0], K(1.0) / scale[1], K(1.0) / scale[2]};
    m3 v_R;
    for (int c = 0; c < 3; ++c)
        for (int r = 0; r < 3; ++r) v_R.m[c][r] = v_M->m[c][r] * s[c];
    quat_to_rotmat_vjp(quat, &v_R, v_quat);
    for (int c = 0; c < 3; ++c)
        v_scale[c] += -s[c] * s[c] *
                      (R->m[c][0] * v_M->m[c][0] + R->m[c][1] * v_M->m[c][1] + R->m[c][2] * v_M->m[c][2]);
}

#ifdef _OPENMP
#define ATOMIC_ADD(p, v) do { _Pragma("omp atomic") *(p) += (v); } while (0)
#else
#define ATOMIC_ADD(p, v) (*(p) += (v))
#endif

/* rasterize_eval3d_bwd_kernel: eval3d_bwd.cu:42-294 (dynamic: eval3d_dynamic_bwd.cu adds
 * v_velocity = -v_(o-mu) * dt and v_dt = -v_(o-mu) . velocity). Gradient outputs must be
 * zero-initialised; v_ray_o / v_ray_d are written for every pixel inside the image.
 *
 * abs_g / abs_px (test diagnostics, NULL or zero-initialised; they change no result): the sum of
 * the absolute per-pair contributions of each gradient component, per Gaussian [means 3, quats 4,
 * scales 3, opacity 1, colours cdim, velocity 3 when given] and per pixel [ray_o 3, ray_d 3,
 * time delta 1]. A component whose contributions cancel (the sum of their magnitudes far above the
 * magnitude of their sum) is rounded differently by every float32 summation order.
 *
 * und_mode (test diagnostics): 0 computes the reference's backward. 1 and 2 force the outcome of
 * every decision float32 rounding can take either way: a pair's alpha against 1/255 and its
 * opacity-times-visibility against the 0.99 gate, judged with the forward's bound on the float32
 * error of alpha (orc_eval3d_fwd's margins); 1 takes every such pair (and its geometry gradients),
 * 2 drops them. A gradient that differs between the two is decided by float32 rounding. */
void orc_eval3d_bwd(int cdim, const real *means, const real *quats, const real *scales,
                    const real *colors, const real *opac, const real *velocity,
                    const real *ray_time_delta, int width, int height, int tile_w, int tile_h,
                    const real *ray_o, const real *ray_d, const int32_t *offsets, int n_tiles_w,
                    int n_tiles_h, int64_t n_isects, const int32_t *flatten_ids,
                    const real *render_alpha, const int32_t *last_ids, const real *v_rgb,
                    const real *v_depth, const real *v_alpha, real *v_means, real *v_quats,
                    real *v_scales, real *v_opac, real *v_colors, real *v_ray_o, real *v_ray_d,
                    real *v_velocity, real *v_time_delta, const uint8_t *tile_mask, real *abs_g,
                    real *abs_px, int und_mode) {
    const orc_grid g = {width, height, tile_w, tile_h, n_tiles_w, n_tiles_h, n_isects};
    const int n_tiles = n_tiles_w * n_tiles_h;
    const real MAX_ALPHA = K(0.99);
    const long ag = 11 + cdim + (velocity ? 3 : 0);   /* abs_g row length */
#define ACC(ptr, val, k) do { const real v_ = (val); ATOMIC_ADD(ptr, v_); \
                              if (abs_g) ATOMIC_ADD(&abs_g[(long)gid * ag + (k)], FABS(v_)); } while (0)
#pragma omp parallel for schedule(dynamic, 4)
    for (int tile = 0; tile < n_tiles; ++tile) {
        if (tile_mask && !tile_mask[tile]) continue;  /* test subset: only these tiles' pixels contribute */
        const int ty = tile / n_tiles_w, tx = tile % n_tiles_w;
        int64_t rs, re;
        tile_range(&g, offsets, tile, &rs, &re);
        real *buffer = (real *)malloc(sizeof(real) * (cdim > 0 ? cdim : 1));
        for (int yy = 0; yy < tile_h; ++yy)
            for (int xx = 0; xx < tile_w; ++xx) {
                const int i = ty * tile_h + yy, j = tx * tile_w + xx;
                if (!(i < height && j < width)) continue;
                const long pid = (long)i * width + j;
                const v3 ro = ld3(ray_o + 3 * pid), rd = ld3(ray_d + 3 * pid);
                const real dtp = ray_time_delta ? ray_time_delta[pid] : K(0);
                const real T_final = K(1.0) - render_alpha[pid];
                real T = T_final;
                for (int c = 0; c < cdim; ++c) buffer[c] = 0;
                const int64_t bin_final = last_ids[pid];
                const real vd = v_depth[pid], va = v_alpha[pid];
                const real *vc = v_rgb ? v_rgb + pid * cdim : NULL;
                v3 v_ro = V3(0, 0, 0), v_rd = V3(0, 0, 0), a_ro = V3(0, 0, 0), a_rd = V3(0, 0, 0);
                real depth_buffer = 0, v_dt = 0, a_dt = 0;
                for (int64_t idx = re - 1; idx >= rs; --idx) {
                    if (idx > bin_final) continue;
                    const int32_t gid = flatten_ids[idx];
                    const real op = opac[gid];
                    v3 xyz = ld3(means + 3 * gid);
                    const v3 vel = velocity ? ld3(velocity + 3 * gid) : V3(0, 0, 0);
                    if (velocity) xyz = add3(xyz, scl3(vel, dtp));
                    const real *scale = scales + 3 * gid;
                    const real *quat = quats + 4 * gid;
                    const m3 R = quat_to_rotmat(quat);
                    const m3 Mt = iscl_rot_of(&R, scale);   /* transpose(R * S) */
                    const v3 omm = sub3(ro, xyz);
                    const v3 gro = mv(&Mt, omm);
                    const v3 grd = mv(&Mt, rd);
                    const v3 grd_n = safe_normalize(grd);
                    const v3 gcrod = cross3(grd_n, gro);
                    const real power = K(-0.5) * dot3(gcrod, gcrod);
                    const real vis = EXP(power);
                    const real alpha = FMIN(MAX_ALPHA, op * vis);
                    int take = alpha >= K(1.0) / K(255.0), gate = op * vis <= MAX_ALPHA;
                    if (und_mode) {
                        /* the forward's float32 error bound of alpha (orc_eval3d_fwd) */
                        const real *s = scales + 3 * gid;
                        const real smin = FMIN(s[0], FMIN(s[1], s[2])), smax = FMAX(s[0], FMAX(s[1], s[2]));
                        const real lom = SQRT(dot3(omm, omm));
                        const real lor = (ro.x != 0 || ro.y != 0 || ro.z != 0) ? SQRT(dot3(ro, ro)) + SQRT(dot3(xyz, xyz)) : 0;
                        const real dist = SQRT(dot3(gcrod, gcrod)), lg = SQRT(dot3(gro, gro));
                        const real e_d = F32_U * (K(3) * (lom / smin + (smax / smin) * lg) + lor / smin);
                        const real ea = K(4) * F32_U + dist * e_d + K(2) * F32_U * FABS(power);
                        const real araw = op * vis, eb = K(2) * ea * araw + (real)1e-30;
                        if (FABS(araw - K(1.0) / K(255.0)) < eb) take = und_mode == 1;
                        if (FABS(araw - MAX_ALPHA) < eb) gate = und_mode == 1;
                    }
                    if (!take) continue;
                    const real last_hit_T = -dot3(grd, gro) / dot3(grd, grd);
                    const real ra = K(1.0) / FMAX(K(1e-6), K(1.0) - alpha);
                    T *= ra;
                    const real fac = alpha * T;
                    const real *rgb = colors ? colors + (long)gid * cdim : NULL;
                    /* grad_alpha: eval3d_bwd.cu:42-63 */
                    real v_a = 0;
                    for (int c = 0; c < cdim; ++c) v_a += (rgb[c] * T - buffer[c] * ra) * vc[c];
                    v_a += (last_hit_T * T - depth_buffer * ra) * vd;
                    v_a += T_final * ra * va;
                    for (int c = 0; c < cdim; ++c) ACC(&v_colors[(long)gid * cdim + c], vc[c] * fac, 11 + c);
                    const real dd = dot3(grd, grd), od = dot3(gro, grd);
                    const real dL_dhitT = vd * fac;
                    v3 v_gro = scl3(scl3(grd, K(-1)), dL_dhitT / dd);
                    v3 v_grd = scl3(sub3(scl3(grd, K(2.0) * od), scl3(gro, dd)), dL_dhitT / (dd * dd));
                    if (gate) {
                        const real v_vis = op * v_a;
                        const real v_gd = K(-0.5) * vis * v_vis;
                        const v3 v_gcrod = scl3(gcrod, K(2.0) * v_gd);
                        const v3 v_grd_n = scl3(cross3(v_gcrod, gro), K(-1));
                        v_gro = add3(v_gro, cross3(v_gcrod, grd_n));
                        { /* safe_normalize_bwd: utils.h:198-206 */
                            const real l = dot3(grd, grd);
                            if (l > 0) {
                                const real il = K(1.0) / SQRT(l), il3 = il * il * il;
                                v_grd = add3(v_grd, sub3(scl3(v_grd_n, il), scl3(grd, il3 * dot3(v_grd_n, grd))));
                            } else {
                                v_grd = add3(v_grd, v_grd_n);
                            }
                        }
                        m3 v_Mt; /* outerProduct(v_grd, rd) + outerProduct(v_gro, omm): [col j][row i] */
                        const real a3[3] = {v_grd.x, v_grd.y, v_grd.z}, b3[3] = {v_gro.x, v_gro.y, v_gro.z};
                        const real d3[3] = {rd.x, rd.y, rd.z}, o3[3] = {omm.x, omm.y, omm.z};
                        for (int cj = 0; cj < 3; ++cj)
                            for (int ri = 0; ri < 3; ++ri) v_Mt.m[cj][ri] = a3[ri] * d3[cj] + b3[ri] * o3[cj];
                        const m3 trMt = transpose3(&Mt);
                        const v3 v_omm = mv(&trMt, v_gro);
                        ACC(&v_means[3 * gid], -v_omm.x, 0);
                        ACC(&v_means[3 * gid + 1], -v_omm.y, 1);
                        ACC(&v_means[3 * gid + 2], -v_omm.z, 2);
                        if (velocity) {
                            ACC(&v_velocity[3 * gid], -v_omm.x * dtp, 11 + cdim);
                            ACC(&v_velocity[3 * gid + 1], -v_omm.y * dtp, 12 + cdim);
                            ACC(&v_velocity[3 * gid + 2], -v_omm.z * dtp, 13 + cdim);
                            v_dt += -dot3(v_omm, vel);
                            a_dt += FABS(dot3(v_omm, vel));
                        }
                        const v3 v_rd_i = mv(&trMt, v_grd);
                        v_ro = add3(v_ro, v_omm);
                        v_rd = add3(v_rd, v_rd_i);
                        a_ro = add3(a_ro, V3(FABS(v_omm.x), FABS(v_omm.y), FABS(v_omm.z)));
                        a_rd = add3(a_rd, V3(FABS(v_rd_i.x), FABS(v_rd_i.y), FABS(v_rd_i.z)));
                        const m3 v_M = transpose3(&v_Mt);
                        real vq[4] = {0, 0, 0, 0}, vs[3] = {0, 0, 0};
                        quat_scale_to_preci_half_vjp(quat, scale, &R, &v_M, vq, vs);
                        for (int k = 0; k < 4; ++k) ACC(&v_quats[4 * gid + k], vq[k], 3 + k);
                        for (int k = 0; k < 3; ++k) ACC(&v_scales[3 * gid + k], vs[k], 7 + k);
                        ACC(&v_opac[gid], vis * v_a, 10);
                    }
                    for (int c = 0; c < cdim; ++c) buffer[c] += rgb[c] * fac;
                    depth_buffer += fac * last_hit_T;
                }
                v_ray_o[3 * pid] = v_ro.x; v_ray_o[3 * pid + 1] = v_ro.y; v_ray_o[3 * pid + 2] = v_ro.z;
                v_ray_d[3 * pid] = v_rd.x; v_ray_d[3 * pid + 1] = v_rd.y; v_ray_d[3 * pid + 2] = v_rd.z;
                if (v_time_delta) v_time_delta[pid] = v_dt;
                if (abs_px) {
                    real *a = abs_px + 7 * pid;
                    a[0] = a_ro.x; a[1] = a_ro.y; a[2] = a_ro.z;
                    a[3] = a_rd.x; a[4] = a_rd.y; a[5] = a_rd.z; a[6] = a_dt;
                }
            }
        free(buffer);
    }
#undef ACC
}

/* Host-side mask_radii: mask_radii.cu:10-58 (bool and packed uint32 masks). */
void orc_mask_radii(int n, const uint8_t *mask, const uint32_t *packed, float *radii) {
    for (int i = 0; i < n; ++i) {
        const int keep = packed ? ((packed[i / 32] & (1u << (i % 32))) != 0) : (mask[i] != 0);
        if (!keep) { radii[2 * i] = 0; radii[2 * i + 1] = 0; }
    }
}

int orc_real_bytes(void) { return (int)sizeof(real); }

/* 1 while the calling thread's decision-margin pointer is set: every exported function clears it
 * before it returns, so that no later call notes a margin through a dead stack slot (test hook). */
int orc_margin_pointer_live(void) { return tl_mg != NULL; }

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
    omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ------------------------------------------------------------------------- */
/* Scene-assembly producers: csrc/nodes/gs_masking.cu, csrc/nodes/container.cu */
/* ------------------------------------------------------------------------- */

/* packed_mask_from_instances (gs_masking.cu:8-47): bit i % 32 of word i / 32 is set when element i
 * belongs to no instance (id < 0) or its instance is enabled (mask byte non-zero). Ids at or past
 * n_instances count as enabled (the reference reads past the mask there). */
void orc_packed_mask_from_instances(long n, const int32_t *ids, const uint8_t *inst_mask, long n_inst,
                                    uint32_t *out) {
    const long nw = (n + 31) / 32;
    for (long w = 0; w < nw; ++w) out[w] = 0;
    for (long i = 0; i < n; ++i) {
        const int32_t id = ids[i];
        const int v = (id < 0 || (long)id >= n_inst) ? 1 : (inst_mask[id] != 0);
        if (v) out[i / 32] |= (uint32_t)1 << (i % 32);
    }
}

/* unit-quaternion (w, x, y, z) rotation p + 2 (w (u x p) + u x (u x p)) and Hamilton product a b */
static v3 qrot(const real *q, v3 p) { return quat_apply(q[0], V3(q[1], q[2], q[3]), p); }

static void qmul(const real *a, const real *b, real *o) {
    const v3 av = V3(a[1], a[2], a[3]), bv = V3(b[1], b[2], b[3]);
    const v3 ov = add3(add3(scl3(bv, a[0]), scl3(av, b[0])), cross3(av, bv));
    o[0] = a[0] * b[0] - dot3(av, bv);
    o[1] = ov.x; o[2] = ov.y; o[3] = ov.z;
}

/* output row of particle i, or -1 when it is skipped: instance out of range or disabled, or a row
 * outside [0, n_out) (the reference writes there unchecked) */
static long rigid_row(long i, const int32_t *inst_id, const uint8_t *imask, long n_inst, long buffer_offset,
                      const int32_t *per_inst_off, const int32_t *gs_inst_off, long n_out, long *id_out) {
    const uint32_t id = (uint32_t)inst_id[i];
    if ((long)id >= n_inst || !imask[id]) return -1;
    const long r = buffer_offset + (gs_inst_off ? (long)(uint32_t)per_inst_off[id] + (long)(uint32_t)gs_inst_off[i] : i);
    if (r < 0 || r >= n_out) return -1;
    *id_out = (long)id;
    return r;
}

/* copy_gs_rigid_transform_fwd_kernel (container.cu:13-75): out_pos = q_k p + t_k, out_rot = q_k q,
 * out_vel = v_k + w_k x (q_k p), out_mask = 1 at row buffer_offset + i (or + per_instance_offsets[k]
 * + gs_inst_offsets[i]); rows of disabled instances are left as they are */
void orc_rigid_fwd(long n, const real *pos, const real *rot, const int32_t *inst_id, const real *iq, const real *it,
                   const real *iv, const real *iw, const uint8_t *imask, long n_inst, long buffer_offset,
                   const int32_t *per_inst_off, const int32_t *gs_inst_off, long n_out, real *out_pos,
                   real *out_rot, real *out_vel, uint8_t *out_mask) {
    for (long i = 0; i < n; ++i) {
        long k;
        const long r = rigid_row(i, inst_id, imask, n_inst, buffer_offset, per_inst_off, gs_inst_off, n_out, &k);
        if (r < 0) continue;
        const v3 pr = qrot(iq + 4 * k, ld3(pos + 3 * i));
        out_pos[3 * r] = pr.x + it[3 * k]; out_pos[3 * r + 1] = pr.y + it[3 * k + 1];
        out_pos[3 * r + 2] = pr.z + it[3 * k + 2];
        qmul(iq + 4 * k, rot + 4 * i, out_rot + 4 * r);
        if (out_vel) {
            const v3 vel = add3(ld3(iv + 3 * k), cross3(ld3(iw + 3 * k), pr));
            out_vel[3 * r] = vel.x; out_vel[3 * r + 1] = vel.y; out_vel[3 * r + 2] = vel.z;
        }
        if (out_mask) out_mask[r] = 1;
    }
}

/* copy_gs_rigid_transform_bwd_kernel (container.cu:78-160): per-particle gradients (0 for skipped
 * particles) and per-instance sums (in double); v_vel may be NULL */
void orc_rigid_bwd(long n, const real *pos, const real *rot, const int32_t *inst_id, const real *iq, const real *iw,
                   const uint8_t *imask, long n_inst, long buffer_offset, const int32_t *per_inst_off,
                   const int32_t *gs_inst_off, long n_out, const real *v_pos, const real *v_rot, const real *v_vel,
                   real *g_pos, real *g_rot, real *g_q, real *g_t, real *g_v, real *g_w) {
    double *acc = (double *)calloc((size_t)n_inst * 13, sizeof(double));
    for (long i = 0; i < 3 * n; ++i) g_pos[i] = 0;
    for (long i = 0; i < 4 * n; ++i) g_rot[i] = 0;
    for (long i = 0; i < n; ++i) {
        long k;
        const long r = rigid_row(i, inst_id, imask, n_inst, buffer_offset, per_inst_off, gs_inst_off, n_out, &k);
        if (r < 0) continue;
        const real *q = iq + 4 * k;
        const v3 u = V3(q[1], q[2], q[3]);
        const v3 p = ld3(pos + 3 * i);
        const v3 g = ld3(v_pos + 3 * r);
        double *a = acc + 13 * k;  /* q(4) t(3) v(3) w(3) */
        a[4] += g.x; a[5] += g.y; a[6] += g.z;
        v3 gp = g;  /* gradient at q p */
        if (v_vel) {
            const v3 gv = ld3(v_vel + 3 * r);
            const v3 pr = qrot(q, p);
            const v3 gw = cross3(pr, gv);
            a[7] += gv.x; a[8] += gv.y; a[9] += gv.z;
            a[10] += gw.x; a[11] += gw.y; a[12] += gw.z;
            gp = add3(gp, cross3(gv, ld3(iw + 3 * k)));
        }
        /* y = p + 2 (w (u x p) + u x (u x p)) */
        const v3 dp = add3(sub3(gp, scl3(cross3(u, gp), K(2.0) * q[0])), scl3(cross3(u, cross3(u, gp)), K(2.0)));
        const real dw = K(2.0) * dot3(gp, cross3(u, p));
        const v3 du = add3(add3(scl3(cross3(p, gp), K(2.0) * q[0]), scl3(p, K(2.0) * dot3(gp, u))),
                           sub3(scl3(gp, K(2.0) * dot3(u, p)), scl3(u, K(4.0) * dot3(gp, p))));
        g_pos[3 * i] = dp.x; g_pos[3 * i + 1] = dp.y; g_pos[3 * i + 2] = dp.z;
        /* out_rot = q_k (x) rot: Hamilton product backward */
        const real *b = rot + 4 * i;
        const v3 bv = V3(b[1], b[2], b[3]);
        const real dqw = v_rot[4 * r];
        const v3 dqv = V3(v_rot[4 * r + 1], v_rot[4 * r + 2], v_rot[4 * r + 3]);
        const real daw = dqw * b[0] + dot3(dqv, bv);
        const v3 dav = add3(sub3(scl3(dqv, b[0]), scl3(bv, dqw)), cross3(bv, dqv));
        const real dbw = dqw * q[0] + dot3(dqv, u);
        const v3 dbv = add3(sub3(scl3(dqv, q[0]), scl3(u, dqw)), cross3(dqv, u));
        g_rot[4 * i] = dbw; g_rot[4 * i + 1] = dbv.x; g_rot[4 * i + 2] = dbv.y; g_rot[4 * i + 3] = dbv.z;
        a[0] += dw + daw; a[1] += du.x + dav.x; a[2] += du.y + dav.y; a[3] += du.z + dav.z;
    }
    for (long k = 0; k < n_inst; ++k) {
        const double *a = acc + 13 * k;
        for (int j = 0; j < 4; ++j) g_q[4 * k + j] = (real)a[j];
        for (int j = 0; j < 3; ++j) {
            g_t[3 * k + j] = (real)a[4 + j];
            g_v[3 * k + j] = (real)a[7 + j];
            g_w[3 * k + j] = (real)a[10 + j];
        }
    }
    free(acc);
}
