/*
 * CPU oracle for the xsimgs Gaussian-splatting hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * A restatement, in plain C, of the reference kernels (whesense/xsimgs, files
 * cited per function in xsg_oracle.c). It is the checker for the HIP kernels of
 * xsimgs_amd and the host-CPU baseline timed by bench.py; nothing in the product
 * path links, loads or calls it.
 *
 * Built twice: REAL=float (xsg_oracle_f32.so, the parity reference) and
 * REAL=double (xsg_oracle_f64.so, used by finite-difference gradient checks).
 */
#ifndef XSG_ORACLE_H
#define XSG_ORACLE_H
#include <stdint.h>

#ifdef ORC_DOUBLE
typedef double real;
#else
typedef float real;
#endif

/* Camera kinds and the flat camera-pack layout shared with the HIP side. */
enum { ORC_PINHOLE = 0, ORC_SPHERICAL = 1, ORC_LIDAR = 2, ORC_DISTORTED = 3, ORC_FISHEYE = 4 };
enum { ORC_MODE_CENTRAL = 0, ORC_MODE_NEG = 1, ORC_MODE_POS = 2 };

typedef struct {
    int kind;
    real q[4];        /* camera-to-world rotation (w, x, y, z) */
    real t[3];
    real v[3];        /* linear velocity */
    real w[3];        /* angular velocity */
    real rolling[2];  /* rolling-shutter duration along u, v */
    real trigger_time;
    real pose_time;
    real impl[4];     /* pinhole, distorted, fisheye f.x f.y c.x c.y |
                         spherical, lidar phi_min phi_range theta_min theta_range */
    const real *beam_v; /* lidar: per-row v coordinate (host memory) */
    int n_beams;
    real dist[8];       /* distorted: k1 k2 p1 p2 k3 k4 k5 k6 | fisheye: k1 k2 k3 k4 */
    real max_radius_sq; /* distorted: largest squared camera-space radius |xy / z|^2 projected */
} orc_camera;

#endif
