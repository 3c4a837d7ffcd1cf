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
enum { ORC_PINHOLE = 0, ORC_SPHERICAL = 1, ORC_LIDAR = 2 };
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
    real impl[4];     /* pinhole f.x f.y c.x c.y | spherical phi_min phi_range theta_min theta_range */
    const real *beam_v; /* lidar: per-row v coordinate (host memory) */
    int n_beams;
} orc_camera;

#endif
