// eval3d compositing kernels (reference csrc/rasterization/eval3d_{fwd,bwd}.cu, eval3d_dynamic_*.cu).
//
// One workgroup per (camera, tile); in the forward one thread per pixel (up to 1024 threads, 16
// wave64s), in the backward two or four pixels per thread. Gaussians of the tile's depth-sorted list are staged in LDS in batches of one
// per thread. Per staged Gaussian the LDS slot holds M = S^-1 R^T (three rows) and, when every ray
// of the tile starts at the same origin (decided by a block vote, always true for a static pinhole
// or spherical camera), gro = M (o - mu): the per-pair work then only maps the ray direction.
// These are the values the reference computes per pair, so results do not depend on the path.
#pragma once
#include "xsg_common.h"

namespace xsg {

constexpr int kTileThreads = 256;
constexpr int kMaxTilePixels = 1024;  // largest tile: the reference's 1024-thread workgroup limit
constexpr int kColorLdsMax = 16;  // colour channels staged in LDS; larger CDIM read from HBM

// The backward's variants of one group are compiled in one translation unit (eval3d_bwd_g<k>.hip).
#define XSG_CDIM_GROUP0(X) X(0) X(1) X(2) X(3) X(4) X(5)
#define XSG_CDIM_GROUP1(X) X(8) X(9) X(16) X(17)
#define XSG_CDIM_GROUP2(X) X(32) X(33)
#define XSG_CDIM_GROUP3(X) X(64) X(65)
#define XSG_CDIM_GROUP4(X) X(128) X(129)
#define XSG_CDIM_GROUP5(X) X(256) X(257)
#define XSG_CDIM_GROUP6(X) X(512)
#define XSG_CDIM_GROUP7(X) X(513)
#define XSG_CDIM_LIST(X)                                                                                \
    XSG_CDIM_GROUP0(X) XSG_CDIM_GROUP1(X) XSG_CDIM_GROUP2(X) XSG_CDIM_GROUP3(X) XSG_CDIM_GROUP4(X) \
    XSG_CDIM_GROUP5(X) XSG_CDIM_GROUP6(X) XSG_CDIM_GROUP7(X)

struct TileGrid {
    int width, height, tile_w, tile_h, n_tiles_w, n_tiles_h, n_cams;
    int64_t n;          // Gaussians (flatten id = cam * n + gaussian)
    int64_t n_isects;
};

struct PixelCtx {
    int cam, tile, tr;
    int i, j;
    bool inside;
    int64_t pix;          // index into [n_cams, H, W]
    int32_t range_start, range_end;
};

XSG_DEV PixelCtx pixel_ctx(const TileGrid& g, const int32_t* __restrict__ offsets) {
    PixelCtx c;
    const int n_tiles = g.n_tiles_w * g.n_tiles_h;
    const int nblocks = n_tiles * g.n_cams;
    const int logical = xcd_tile((int)blockIdx.x, nblocks);
    c.cam = logical / n_tiles;
    c.tile = logical - c.cam * n_tiles;
    c.tr = threadIdx.x;
    const int ty = c.tr / g.tile_w, tx = c.tr - ty * g.tile_w;
    const int trow = c.tile / g.n_tiles_w, tcol = c.tile - trow * g.n_tiles_w;
    c.i = trow * g.tile_h + ty;  // utils.h:32-44
    c.j = tcol * g.tile_w + tx;
    c.inside = c.tr < g.tile_w * g.tile_h && c.i < g.height && c.j < g.width;
    const int64_t hw = (int64_t)g.width * g.height;
    c.pix = (int64_t)c.cam * hw + min((int64_t)c.i * g.width + c.j, hw - 1);
    const int gt = c.cam * n_tiles + c.tile;  // utils.h:48-58
    c.range_start = offsets[gt];
    c.range_end = (gt == nblocks - 1) ? (int32_t)g.n_isects : offsets[gt + 1];
    return c;
}

// Rows of M = S^-1 R^T from the raw quaternion (w, x, y, z) and activated scales: row i is column i
// of R / s_i (utils.h:61-83 and eval3d_fwd.cu:92-107).
XSG_DEV void iscl_rot_rows(float4 q, f3 s, f3& r0, f3& r1, f3& r2) {
    float w = q.x, x = q.y, y = q.z, z = q.w;
    const float inv = rsqrtf(x * x + y * y + z * z + w * w);
    x *= inv; y *= inv; z *= inv; w *= inv;
    const float x2 = x * x, y2 = y * y, z2 = z * z;
    const float xy = x * y, xz = x * z, yz = y * z;
    const float wx = w * x, wy = w * y, wz = w * z;
    const float i0 = 1.0f / s.x, i1 = 1.0f / s.y, i2 = 1.0f / s.z;
    r0 = mk3(i0 * (1.f - 2.f * (y2 + z2)), i0 * (2.f * (xy + wz)), i0 * (2.f * (xz - wy)));
    r1 = mk3(i1 * (2.f * (xy - wz)), i1 * (1.f - 2.f * (x2 + z2)), i1 * (2.f * (yz + wx)));
    r2 = mk3(i2 * (2.f * (xz + wy)), i2 * (2.f * (yz - wx)), i2 * (1.f - 2.f * (x2 + y2)));
}

XSG_DEV f3 rows_mul(f3 r0, f3 r1, f3 r2, f3 v) { return mk3(dot(r0, v), dot(r1, v), dot(r2, v)); }
XSG_DEV f3 rows_tmul(f3 r0, f3 r1, f3 r2, f3 v) {  // M^T v
    return mk3(r0.x * v.x + r1.x * v.y + r2.x * v.z, r0.y * v.x + r1.y * v.y + r2.y * v.z,
               r0.z * v.x + r1.z * v.y + r2.z * v.z);
}

// 1/sqrt(l) for l > 0, else 1: safe_normalize(v) (utils.h:85-88) is v * inv_len(|v|^2). The raw
// v_rsq_f32 (1 ulp) replaces rsqrtf, whose denormal-range scaling costs five more instructions.
XSG_DEV float inv_len(float l) { return l > 0.0f ? __builtin_amdgcn_rsqf(l) : 1.0f; }

XSG_DEV f3 safe_normalize(f3 v) { return v * inv_len(dot(v, v)); }

// safe_normalize_bwd (utils.h:198-206) with il = inv_len(|v|^2) already known
XSG_DEV f3 safe_normalize_bwd_il(f3 v, float il, f3 d_out) {
    return il * d_out - (il * il * il * dot(d_out, v)) * v;
}

// ---------------------------------------------------------------------------------------------
// Conservative (wavefront, Gaussian) culling.
//
// A pair adds nothing unless alpha = min(0.999, op exp(-d^2 / 2)) >= 1/255, d = |n x gro| being
// the distance, in the Gaussian's normalised frame (x -> M x, M = S^-1 R^T, centre at 0), from the
// centre to the pixel's ray line {gro + t n}. For a wavefront, every ray starts within rho of a
// point c and points within angle theta of a unit axis a. In the normalised frame the origins lie
// within rho / s_min of g0 = M (c - mu), and each direction M d is within theta' of M a, with
//   sin theta' <= sin theta |Ma x Mb| / (|Ma| |Md|) <= sin theta (s_max / (s1 s2 s3)) /
//                 (|Ma| (|Ma| cos theta - sin theta / s_min))
// (d = cos phi a + sin phi b, (Ma) x (Mb) = det M M^-T (a x b), |M^-T| = s_max, |Mb| <= 1/s_min).
// So d >= (|g0 x Ma| cos theta' - |g0 . Ma| sin theta') / |Ma| - rho / s_min. Independently, as
// |M w| >= |w| / s_max, d >= dist(mu, line) / s_max >= (|v x a| cos theta - |v . a| sin theta - rho)
// / s_max with v = mu - c, which stays tight for very flat Gaussians where theta' is large. When
// either bound exceeds d_lim = sqrt(2 ln(255 op)) (plus a bound on the f32 error of the per-pair
// d) no pixel of the wavefront can take the Gaussian: the pair would be evaluated and skipped by the alpha test, and
// skipping it unevaluated changes no output. Pairs whose per-pair math could overflow or produce
// NaN (non-finite inputs, degenerate scales or rays) are always kept, so they reach the alpha test
// as in the reference.
struct RayBundle {
    float cx, cy, cz;    // centre of the ray origins
    float ax, ay, az;    // unit axis
    float cos_t, sin_t;  // bound on the angle between a ray and the axis
    float rho;           // bound on |o_i - c|
    float rt_max;        // bound on |time delta| (dynamic)
    float rd_max;        // bound on |rd_i|
    int mode;            // kBundleCull, kBundleKeepAll or kBundleEmpty
};
constexpr int kBundleCull = 0, kBundleKeepAll = 1, kBundleEmpty = 2;

XSG_DEV float wave_sum_f(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
XSG_DEV float wave_max_f(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
XSG_DEV float wave_min_f(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fminf(v, __shfl_xor(v, off, 64));
    return v;
}
// A wave-uniform 64-bit value read from LDS, moved to scalar registers (readfirstlane is signed:
// each half goes through uint32_t so that the low half is not sign-extended).
XSG_DEV uint64_t uniform_u64(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}
XSG_DEV bool finite3(f3 v) { return isfinite(v.x) && isfinite(v.y) && isfinite(v.z); }
XSG_DEV f3 sel3(bool c, f3 a, f3 b) { return mk3(c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z); }

// Bundle of the P pixels per lane of a full wavefront (all 64 lanes active). Pixels outside the
// image do not count; one inside pixel with a degenerate ray turns culling off for the wavefront.
template <int P>
XSG_DEV RayBundle wave_bundle(const bool (&inside)[P], const f3 (&ro)[P], const f3 (&rd)[P],
                              const float (&rt)[P]) {
    RayBundle b;
    bool irregular = false, any = false;
    f3 dn[P], sum = mk3(0.f, 0.f, 0.f), first = mk3(0.f, 0.f, 0.f);
    bool use[P];
    float rd2 = 0.f, rtm = 0.f;
#pragma unroll
    for (int h = P - 1; h >= 0; --h) {
        const float l = dot(rd[h], rd[h]);
        const bool reg = l >= 1e-12f && l <= 1e12f && finite3(ro[h]) && isfinite(rt[h]);
        irregular = irregular || (inside[h] && !reg);
        use[h] = inside[h] && reg;
        any = any || use[h];
        dn[h] = sel3(use[h], rd[h] * __builtin_amdgcn_rsqf(l), mk3(0.f, 0.f, 0.f));
        sum = sum + dn[h];
        rd2 = use[h] ? fmaxf(rd2, l) : rd2;
        rtm = use[h] ? fmaxf(rtm, fabsf(rt[h])) : rtm;
        first = sel3(use[h], ro[h], first);  // the lowest usable pixel of the lane
    }
    const uint64_t any_mask = __ballot(any);
    const bool irr = __ballot(irregular) != 0;
    sum = mk3(wave_sum_f(sum.x), wave_sum_f(sum.y), wave_sum_f(sum.z));
    const float sl = dot(sum, sum);
    const f3 a = sum * (sl > 0.f ? __builtin_amdgcn_rsqf(sl) : 0.f);
    float smax = 0.f, cmin = 1.f;
#pragma unroll
    for (int h = 0; h < P; ++h) {
        const f3 x = cross(dn[h], a);
        smax = use[h] ? fmaxf(smax, __builtin_amdgcn_sqrtf(dot(x, x))) : smax;
        cmin = use[h] ? fminf(cmin, dot(dn[h], a)) : cmin;
    }
    smax = wave_max_f(smax);
    cmin = wave_min_f(cmin);
    const int src = any_mask ? (int)__builtin_ctzll(any_mask) : 0;
    const f3 c = mk3(__shfl(first.x, src, 64), __shfl(first.y, src, 64), __shfl(first.z, src, 64));
    float rho = 0.f;
#pragma unroll
    for (int h = 0; h < P; ++h) {
        const f3 u = ro[h] - c;
        rho = use[h] ? fmaxf(rho, __builtin_amdgcn_sqrtf(dot(u, u))) : rho;
    }
    rho = wave_max_f(rho);
    b.cx = c.x; b.cy = c.y; b.cz = c.z;
    b.ax = a.x; b.ay = a.y; b.az = a.z;
    b.sin_t = fminf(1.f, smax * 1.00001f + 1e-6f);
    b.cos_t = __builtin_amdgcn_sqrtf(fmaxf(0.f, 1.f - b.sin_t * b.sin_t));
    b.rho = rho * 1.000001f;
    b.rt_max = wave_max_f(rtm);
    b.rd_max = __builtin_amdgcn_sqrtf(wave_max_f(rd2)) * 1.000001f;
    // a bundle wider than 60 degrees is not worth bounding
    b.mode = any_mask == 0 ? kBundleEmpty : ((irr || !(sl > 0.f) || !(cmin > 0.5f)) ? kBundleKeepAll : kBundleCull);
    return b;
}

// Per-Gaussian part of the test, computed once per staged Gaussian.
struct CullGauss {
    f3 mu, r0, r1, r2;  // centre and rows of M
    float inv_smin;     // 1 / s_min
    float s_max;
    float cone;         // s_max / (s1 s2 s3) = 1 / (product of the two smaller scales)
    float s_min, d_lim, vel_len;
    bool ok;            // finite inputs, scales in [1e-12, 1e9], a quaternion that normalises
    bool op_low;        // op < 1/255: alpha never reaches the threshold
};

XSG_DEV CullGauss cull_gauss(f3 mu, f3 r0, f3 r1, f3 r2, f3 s, float4 q, float op, f3 vel) {
    CullGauss g;
    g.mu = mu; g.r0 = r0; g.r1 = r1; g.r2 = r2;
    const float s_max = fmaxf(s.x, fmaxf(s.y, s.z));
    g.s_max = s_max;
    g.s_min = fminf(s.x, fminf(s.y, s.z));
    g.inv_smin = 1.f / g.s_min;
    g.cone = s_max / (s.x * s.y * s.z);
    const float q2 = q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w;
    g.vel_len = __builtin_amdgcn_sqrtf(dot(vel, vel));
    g.ok = finite3(mu) && g.s_min >= 1e-12f && s_max <= 1e9f && q2 >= 1e-30f && q2 <= 1e30f && isfinite(op) &&
           isfinite(g.vel_len);
    g.op_low = op < 1.f / 255.f;
    // 2 ln(255 op) through log2; + 3e-3 covers the rounding of log, exp, the product and the compare
    const float l2 = 2.f * 0.69314718f * __builtin_amdgcn_logf(fmaxf(255.f * op, 1.f));
    g.d_lim = __builtin_amdgcn_sqrtf(fmaxf(0.f, l2)) * 1.0001f + 3e-3f;
    return g;
}

// True unless no pixel of the bundle can take the Gaussian.
template <bool DYN>
XSG_DEV bool cull_keep(const RayBundle& b, const CullGauss& g) {
    if (b.mode != kBundleCull) return b.mode == kBundleKeepAll;
    const f3 v = mk3(b.cx, b.cy, b.cz) - g.mu, a = mk3(b.ax, b.ay, b.az);
    const f3 g0 = rows_mul(g.r0, g.r1, g.r2, v);  // M (c - mu)
    const f3 ma = rows_mul(g.r0, g.r1, g.r2, a);  // M a
    const float ma_len = __builtin_amdgcn_sqrtf(dot(ma, ma));
    const float shift = b.rho + (DYN ? b.rt_max * g.vel_len : 0.f);  // |o_i - c| + |mu(t) - mu|
    const float Dr = __builtin_amdgcn_sqrtf(dot(v, v)) + shift;     // bound on |o_i - mu(t)|
    const float L = Dr * g.inv_smin;                                 // bound on |gro| of every pair
    // per-pair products stay below 1e18, so the alpha test sees finite values
    const bool safe = g.s_min * g.s_min * 1e18f >= Dr * b.rd_max;
    const float mc = ma_len * b.cos_t, ms = b.sin_t * g.inv_smin;
    const bool narrow = mc - ms > 0.01f * mc;  // the direction bound below holds, to 1% cancellation
    const float sin_tp = fminf(1.f, b.sin_t * g.cone / (ma_len * (mc - ms)) * 1.00001f + 1e-6f);
    const float cos_tp = __builtin_amdgcn_sqrtf(fmaxf(0.f, 1.f - sin_tp * sin_tp));
    const f3 x = cross(g0, ma);
    const float lhs = (__builtin_amdgcn_sqrtf(dot(x, x)) * cos_tp - fabsf(dot(g0, ma)) * sin_tp) / ma_len;
    // 2e-5 L bounds the f32 error of the per-pair d (about 17 ulp of |gro|) and of these tests
    const float d_err = g.d_lim + 2e-5f * L;
    const bool far_n = narrow && lhs > d_err + shift * g.inv_smin * 1.00001f;
    // world-space bound (1e-5 Dr: this test's own rounding)
    const f3 xw = cross(v, a);
    const float lhs_w = __builtin_amdgcn_sqrtf(dot(xw, xw)) * b.cos_t - fabsf(dot(v, a)) * b.sin_t;
    const bool far_w = lhs_w > d_err * g.s_max * 1.0001f + shift * 1.00001f + 1e-5f * Dr;
    const bool skip = g.ok && safe && (g.op_low || far_n || far_w);
    return !skip;
}

// Lane-to-lane moves inside rows of 16 lanes (DPP). `update_dpp` with all rows/banks enabled and
// in-bounds patterns returns the source lane's value for every lane.
template <int CTRL>
XSG_DEV float dpp_mov(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
constexpr int kDppQuadSwap1 = 0xB1;    // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuadSwap2 = 0x4E;    // quad_perm [2,3,0,1]: lane ^ 2

struct Eval3dParams {
    TileGrid g;
    const float* means;
    const float4* quats;
    const float* scales;
    const float* colors;
    const float* opac;
    const float* velocity;
    const float* rtd;
    const float* ray_o;
    const float* ray_d;
    const int32_t* offsets;
    const int32_t* flatten;
    float* out_rgb;
    float* out_depth;
    float* out_alpha;
    int32_t* out_last;
    const float* render_alpha;
    const int32_t* last_ids;
    const float* v_rgb;
    const float* v_depth;
    const float* v_alpha;
    float* v_means;
    float* v_opac;
    float* v_colors;
    float* v_ray_o;
    float* v_ray_d;
    float* v_velocity;
    float* v_time;
    float* v_mt;         // workspace [n, 6]: upper triangle of the symmetric Q = sum of v_grd (x) grd + v_gro (x) gro
    // colours of flatten id fid in camera cam sit at fid * CDIM - cam * col_shift: 0 for per-camera
    // colours [n_cams, n, CDIM], n * CDIM for one colour set [n, CDIM] that every camera shares
    int64_t col_shift;
    unsigned long long* pair_counts;  // optional: += [evaluated, composited] pixel-pairs
    // optional (backward): logical (camera, tile) block launched at each position of xcd_tile's order
    const int32_t* tile_order;
    int px_hint;  // backward pixels per lane for 129..256-pixel tiles: 0 (by grid size), 2 or 4
    // optional (forward): per (camera, tile) the backward's work estimate, the tile's intersections up
    // to its pixels' largest last id (what tile_work_kernel derives from the last ids)
    int32_t* tile_work;
};

int eval3d_fwd_launch(int cdim, bool dyn, const Eval3dParams& p, hipStream_t s);
int eval3d_bwd_launch(int cdim, bool dyn, const Eval3dParams& p, hipStream_t s);
// per-CDIM backward launcher, instantiated for each supported CDIM by eval3d_bwd_g<k>.hip
template <int CDIM>
int eval3d_bwd_cdim(bool dyn, bool ray_grads, const Eval3dParams& p, hipStream_t s);

}  // namespace xsg
