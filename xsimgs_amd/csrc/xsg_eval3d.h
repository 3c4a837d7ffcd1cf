// eval3d compositing kernels (reference csrc/rasterization/eval3d_{fwd,bwd}.cu, eval3d_dynamic_*.cu).
//
// One workgroup per (camera, tile); one thread per pixel (tile_w * tile_h <= 256 threads, i.e. up
// to four wave64s). Gaussians of the tile's depth-sorted list are staged in LDS in batches of one
// per thread. Per staged Gaussian the LDS slot holds M = S^-1 R^T (three rows) and, when every ray
// of the tile starts at the same origin (decided by a block vote, always true for a static pinhole
// or spherical camera), gro = M (o - mu): the per-pair work then only maps the ray direction.
// These are the values the reference computes per pair, so results do not depend on the path.
#pragma once
#include "xsg_common.h"

namespace xsg {

constexpr int kTileThreads = 256;
constexpr int kColorLdsMax = 16;  // colour channels staged in LDS; larger CDIM read from HBM

#define XSG_CDIM_LIST(X) \
    X(0) X(1) X(2) X(3) X(4) X(5) X(8) X(9) X(16) X(17) X(32) X(33) X(64) X(65) X(128) X(129) \
    X(256) X(257) X(512) X(513)

struct TileGrid {
    int width, height, tile_w, tile_h, n_tiles_w, n_tiles_h, n_cams;
    int64_t n;          // Gaussians (flatten id = cam * n + gaussian)
    int64_t n_isects;
};

// Workgroups are dispatched round-robin over the 8 XCDs; give each XCD a contiguous run of tiles so
// that neighbouring tiles, which share most of their Gaussians, share an L2.
XSG_DEV int xcd_tile(int b, int nblocks) {
    const int x = b & 7, q = nblocks >> 3, r = nblocks & 7;
    return x * q + min(x, r) + (b >> 3);
}

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
    c.inside = c.i < g.height && c.j < g.width;
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

// Lane-to-lane moves inside rows of 16 lanes (DPP). `update_dpp` with all rows/banks enabled and
// in-bounds patterns returns the source lane's value for every lane.
template <int CTRL>
XSG_DEV float dpp_mov(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
constexpr int kDppQuadSwap1 = 0xB1;    // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuadSwap2 = 0x4E;    // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppRowMirror = 0x140;   // lane i <-> 15 - i within a row of 16
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within each half row of 8

// One halving step with the gfx950 lane-swap instructions. v_permlane32_swap(x, y) exchanges
// lanes 32-63 of x with lanes 0-31 of y; v_permlane16_swap(x, y) exchanges the odd 16-lane rows
// of x with the even rows of y. With x = the component a lower lane keeps and y = the one its
// partner keeps, afterwards x + y is, on every lane, its kept component summed over the pair.
XSG_DEV float swap_add32(float keep_lo, float keep_hi) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(keep_lo), __float_as_uint(keep_hi), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
XSG_DEV float swap_add16(float keep_lo, float keep_hi) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(keep_lo), __float_as_uint(keep_hi), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Reduce-scatter of 16 per-lane values over the 64 lanes of a wavefront by recursive halving:
// each step pairs every lane with a partner, keeps half of its values and adds the partner's
// copy of that half. Partners at distance 32 and 16 exchange through lane swaps (lanes 0-31 keep
// v[0..7], lanes 16-31 of each half keep the upper half of what is left), then the row and
// half-row mirrors (DPP) and a final quad sum: lane l holds the wave total of value l >> 2.
// Must be called with all 64 lanes active.
XSG_DEV float wave_reduce_scatter16(const float (&v)[16]) {
    const int lane = __lane_id();
    float w[8], x[4], y[2];
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = swap_add32(v[j], v[j + 8]);
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = swap_add16(w[j], w[j + 4]);
    {
        const bool up = (lane & 15) >= 8;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float send = up ? x[j] : x[j + 2];
            const float keep = up ? x[j + 2] : x[j];
            y[j] = keep + dpp_mov<kDppRowMirror>(send);
        }
    }
    float z;
    {
        const bool up = (lane & 7) >= 4;
        const float send = up ? y[0] : y[1];
        const float keep = up ? y[1] : y[0];
        z = keep + dpp_mov<kDppHalfMirror>(send);
    }
    z += dpp_mov<kDppQuadSwap2>(z);
    z += dpp_mov<kDppQuadSwap1>(z);
    return z;
}

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
    float* v_mt;         // workspace [n, 9]: sum of dL/dM^T per Gaussian (row-major of M^T)
    unsigned long long* pair_counts;  // forward, optional: += [evaluated, contributing] pairs
};

int eval3d_fwd_launch(int cdim, bool dyn, const Eval3dParams& p, hipStream_t s);
int eval3d_bwd_launch(int cdim, bool dyn, const Eval3dParams& p, hipStream_t s);

}  // namespace xsg
