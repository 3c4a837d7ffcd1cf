// C-ABI entry points of the eval3d compositor and the per-Gaussian backward epilogue.
#include <algorithm>
#include <cstdint>

#include "xsg_eval3d.h"

namespace xsg {
namespace {

constexpr int kBlock = 256;

// Zero fill of up to five float arrays, a group of workgroups each: 16-byte stores over the aligned
// body, single floats before and after it.
struct ZeroList {
    float* p[5];
    int64_t n[5];
};

// Workgroup g of `groups` workgroups (blockDim.x threads each) clearing array `list`.
XSG_DEV void zero_part(const ZeroList& z, int list, int g, int groups) {
    float* __restrict__ p = z.p[list];
    const int64_t n = z.n[list];
    if (!p || n <= 0) return;
    const int64_t head = min<int64_t>(n, (int64_t)(((16 - ((uintptr_t)p & 15)) & 15) / 4));
    const int64_t n4 = (n - head) / 4;
    const int64_t tail = head + 4 * n4;
    const int64_t stride = (int64_t)groups * blockDim.x;
    const int64_t t0 = (int64_t)g * blockDim.x + threadIdx.x;
    if (t0 < head) p[t0] = 0.f;
    if (t0 < n - tail) p[tail + t0] = 0.f;
    float4* __restrict__ p4 = reinterpret_cast<float4*>(p + head);
    for (int64_t i = t0; i < n4; i += stride) p4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

// quat_scale_to_preci_half_vjp + quat_to_rotmat_vjp (utils.h:208-263) applied once per Gaussian to
// the accumulated Q = sum over pairs of v_grd (x) grd + v_gro (x) gro, which is symmetric and kept
// as its upper triangle (Q_00, Q_01, Q_02, Q_11, Q_12, Q_22; index i is the row of M = S^-1 R^T).
// With rd = R S grd and o - mu = R S gro, dL/dM_ir = sum_k Q_ik s_k R_rk; the scale gradient is
// -Q_ii / s_i.
__global__ __launch_bounds__(kBlock) void bwd_epilogue_kernel(int64_t n, const float4* __restrict__ quats,
                                                              const float* __restrict__ scales,
                                                              const float* __restrict__ qacc,
                                                              float4* __restrict__ v_quats,
                                                              float* __restrict__ v_scales) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const float* qa = qacc + 6 * i;
    const float2 q01 = *reinterpret_cast<const float2*>(qa), q23 = *reinterpret_cast<const float2*>(qa + 2),
                 q45 = *reinterpret_cast<const float2*>(qa + 4);
    if (q01.x == 0.f && q01.y == 0.f && q23.x == 0.f && q23.y == 0.f && q45.x == 0.f && q45.y == 0.f) {
        // no pair reached this Gaussian (most of them): zero gradients without reading its shape
        v_quats[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        v_scales[3 * i] = 0.f; v_scales[3 * i + 1] = 0.f; v_scales[3 * i + 2] = 0.f;
        return;
    }
    const float4 q = quats[i];
    float w = q.x, x = q.y, y = q.z, z = q.w;
    const float inv_norm = rsqrtf(x * x + y * y + z * z + w * w);
    x *= inv_norm; y *= inv_norm; z *= inv_norm; w *= inv_norm;
    const float sc[3] = {scales[3 * i], scales[3 * i + 1], scales[3 * i + 2]};
    const float s[3] = {1.0f / sc[0], 1.0f / sc[1], 1.0f / sc[2]};
    // R columns (glm R[c], R[c][r] = R_rc) from quat_to_rotmat (utils.h:61-83)
    const float x2 = x * x, y2 = y * y, z2 = z * z, xy = x * y, xz = x * z, yz = y * z;
    const float wx = w * x, wy = w * y, wz = w * z;
    const float R[3][3] = {{1.f - 2.f * (y2 + z2), 2.f * (xy + wz), 2.f * (xz - wy)},
                           {2.f * (xy - wz), 1.f - 2.f * (x2 + z2), 2.f * (yz + wx)},
                           {2.f * (xz + wy), 2.f * (yz - wx), 1.f - 2.f * (x2 + y2)}};
    const float Q[3][3] = {{q01.x, q01.y, q23.x}, {q01.y, q23.y, q45.x}, {q23.x, q45.x, q45.y}};
    float vm[3][3];  // glm v_M[c][r]: dL/dM for row c of M, component r
#pragma unroll
    for (int cc = 0; cc < 3; ++cc)
#pragma unroll
        for (int r = 0; r < 3; ++r)
            vm[cc][r] = Q[cc][0] * sc[0] * R[0][r] + Q[cc][1] * sc[1] * R[1][r] + Q[cc][2] * sc[2] * R[2][r];
    // v_R = v_M * S  -> glm v_R[c][r] = v_M[c][r] * s_c
    float V[3][3];
#pragma unroll
    for (int cc = 0; cc < 3; ++cc)
#pragma unroll
        for (int r = 0; r < 3; ++r) V[cc][r] = vm[cc][r] * s[cc];
    float vq[4];
    vq[0] = 2.f * (x * (V[1][2] - V[2][1]) + y * (V[2][0] - V[0][2]) + z * (V[0][1] - V[1][0]));
    vq[1] = 2.f * (-2.f * x * (V[1][1] + V[2][2]) + y * (V[0][1] + V[1][0]) + z * (V[0][2] + V[2][0]) +
                   w * (V[1][2] - V[2][1]));
    vq[2] = 2.f * (x * (V[0][1] + V[1][0]) - 2.f * y * (V[0][0] + V[2][2]) + z * (V[1][2] + V[2][1]) +
                   w * (V[2][0] - V[0][2]));
    vq[3] = 2.f * (x * (V[0][2] + V[2][0]) + y * (V[1][2] + V[2][1]) - 2.f * z * (V[0][0] + V[1][1]) +
                   w * (V[0][1] - V[1][0]));
    const float qn[4] = {w, x, y, z};
    const float dp = vq[0] * qn[0] + vq[1] * qn[1] + vq[2] * qn[2] + vq[3] * qn[3];
    v_quats[i] = make_float4((vq[0] - dp * qn[0]) * inv_norm, (vq[1] - dp * qn[1]) * inv_norm,
                             (vq[2] - dp * qn[2]) * inv_norm, (vq[3] - dp * qn[3]) * inv_norm);
#pragma unroll
    for (int cc = 0; cc < 3; ++cc) v_scales[3 * i + cc] = -Q[cc][cc] * s[cc];
}

// Launch order of the backward's tiles. A tile's backward work is about the number of its Gaussians
// from its first intersection up to the largest last id of its pixels (compositing stops there for
// every pixel), and tiles differ by a factor of two or more; with about three tiles per wave slot,
// the heavy tiles that happen to start last set the kernel's end. Each XCD keeps the same contiguous
// run of tiles (xcd_tile: neighbouring tiles share their Gaussians in its L2) and launches it heaviest
// first.
//
// tile_work_kernel: one wavefront per (camera, tile), the largest last id of the tile's pixels.
__global__ __launch_bounds__(kBlock) void tile_work_kernel(TileGrid g, const int32_t* __restrict__ last_ids,
                                                           const int32_t* __restrict__ offsets,
                                                           int32_t* __restrict__ work) {
    const int n_tiles = g.n_tiles_w * g.n_tiles_h;
    const int nblocks = n_tiles * g.n_cams;
    const int t = blockIdx.x * (kBlock / 64) + (int)(threadIdx.x >> 6);
    if (t >= nblocks) return;  // wave-uniform
    const int cam = t / n_tiles, tile = t - cam * n_tiles;
    const int trow = tile / g.n_tiles_w, tcol = tile - trow * g.n_tiles_w;
    const int bs = g.tile_w * g.tile_h;
    const int64_t hw = (int64_t)g.width * g.height;
    int m = -1;
    for (int qi = __lane_id(); qi < bs; qi += 64) {
        const int ty = qi / g.tile_w, tx = qi - ty * g.tile_w;
        const int i = trow * g.tile_h + ty, j = tcol * g.tile_w + tx;
        if (i < g.height && j < g.width) m = max(m, last_ids[(int64_t)cam * hw + (int64_t)i * g.width + j]);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = max(m, __shfl_xor(m, off, 64));
    if (__lane_id() == 0) {
        const int32_t rs = offsets[t];
        const int32_t re = (t == nblocks - 1) ? (int32_t)g.n_isects : offsets[t + 1];
        work[t] = max(0, min(re - 1, m) - rs + 1);
    }
}

// The tile order: one workgroup of kOrderThreads per XCD (8). XCD x runs the logical blocks
// [x q + min(x, r), + q + (x < r)) of xcd_tile; they are placed heaviest first by a counting sort on
// the top 8 bits of the work (LDS histogram, scan, scatter; ties in no particular order). Negative
// estimates count as zero, so that any values give a permutation.
constexpr int kOrderThreads = 1024;
XSG_DEV void tile_order_part(int x, int nblocks, const int32_t* __restrict__ work, int32_t* __restrict__ order) {
    __shared__ int hist[256];
    __shared__ int wmax[kOrderThreads / 64];
    const int q = nblocks >> 3, r = nblocks & 7;
    const int s0 = x * q + min(x, r), cnt = q + (x < r ? 1 : 0);
    int mx = 0;
    for (int i = threadIdx.x; i < cnt; i += kOrderThreads) mx = max(mx, work[s0 + i]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = max(mx, __shfl_xor(mx, off, 64));
    if (__lane_id() == 0) wmax[threadIdx.x >> 6] = mx;
    if (threadIdx.x < 256) hist[threadIdx.x] = 0;
    __syncthreads();
    mx = 0;
#pragma unroll
    for (int k = 0; k < kOrderThreads / 64; ++k) mx = max(mx, wmax[k]);
    const int shift = max(0, 32 - __clz(mx) - 8);  // work >> shift < 256
    for (int i = threadIdx.x; i < cnt; i += kOrderThreads) atomicAdd(&hist[255 - (max(0, work[s0 + i]) >> shift)], 1);
    __syncthreads();
    if (threadIdx.x < 64) {  // exclusive scan of the 256 bins: four per lane, then across the wavefront
        const int l = threadIdx.x;
        const int a0 = hist[4 * l], a1 = hist[4 * l + 1], a2 = hist[4 * l + 2], a3 = hist[4 * l + 3];
        const int sum = a0 + a1 + a2 + a3;
        int inc = sum;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int v = __shfl_up(inc, off, 64);
            if (l >= off) inc += v;
        }
        const int ex = inc - sum;
        hist[4 * l] = ex;
        hist[4 * l + 1] = ex + a0;
        hist[4 * l + 2] = ex + a0 + a1;
        hist[4 * l + 3] = ex + a0 + a1 + a2;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < cnt; i += kOrderThreads) {
        const int pos = atomicAdd(&hist[255 - (max(0, work[s0 + i]) >> shift)], 1);
        order[s0 + pos] = s0 + i;
    }
}

// The backward's set-up in one launch of kOrderThreads-thread workgroups: workgroups [0, n_order) (8,
// or 0 without tiles) order one XCD's tiles each, the others clear the accumulated outputs,
// zero_groups workgroups per array.
__global__ __launch_bounds__(kOrderThreads) void bwd_prep_kernel(ZeroList z, int zero_groups, int n_order,
                                                                 int nblocks, const int32_t* __restrict__ work,
                                                                 int32_t* __restrict__ order) {
    const int b = (int)blockIdx.x;
    if (b < n_order) {
        tile_order_part(b, nblocks, work, order);
    } else {
        zero_part(z, (b - n_order) / zero_groups, (b - n_order) % zero_groups, zero_groups);
    }
}

struct BwdWorkspace {
    size_t order_off, work_off, bytes;
};

constexpr size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

BwdWorkspace bwd_workspace(int64_t n, int64_t nblocks) {
    BwdWorkspace w;
    w.work_off = align256((size_t)(n > 0 ? n : 1) * 6 * sizeof(float));
    w.order_off = w.work_off + align256((size_t)(nblocks > 0 ? nblocks : 1) * sizeof(int32_t));
    w.bytes = w.order_off + align256((size_t)(nblocks > 0 ? nblocks : 1) * sizeof(int32_t));
    return w;
}

bool cdim_supported(int c) {
    switch (c) {
#define XSG_CASE(C) case C: return true;
        XSG_CDIM_LIST(XSG_CASE)
#undef XSG_CASE
        default: return false;
    }
}

int fill_params(const xsg_eval3d_args* a, Eval3dParams& p, const char* who) {
    if (!a) return xsg_fail(XSG_ERR_INVALID, "%s: null arguments", who);
    if (!cdim_supported(a->cdim)) return xsg_fail(XSG_ERR_INVALID, "Unsupported number of channels: %d", a->cdim);
    if (a->tile_w <= 0 || a->tile_h <= 0 || a->width < 0 || a->height < 0 || a->n_cams < 1 || a->n < 0 ||
        a->n_isects < 0 || a->n_tiles_w <= 0 || a->n_tiles_h <= 0)
        return xsg_fail(XSG_ERR_INVALID, "%s: invalid sizes", who);
    if (a->tile_w * a->tile_h > kMaxTilePixels)
        return xsg_fail(XSG_ERR_LDS, "Failed to set maximum shared memory size (tile %dx%d has more than %d pixels), "
                        "try lowering tile_size.", a->tile_w, a->tile_h, kMaxTilePixels);
    if ((int64_t)a->n_tiles_w * a->tile_w < a->width || (int64_t)a->n_tiles_h * a->tile_h < a->height)
        return xsg_fail(XSG_ERR_INVALID, "%s: tile grid %dx%d of %dx%d tiles does not cover %dx%d pixels", who,
                        a->n_tiles_w, a->n_tiles_h, a->tile_w, a->tile_h, a->width, a->height);
    if ((int64_t)a->n_cams * a->n_tiles_w * a->n_tiles_h > INT32_MAX)
        return xsg_fail(XSG_ERR_INVALID, "%s: %d cameras x %dx%d tiles exceed the launch grid", who, a->n_cams,
                        a->n_tiles_w, a->n_tiles_h);
    if ((int64_t)a->n_cams * a->n > INT32_MAX)
        return xsg_fail(XSG_ERR_INVALID, "%s: %d cameras x %lld Gaussians exceed the int32 flatten ids", who,
                        a->n_cams, (long long)a->n);
    if (a->cdim > 0 && !a->colors) return xsg_fail(XSG_ERR_INVALID, "%s: colors missing for cdim %d", who, a->cdim);
    if (!a->means || !a->quats || !a->scales || !a->opacities || !a->ray_o || !a->ray_d || !a->tile_offsets ||
        (a->n_isects > 0 && !a->flatten_ids))
        return xsg_fail(XSG_ERR_INVALID, "%s: null input", who);
    p = Eval3dParams{};
    p.g = TileGrid{a->width, a->height, a->tile_w, a->tile_h, a->n_tiles_w, a->n_tiles_h, a->n_cams, a->n,
                   a->n_isects};
    p.means = a->means; p.quats = (const float4*)a->quats; p.scales = a->scales; p.colors = a->colors;
    p.opac = a->opacities; p.velocity = a->velocity; p.rtd = a->ray_time_delta;
    p.ray_o = a->ray_o; p.ray_d = a->ray_d; p.offsets = a->tile_offsets; p.flatten = a->flatten_ids;
    p.col_shift = a->colors_shared ? a->n * a->cdim : 0;
    if (a->bwd_pixels_per_lane != 0 && a->bwd_pixels_per_lane != 2 && a->bwd_pixels_per_lane != 4)
        return xsg_fail(XSG_ERR_INVALID, "%s: bwd_pixels_per_lane must be 0, 2 or 4 (got %d)", who,
                        a->bwd_pixels_per_lane);
    p.px_hint = a->bwd_pixels_per_lane;
    return XSG_OK;
}

}  // namespace
}  // namespace xsg

using namespace xsg;

extern "C" int xsg_eval3d_supported_ndims(int* out, int cap) {
    static const int dims[] = {
#define XSG_ITEM(C) C,
        XSG_CDIM_LIST(XSG_ITEM)
#undef XSG_ITEM
    };
    const int n = (int)(sizeof(dims) / sizeof(dims[0]));
    for (int i = 0; i < n && i < cap && out; ++i) out[i] = dims[i];
    return n;
}

extern "C" int xsg_eval3d_fwd(const xsg_eval3d_args* a, xsg_stream_t stream) {
    Eval3dParams p;
    int rc = fill_params(a, p, "xsg_eval3d_fwd");
    if (rc) return rc;
    if (!a->out_depth || !a->out_alpha || !a->out_last_ids || (a->cdim > 0 && !a->out_rgb))
        return xsg_fail(XSG_ERR_INVALID, "xsg_eval3d_fwd: null output");
    if ((int64_t)a->width * a->height == 0) return XSG_OK;
    p.out_rgb = a->out_rgb; p.out_depth = a->out_depth; p.out_alpha = a->out_alpha; p.out_last = a->out_last_ids;
    p.pair_counts = (unsigned long long*)a->pair_counts;
    p.tile_work = a->tile_work;
    const bool dyn = a->velocity != nullptr || a->ray_time_delta != nullptr;
    rc = eval3d_fwd_launch(a->cdim, dyn, p, (hipStream_t)stream);
    if (rc) return rc;
    XSG_TRY_LAUNCH("eval3d_fwd");
    return XSG_OK;
}

extern "C" size_t xsg_eval3d_bwd_workspace_bytes(const xsg_eval3d_args* a) {
    if (!a) return 0;
    const int64_t nblocks = (int64_t)std::max(a->n_cams, 0) * std::max(a->n_tiles_w, 0) * std::max(a->n_tiles_h, 0);
    return bwd_workspace(a->n, nblocks).bytes;
}

extern "C" int xsg_eval3d_bwd(const xsg_eval3d_args* a, void* workspace, xsg_stream_t stream) {
    Eval3dParams p;
    int rc = fill_params(a, p, "xsg_eval3d_bwd");
    if (rc) return rc;
    const bool dyn = a->velocity != nullptr;
    if (dyn && !a->ray_time_delta)
        return xsg_fail(XSG_ERR_INVALID, "dynamic backward needs both velocity and ray_time_delta");
    if (!a->render_alpha || !a->last_ids || !a->v_depth || !a->v_alpha || (a->cdim > 0 && !a->v_rgb) ||
        !a->v_means || !a->v_quats || !a->v_scales || !a->v_opacities || (a->cdim > 0 && !a->v_colors) ||
        ((a->v_ray_o == nullptr) != (a->v_ray_d == nullptr)) ||
        (dyn && (!a->v_velocity || !a->v_time_delta)) || !workspace)
        return xsg_fail(XSG_ERR_INVALID, "xsg_eval3d_bwd: null buffer");
    if ((rc = xsg_check_workspace(workspace, "xsg_eval3d_bwd"))) return rc;
    const hipStream_t s = (hipStream_t)stream;
    p.render_alpha = a->render_alpha; p.last_ids = a->last_ids; p.v_rgb = a->v_rgb; p.v_depth = a->v_depth;
    p.v_alpha = a->v_alpha; p.v_means = a->v_means; p.v_opac = a->v_opacities; p.v_colors = a->v_colors;
    p.v_ray_o = a->v_ray_o; p.v_ray_d = a->v_ray_d; p.v_velocity = a->v_velocity; p.v_time = a->v_time_delta;
    p.v_mt = (float*)workspace;
    p.pair_counts = (unsigned long long*)a->pair_counts;
    const int64_t n = a->n;
    const int64_t ncol = a->cdim > 0 ? (a->colors_shared ? 1 : (int64_t)a->n_cams) * n * a->cdim : 0;
    const ZeroList zl{{a->v_means, a->v_opacities, a->v_colors, p.v_mt, dyn ? a->v_velocity : nullptr},
                      {3 * n, n, ncol, 6 * n, dyn ? 3 * n : 0}};
    int64_t longest = 0;
    for (int k = 0; k < 5; ++k) longest = std::max(longest, zl.n[k]);
    const int zero_groups =
        (int)std::min<int64_t>((longest / 4 + kOrderThreads - 1) / kOrderThreads + 1, 256);
    const bool pixels = (int64_t)a->width * a->height > 0;
    const int nblocks = a->n_cams * a->n_tiles_w * a->n_tiles_h;
    const BwdWorkspace w = bwd_workspace(n, nblocks);
    int32_t* work = reinterpret_cast<int32_t*>((char*)workspace + w.work_off);
    int32_t* order = reinterpret_cast<int32_t*>((char*)workspace + w.order_off);
    if (pixels) {
        if (a->tile_work)  // written by the forward
            work = a->tile_work;
        else
            tile_work_kernel<<<(unsigned)((nblocks + kBlock / 64 - 1) / (kBlock / 64)), kBlock, 0, s>>>(
                p.g, a->last_ids, a->tile_offsets, work);
    }
    const int n_order = pixels ? 8 : 0;
    if (n_order > 0 || longest > 0)
        bwd_prep_kernel<<<(unsigned)(n_order + (longest > 0 ? 5 * zero_groups : 0)), kOrderThreads, 0, s>>>(
            zl, zero_groups, n_order, nblocks, work, order);
    if (pixels) {
        p.tile_order = order;
        rc = eval3d_bwd_launch(a->cdim, dyn, p, s);
        if (rc) return rc;
    }
    if (n > 0)
        bwd_epilogue_kernel<<<(unsigned)((n + kBlock - 1) / kBlock), kBlock, 0, s>>>(
            n, (const float4*)a->quats, a->scales, p.v_mt, (float4*)a->v_quats, a->v_scales);
    XSG_TRY_LAUNCH("eval3d_bwd");
    return XSG_OK;
}
