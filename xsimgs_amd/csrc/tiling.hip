// Tile binning: per-Gaussian tile rectangles, intersection keys, stable sort, per-tile ranges.
//
// Reference: csrc/tiling/regular_tiling.cu, phm_lidar_tiling.cu, phm_spherical_tiling.cu,
// tiling_common.cu(h), mask_radii.cu.
//
// The reference sorts 64-bit keys (tile << 32 | depth bits) over bits [0, 32 + tile_n_bits) with a
// stable radix sort whose input is in Gaussian order. This build produces the identical arrays
// with less traffic:
//   1. count  : one thread per Gaussian instance computes its tile rectangle(s) (the seam spans of
//               lidar / spherical flag-2 Gaussians are re-projected densely by seam_span_kernel)
//               and writes tiles_per_gauss plus the rectangles; a two-level scan of the block
//               partials gives every compaction block its offset, and the totals are published.
//   2. compact: one packed 64-bit scan ((count > 0) << 32 | count) gives every visible
//               instance both its intersection offset and its rank among visible instances.
//   3. depth  : the visible instances are sorted stably by the low 32 key bits (depth bits).
//   4. runs   : every depth-ordered instance is cut into row runs (one per tile row it covers),
//               written with their records, and sorted stably by row bucket (camera, row).
//   5. write  : per row segment, column counts give every (tile, segment) its first output
//               position; the writers store keys and flattened ids in (camera, tile, depth) order.
// Stable by (high bits, low bits, Gaussian order) in both cases, so the result is bit-identical
// to sorting the reference keys; ties keep Gaussian order as the reference's fill does.
#include <algorithm>
#include <atomic>
#include <vector>

#include "xsg_sort.h"

UtWeights xsg_ut_weights(float a, float b, float k);

namespace {
using namespace xsg;

constexpr int kBlock = 256;
constexpr int kExpandPerBlock = 1024;
// keys per thread of the run sort (one or two passes over the row runs); an expansion block writes
// exactly one tile of it, with that tile's first-digit histogram
constexpr int kRunSortItems = 4;
// Digit width of the run sort: one pass of 8, 9 or 10 bits for up to 1024 row buckets (a rig of several
// cameras), 8-bit passes beyond.
inline int run_sort_rb(int row_bits) { return row_bits <= 8 ? 8 : row_bits <= 10 ? row_bits : 8; }
constexpr int kMaxLdsElev = 1024;  // lidar elevation boundaries staged in LDS by the count pass
constexpr int kMaxLdsRows = 8192;  // row buckets whose segment bases row_segments_kernel searches in LDS

struct Rect { uint16_t x0, y0, x1, y1; };  // exclusive [x0, x1) x [y0, y1)

XSG_DEV uint32_t rect_count(Rect r) { return (uint32_t)(r.x1 - r.x0) * (uint32_t)(r.y1 - r.y0); }
XSG_DEV uint64_t pack_count(uint32_t c) { return ((uint64_t)(c > 0) << 32) | (uint64_t)c; }

// regular_tiling.cu:35-56
XSG_DEV Rect regular_rect(float2 m, float2 r, float tsx, float tsy, int ntx, int nty) {
    Rect out = {0, 0, 0, 0};
    if (r.x <= 0 || r.y <= 0) return out;
    const float mx = m.x / tsx, my = m.y / tsy;
    const float rx = r.x / tsx, ry = r.y / tsy;
    out.x0 = (uint16_t)min(ntx, max(0, (int)floorf(mx - rx)));
    out.y0 = (uint16_t)min(nty, max(0, (int)floorf(my - ry)));
    out.x1 = (uint16_t)min(ntx, max(0, (int)ceilf(mx + rx)));
    out.y1 = (uint16_t)min(nty, max(0, (int)ceilf(my + ry)));
    return out;
}

// First index at or after i whose boundary is not below v (n_elev if none), scanning up the table as
// find_bounds_increasing does (phm_lidar_tiling.cu:35-60).
XSG_DEV int elev_scan_up(const float* elev, int n_elev, int i, float v) {
    while (i < n_elev && elev[i] < v) ++i;
    return i;
}
// The same index by bisection, for a table known to be non-decreasing: the first index of [i, n_elev)
// whose boundary is not below v. (A NaN v stops both at i.)
XSG_DEV int elev_search_up(const float* elev, int n_elev, int i, float v) {
    int lo = i, hi = n_elev;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (elev[mid] < v) lo = mid + 1; else hi = mid;
    }
    return lo;
}

// find_bounds_increasing + tile_limits_irregular (phm_lidar_tiling.cu:35-91), inclusive bounds
// returned as an exclusive rectangle. SORTED: the table is non-decreasing, so its two scans are done
// by bisection with the same results.
template <bool SORTED = false>
XSG_DEV Rect lidar_rect(float mx, float my, float rx, float ry, float u_min, float u_max, float u_per_tile,
                        int n_elev, const float* __restrict__ elev, int ntx) {
    Rect out = {0, 0, 0, 0};
    const float lo = fmaxf(mx - rx, u_min), hi = fminf(mx + rx, u_max);
    if (hi <= lo) return out;
    const int x0 = (int)floorf(lo / u_per_tile);
    const int x1 = (int)ceilf(hi / u_per_tile) - 1;
    const float vmin = my - ry, vmax = my + ry;
    int i = SORTED ? elev_search_up(elev, n_elev, 0, vmin) : elev_scan_up(elev, n_elev, 0, vmin);
    const int y0 = min(max(i - 1, 0), n_elev - 1);
    i = SORTED ? elev_search_up(elev, n_elev, i, vmax) : elev_scan_up(elev, n_elev, i, vmax);
    const int y1 = min(max(i - 1, 0), n_elev - 1);
    out.x0 = (uint16_t)min(x0, ntx); out.x1 = (uint16_t)min(x1 + 1, ntx);
    out.y0 = (uint16_t)y0; out.y1 = (uint16_t)(y1 + 1);
    return out;
}

// tile_limits_regular (phm_spherical_tiling.cu:15-45)
XSG_DEV Rect spherical_rect(float mx, float my, float rx, float ry, float u_min, float u_max, float u_per_tile,
                            int n_v, float v_per_tile, int ntx) {
    Rect out = {0, 0, 0, 0};
    const float lo = fmaxf(mx - rx, u_min), hi = fminf(mx + rx, u_max);
    if (hi <= lo) return out;
    out.x0 = (uint16_t)min((int)floorf(lo / u_per_tile), ntx);
    out.y0 = (uint16_t)min(n_v, max(0, (int)floorf((my - ry) / v_per_tile)));
    out.x1 = (uint16_t)min((int)ceilf(hi / u_per_tile), ntx);
    out.y1 = (uint16_t)min(n_v, max(0, (int)ceilf((my + ry) / v_per_tile)));
    return out;
}

struct Geometry {
    int kind, n_cams;
    int64_t n;          // Gaussians per camera
    int ntx, nty;       // tiles along u / v
    int n_tiles;
    int tnb;            // tile_n_bits
    int cam_bits;
    int spans;          // virtual instances per Gaussian instance: 1 (regular) or 2 (seam split)
    int sort;           // the fill sorts (the count pass orders the spans by depth)
};

// Blocks of the count-phase kernels (count, compaction, row-run offsets): 1024 virtual instances,
// four per thread, so that a 1 M-Gaussian pass spreads over about a thousand workgroups.
constexpr int kCountItems = 4;
constexpr int kCountTile = kBlock * kCountItems;

// Smallest and largest of the threads' (lo, hi) over a 256-thread block, on thread 0 (the block's
// range of visible depth keys, which the depth pre-order's first digit is taken from).
XSG_DEV void block_key_range(uint32_t& lo, uint32_t& hi, uint32_t* s_lo, uint32_t* s_hi) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        lo = min(lo, (uint32_t)__shfl_xor((int)lo, off, 64));
        hi = max(hi, (uint32_t)__shfl_xor((int)hi, off, 64));
    }
    if (__lane_id() == 0) { s_lo[threadIdx.x >> 6] = lo; s_hi[threadIdx.x >> 6] = hi; }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 1; w < kWaves; ++w) { lo = min(lo, s_lo[w]); hi = max(hi, s_hi[w]); }
    }
}

// Orders one wavefront's LDS accesses before and after it (a wavefront-private LDS buffer needs no
// workgroup barrier, only this).
XSG_DEV void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Sums of three 64-bit values over a 256-thread block, on every thread (one barrier pair for all three).
XSG_DEV void block_reduce_sum3(uint64_t& a, uint64_t& b, uint64_t& c, uint64_t (*lds)[kWaves]) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        a += (uint64_t)__shfl_xor((unsigned long long)a, off, 64);
        b += (uint64_t)__shfl_xor((unsigned long long)b, off, 64);
        c += (uint64_t)__shfl_xor((unsigned long long)c, off, 64);
    }
    const int wave = threadIdx.x >> 6;
    if (__lane_id() == 0) { lds[0][wave] = a; lds[1][wave] = b; lds[2][wave] = c; }
    __syncthreads();
    a = b = c = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) { a += lds[0][w]; b += lds[1][w]; c += lds[2][w]; }
    __syncthreads();
}

// Count pass over regular-tiling Gaussian instances (one span each). A block covers kCountTile
// instances; it writes tiles_per_gauss and the rectangle of every instance, and the block's packed
// count sum. The compaction takes the counts from tiles_per_gauss and the depth bits from the depths.
// With key_range (the bucketed depth pre-order), also the block's range of visible depth keys.
__global__ __launch_bounds__(kBlock) void count_regular_kernel(
    int64_t n_total, const float2* __restrict__ means2d, const float2* __restrict__ radii, float tsx, float tsy,
    int ntx, int nty, int32_t* __restrict__ tpg, Rect* __restrict__ rects, uint64_t* __restrict__ partials,
    uint64_t* __restrict__ cpart, const float* __restrict__ depths, uint32_t* __restrict__ key_range) {
    __shared__ uint64_t lds[3][kWaves];
    __shared__ uint32_t s_lo[kWaves], s_hi[kWaves];
    uint64_t acc = 0, acc_c = 0, acc_r = 0;
    uint32_t lo = 0xffffffffu, hi = 0u;
    const int64_t base = (int64_t)blockIdx.x * kCountTile;
    // every item's inputs loaded before any is binned (one memory round trip instead of one per item;
    // indices past the end read the last instance and are not binned)
    float2 mv[kCountItems], rv[kCountItems];
    uint32_t kv[kCountItems];
#pragma unroll
    for (int k = 0; k < kCountItems; ++k) {
        const int64_t j = min(base + (int64_t)k * kBlock + threadIdx.x, n_total - 1);
        mv[k] = means2d[j];
        rv[k] = radii[j];
        kv[k] = key_range ? __float_as_uint(depths[j]) : 0u;
    }
#pragma unroll
    for (int k = 0; k < kCountItems; ++k) {
        const int64_t j = base + (int64_t)k * kBlock + threadIdx.x;
        if (j < n_total) {
            const Rect r = regular_rect(mv[k], rv[k], tsx, tsy, ntx, nty);
            const uint32_t c = rect_count(r);
            tpg[j] = (int32_t)c;  // also the compaction's count (one span per instance)
            rects[j] = r;
            acc += pack_count(c);
            acc_c += c;
            acc_r += c > 0 ? (uint32_t)(r.y1 - r.y0) : 0u;
            if (c > 0) {
                lo = min(lo, kv[k]);
                hi = max(hi, kv[k]);
            }
        }
    }
    block_reduce_sum3(acc, acc_c, acc_r, lds);
    if (key_range) block_key_range(lo, hi, s_lo, s_hi);  // block-uniform
    if (threadIdx.x == 0) {
        partials[blockIdx.x] = acc;
        cpart[2 * blockIdx.x] = acc_c;
        cpart[2 * blockIdx.x + 1] = acc_r;
        if (key_range) { key_range[2 * blockIdx.x] = lo; key_range[2 * blockIdx.x + 1] = hi; }
    }
}

// isect_lidar_tiles_kernel (phm_lidar_tiling.cu:96-234) / isect_spherical_tiles_kernel
// (phm_spherical_tiling.cu:47-174), count part: every Gaussian's first span (virtual instance 2j).
// A seam Gaussian (flag 2) is appended to a queue instead of being re-projected here: about one
// Gaussian in a hundred is one, so re-projecting inline would hold about half of the wavefronts for a
// whole UT; seam_span_kernel re-projects the queue densely and adds the second spans.
template <int KIND, bool LIDAR>
__global__ __launch_bounds__(kBlock) void count_spherical_kernel(
    int64_t n, const float* __restrict__ pack, f2 img, const uint8_t* __restrict__ flags,
    const float2* __restrict__ means2d, const float2* __restrict__ radii, const float* __restrict__ depths,
    const float* __restrict__ elev, int n_elev, float u_per_tile, float v_per_tile, int ntx, int n_v,
    int32_t* __restrict__ tpg, Rect* __restrict__ rects, uint32_t* __restrict__ vcnt, uint32_t* __restrict__ vkey,
    uint64_t* __restrict__ partials, uint64_t* __restrict__ cpart, uint32_t* __restrict__ seam_cnt,
    uint32_t* __restrict__ seam_ids, uint32_t* __restrict__ key_range) {
    __shared__ uint64_t lds[3][kWaves];
    __shared__ uint32_t s_lo[kWaves], s_hi[kWaves];
    __shared__ uint32_t s_seam;
    // every item's inputs loaded first, before the set-up below, and before any is binned (indices
    // past the end read the last Gaussian and are not binned)
    const int64_t base = (int64_t)blockIdx.x * (kCountTile / 2);
    constexpr int kItems = kCountItems / 2;
    float2 rv[kItems], mv[kItems];
    int fv[kItems];
    uint32_t kv[kItems];
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
        const int64_t j = min(base + (int64_t)k * kBlock + threadIdx.x, n - 1);
        rv[k] = radii[j];
        fv[k] = flags[j];
        mv[k] = means2d[j];
        kv[k] = __float_as_uint(depths[j]);
    }
    // lidar: the elevation table in LDS; when it is non-decreasing (as find_bounds_increasing
    // expects) its scans become bisections (same bounds), else they scan as the reference does
    __shared__ float s_elev[LIDAR ? kMaxLdsElev : 1];
    if (threadIdx.x == 0) s_seam = 0;
    bool sorted_elev = false;
    const float* tab = elev;
    if constexpr (LIDAR) {
        const bool fits = n_elev <= kMaxLdsElev;
        if (fits) {
            for (int i = threadIdx.x; i < n_elev; i += kBlock) s_elev[i] = elev[i];
            tab = s_elev;
        }
        __syncthreads();
        bool ok = fits;
        if (fits)
            for (int i = threadIdx.x; i + 1 < n_elev; i += kBlock) ok = ok && (s_elev[i] <= s_elev[i + 1]);
        sorted_elev = __syncthreads_and(ok) != 0;  // block-uniform
    } else {
        __syncthreads();
    }
    const Camera cam = load_camera(pack, KIND);
    const int lane = __lane_id();
    const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    uint64_t acc = 0, acc_c = 0, acc_r = 0;
    uint32_t lo = 0xffffffffu, hi = 0u;
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
        const int64_t j = base + (int64_t)k * kBlock + threadIdx.x;
        bool seam = false;
        if (j < n) {
            const float2 r = rv[k];
            const int flag = fv[k];
            Rect a = {0, 0, 0, 0};
            if (!(r.x <= 0 || r.y <= 0 || flag == 0)) {
                float u_min = 0.0f, u_max = 1.0f;
                if (flag == 2) {
                    seam = true;
                    if (cam.roll_u > 0) u_max = u_pose_of(cam); else u_min = u_pose_of(cam);
                }
                const float2 m = mv[k];
                const float mx = m.x / img.x, my = m.y / img.y, rx = r.x / img.x, ry = r.y / img.y;
                if (LIDAR) {
                    a = sorted_elev ? lidar_rect<true>(mx, my, rx, ry, u_min, u_max, u_per_tile, n_elev, tab, ntx)
                                    : lidar_rect<false>(mx, my, rx, ry, u_min, u_max, u_per_tile, n_elev, tab, ntx);
                } else {
                    a = spherical_rect(mx, my, rx, ry, u_min, u_max, u_per_tile, n_v, v_per_tile, ntx);
                }
            }
            const uint32_t ca = rect_count(a);
            tpg[j] = (int32_t)ca;
            // both spans of the instance, the second empty until seam_span_kernel fills it (one vector
            // store per array; the workspace arrays are 256-byte aligned)
            reinterpret_cast<uint4*>(rects)[j] =
                make_uint4((uint32_t)a.x0 | ((uint32_t)a.y0 << 16), (uint32_t)a.x1 | ((uint32_t)a.y1 << 16), 0u, 0u);
            reinterpret_cast<uint2*>(vcnt)[j] = make_uint2(ca, 0u);
            reinterpret_cast<uint2*>(vkey)[j] = make_uint2(kv[k], 0u);
            if (ca > 0) {
                lo = min(lo, kv[k]);
                hi = max(hi, kv[k]);
            }
            acc += pack_count(ca);
            acc_c += ca;
            acc_r += ca > 0 ? (uint32_t)(a.y1 - a.y0) : 0u;
        }
        // the block's seam Gaussians go to its own slice of the queue (one LDS slot reservation per
        // wavefront; their order there does not matter)
        const uint64_t sm = __ballot(seam);
        if (sm) {
            const int leader = (int)__builtin_ctzll(sm);
            uint32_t slot = 0;
            if (lane == leader) slot = atomicAdd(&s_seam, (uint32_t)__popcll(sm));
            slot = (uint32_t)__shfl((int)slot, leader, 64);
            if (seam) seam_ids[base + slot + (uint32_t)__popcll(sm & lt_mask)] = (uint32_t)j;
        }
    }
    block_reduce_sum3(acc, acc_c, acc_r, lds);  // its barriers also order the LDS reservations
    if (key_range) block_key_range(lo, hi, s_lo, s_hi);  // block-uniform
    if (threadIdx.x == 0) {
        partials[blockIdx.x] = acc;
        cpart[2 * blockIdx.x] = acc_c;
        cpart[2 * blockIdx.x + 1] = acc_r;
        seam_cnt[blockIdx.x] = s_seam;
        if (key_range) { key_range[2 * blockIdx.x] = lo; key_range[2 * blockIdx.x + 1] = hi; }
    }
}

// Second spans of the queued seam Gaussians (phm_lidar_tiling.cu:183-229): re-projected with
// PositiveDelta, binned past the tile boundary after u_pose and keyed with the re-projected depth
// (virtual instance 2j + 1). A workgroup takes the queues of kSeamBlocks consecutive count blocks (a
// few seam Gaussians each) and spreads them over its threads, one Gaussian per thread, so that the
// re-projections run on mostly full wavefronts; it alone adds those blocks' second spans to their
// partials, before the compaction reads them.
constexpr int kSeamBlocks = 16;

template <int KIND, bool LIDAR>
__global__ __launch_bounds__(kBlock) void seam_span_kernel(
    unsigned n_count_blocks, const uint32_t* __restrict__ seam_cnt, const uint32_t* __restrict__ seam_ids,
    const float* __restrict__ pack, UtWeights ut, f2 img, const float* __restrict__ points,
    const float* __restrict__ vel, const float* __restrict__ scales, const float4* __restrict__ quats,
    const float* __restrict__ opacity, const float* __restrict__ elev, int n_elev, float u_per_tile,
    float v_per_tile, int ntx, int n_v, int32_t* __restrict__ tpg, Rect* __restrict__ rects,
    uint32_t* __restrict__ vcnt, uint32_t* __restrict__ vkey, uint64_t* __restrict__ partials,
    uint64_t* __restrict__ cpart, uint32_t* __restrict__ key_range) {
    __shared__ uint32_t s_off[kSeamBlocks + 1];
    __shared__ uint32_t s_vis[kSeamBlocks], s_cnt[kSeamBlocks], s_rows[kSeamBlocks];
    __shared__ uint32_t s_klo[kSeamBlocks], s_khi[kSeamBlocks];
    const unsigned blk0 = blockIdx.x * kSeamBlocks;
    const int nb = (int)min<unsigned>(kSeamBlocks, n_count_blocks - blk0);
    if (threadIdx.x == 0) {
        uint32_t o = 0;
        for (int b = 0; b < nb; ++b) { s_off[b] = o; o += seam_cnt[blk0 + b]; }
        s_off[nb] = o;
    }
    if (threadIdx.x < kSeamBlocks) {
        s_vis[threadIdx.x] = 0; s_cnt[threadIdx.x] = 0; s_rows[threadIdx.x] = 0;
        s_klo[threadIdx.x] = 0xffffffffu; s_khi[threadIdx.x] = 0u;
    }
    __syncthreads();
    const uint32_t total = s_off[nb];
    if (total == 0) return;  // workgroup-uniform
    const Camera cam = load_camera(pack, KIND);
    const bool is_static = camera_is_static(cam, vel != nullptr);
    const PhaseUnwrap unwrap = phase_unwrap(cam);
    for (uint32_t q = threadIdx.x; q < total; q += kBlock) {
        int b = 0;
        while (b + 1 < nb && s_off[b + 1] <= q) ++b;
        const int64_t j = seam_ids[(int64_t)(blk0 + b) * (kCountTile / 2) + (q - s_off[b])];
        f3 d[3];
        ut_deltas(ut.sqrt_dl, quats[j], ld3(scales + 3 * j), d);
        const float op = opacity ? opacity[j] : 1.0f;
        const ProjParams pp{1e-4f, 0.002f, 1.0f};
        const f3 pw = ld3(points + 3 * j);
        f2 m2 = mk2(0.f, 0.f), r2 = mk2(0.f, 0.f);
        float dd = 0.f, ud = 0.f;
        bool ok;
        if (is_static) {
            // the phase-modelled projection's own static-pose path (ut_project_phm_kernel), so that
            // the re-projected depth -- the centre point's range, which no phase mode changes -- is
            // the stored depth bit for bit, as both spans' keys carry one depth in the reference
            SigmaUv sa;
            sigma_uv(cam, pw, d, sa);
            ok = ut_projection_sigma_uv(cam, unwrap, XSG_MODE_POSITIVE, ut, img, pp, ut_extend(op), sa, m2, r2, dd,
                                        ud);
        } else {
            const f3 pv = vel ? ld3(vel + 3 * j) : mk3(0.f, 0.f, 0.f);
            ok = ut_projection<KIND>(cam, XSG_MODE_POSITIVE, ut, img, pp, pw, pv, op, d, false, m2, r2, dd, ud);
        }
        if (!ok) continue;
        const float u_pose = u_pose_of(cam);
        float u_min, u_max;
        if (cam.roll_u > 0) {
            u_min = ceilf(u_pose / u_per_tile) * u_per_tile + 1e-6f;
            u_max = 1.0f;
        } else {
            u_min = 0.0f;
            u_max = floorf(u_pose / u_per_tile) * u_per_tile - 1e-6f;
        }
        const float mx2 = m2.x / img.x, my2 = m2.y / img.y, rx2 = r2.x / img.x, ry2 = r2.y / img.y;
        Rect r;
        if (LIDAR) r = lidar_rect(mx2, my2, rx2, ry2, u_min, u_max, u_per_tile, n_elev, elev, ntx);
        else r = spherical_rect(mx2, my2, rx2, ry2, u_min, u_max, u_per_tile, n_v, v_per_tile, ntx);
        const uint32_t cb = rect_count(r);
        rects[2 * j + 1] = r;
        vcnt[2 * j + 1] = cb;
        vkey[2 * j + 1] = __float_as_uint(dd);
        if (cb > 0) {
            tpg[j] += (int32_t)cb;
            atomicAdd(&s_vis[b], 1u);
            atomicAdd(&s_cnt[b], cb);
            atomicAdd(&s_rows[b], (uint32_t)(r.y1 - r.y0));
            if (key_range) {  // LDS atomics: the block's second spans join its key range
                atomicMin(&s_klo[b], __float_as_uint(dd));
                atomicMax(&s_khi[b], __float_as_uint(dd));
            }
        }
    }
    __syncthreads();
    if ((int)threadIdx.x < nb && s_vis[threadIdx.x] > 0) {
        const unsigned blk = blk0 + threadIdx.x;
        partials[blk] += ((uint64_t)s_vis[threadIdx.x] << 32) + s_cnt[threadIdx.x];
        cpart[2 * blk] += s_cnt[threadIdx.x];
        cpart[2 * blk + 1] += s_rows[threadIdx.x];
        if (key_range) {
            key_range[2 * blk] = min(key_range[2 * blk], s_klo[threadIdx.x]);
            key_range[2 * blk + 1] = max(key_range[2 * blk + 1], s_khi[threadIdx.x]);
        }
    }
}

// Two-level scans of per-block partials. slice_scan_kernel: workgroup s scans the kSlice partials
// [kSlice s, kSlice (s + 1)) in place (exclusive within the slice) and stores their total in
// slice_sum[s]; with `extra` (the count blocks' exact intersection and row-run sums, two per block)
// it also stores their slice totals. A consumer block b then starts at
// slice_offset(slice_sum, b / kSlice) + partials[b]: the slices before it are few (kSlice = 256 count
// blocks of 1024 instances each), so each consumer sums them itself.
constexpr int kSlice = kBlock;

template <typename T>
__global__ __launch_bounds__(kBlock) void slice_scan_kernel(unsigned n, T* __restrict__ partials,
                                                            T* __restrict__ slice_sum,
                                                            const uint64_t* __restrict__ extra,
                                                            uint64_t* __restrict__ slice_extra,
                                                            const uint32_t* __restrict__ block_range = nullptr,
                                                            uint32_t* __restrict__ slice_range = nullptr) {
    __shared__ T lds[kWaves];
    __shared__ uint64_t lds64[kWaves];
    __shared__ uint32_t s_lo[kWaves], s_hi[kWaves];
    const unsigned i = blockIdx.x * kSlice + threadIdx.x;
    if (block_range) {  // the slice's range of visible depth keys from its blocks' (block-uniform)
        uint32_t lo = i < n ? block_range[2 * i] : 0xffffffffu, hi = i < n ? block_range[2 * i + 1] : 0u;
        block_key_range(lo, hi, s_lo, s_hi);
        if (threadIdx.x == 0) { slice_range[2 * blockIdx.x] = lo; slice_range[2 * blockIdx.x + 1] = hi; }
    }
    const T v = i < n ? partials[i] : T(0);
    T tot;
    const T ex = block_exclusive_scan<T>(v, lds, tot);
    if (i < n) partials[i] = ex;
    if (threadIdx.x == 0) slice_sum[blockIdx.x] = tot;
    if (extra) {
        const uint64_t e0 = block_reduce_sum<uint64_t>(i < n ? extra[2 * i] : 0ull, lds64);
        const uint64_t e1 = block_reduce_sum<uint64_t>(i < n ? extra[2 * i + 1] : 0ull, lds64);
        if (threadIdx.x == 0) {
            slice_extra[2 * blockIdx.x] = e0;
            slice_extra[2 * blockIdx.x + 1] = e1;
        }
    }
}

// sum of slice_sum[0, k), by the whole workgroup (block-uniform result)
template <typename T>
XSG_DEV T slice_offset(const T* __restrict__ slice_sum, unsigned k, T* lds) {
    T acc = 0;
    for (unsigned j = threadIdx.x; j < k; j += kBlock) acc += slice_sum[j];
    return block_reduce_sum<T>(acc, lds);
}

// Compaction of the visible virtual instances in instance order: id, intersection offset, depth bits.
// Block b starts at the packed prefix of the count blocks before it (slice_scan_kernel's two levels).
// Block 0 also sums the slices: the packed total (visible << 32 | count, whose count field may carry)
// and the exact 64-bit intersection and row-run totals go to `publish` (mapped host memory, read by the
// host after an event) and the visible count to m_dev, for the kernels queued ahead of that readback.
__global__ __launch_bounds__(kBlock) void compact_kernel(
    int64_t n_virtual, const uint32_t* __restrict__ vcnt, const uint32_t* __restrict__ vkey,
    const uint64_t* __restrict__ pbase, const uint64_t* __restrict__ slice_sum,
    const uint64_t* __restrict__ slice_extra, unsigned n_slices, uint32_t* __restrict__ comp_id,
    uint32_t* __restrict__ comp_off, uint32_t* __restrict__ comp_key, uint32_t* __restrict__ m_dev,
    uint64_t* __restrict__ publish) {
    __shared__ uint64_t lds[kWaves];
    // each thread its kCountItems consecutive instances: counts and depth bits loaded first (their
    // latency then overlaps the block's offset), one block scan places them all
    const int64_t v0 = (int64_t)blockIdx.x * kCountTile + (int64_t)threadIdx.x * kCountItems;
    uint32_t c[kCountItems], key[kCountItems];
    static_assert(kCountItems == 4, "one 16-byte vector of counts and one of keys per thread");
    const bool vec = v0 + kCountItems <= n_virtual && ((uintptr_t)vcnt & 15) == 0 && ((uintptr_t)vkey & 15) == 0;
    if (vec) {  // the whole item run in range and both arrays 16-byte aligned: one vector load each
        const uint4 cv = *reinterpret_cast<const uint4*>(vcnt + v0);
        const uint4 kv = *reinterpret_cast<const uint4*>(vkey + v0);
        c[0] = cv.x; c[1] = cv.y; c[2] = cv.z; c[3] = cv.w;
        key[0] = kv.x; key[1] = kv.y; key[2] = kv.z; key[3] = kv.w;
    } else {
#pragma unroll
        for (int k = 0; k < kCountItems; ++k) {
            const int64_t v = min(v0 + k, n_virtual - 1);
            const uint32_t cv = vcnt[v];
            key[k] = vkey[v];
            c[k] = v0 + k < n_virtual ? cv : 0u;
        }
    }
    uint64_t carry = slice_offset<uint64_t>(slice_sum, blockIdx.x / kSlice, lds) + pbase[blockIdx.x];
    if (blockIdx.x == 0) {  // block-uniform
        const uint64_t tot = slice_offset<uint64_t>(slice_sum, n_slices, lds);
        uint64_t e0 = 0, e1 = 0;
        for (unsigned j = threadIdx.x; j < n_slices; j += kBlock) {
            e0 += slice_extra[2 * j];
            e1 += slice_extra[2 * j + 1];
        }
        e0 = block_reduce_sum<uint64_t>(e0, lds);
        e1 = block_reduce_sum<uint64_t>(e1, lds);
        if (threadIdx.x == 0) {
            if (m_dev) *m_dev = (uint32_t)(tot >> 32);
            publish[0] = tot;
            publish[1] = e0;
            publish[2] = e1;
        }
    }
    uint64_t sum = 0;
#pragma unroll
    for (int k = 0; k < kCountItems; ++k) sum += pack_count(c[k]);
    uint64_t tot;
    uint64_t s = carry + block_exclusive_scan<uint64_t>(sum, lds, tot);
#pragma unroll
    for (int k = 0; k < kCountItems; ++k) {
        if (c[k] > 0) {
            const uint64_t p = s >> 32;
            if (p < (uint64_t)n_virtual) {
                comp_id[p] = (uint32_t)(v0 + k);
                comp_off[p] = (uint32_t)s;
                comp_key[p] = key[k];
            }
        }
        s += pack_count(c[k]);
    }
}

// Depth pre-order, second stage. A most-significant-digit pass (the top RB bits of each key's offset
// from the smallest visible key, stable) has split the visible instances into buckets of consecutive
// key values, each in instance order. One workgroup per bucket sorts it stably by the key bits below
// that digit, 8 bits per pass: in LDS when it holds at most kBucketCap keys, else chunk by chunk
// through global memory (ping-ponging between the bucket's ranges of the two arrays). The result is
// the stable order of the keys, which is what LSD passes over all 32 bits give.
constexpr int kBucketThreads = 1024;
constexpr int kBucketWaves = kBucketThreads / 64;
constexpr int kBucketCap = 8192;
constexpr int kBucketSteps = kBucketCap / kBucketThreads;  // steps of 64 keys per wavefront, at most

struct BucketLds {
    uint32_t key[2][kBucketCap];
    uint32_t id[2][kBucketCap];
    uint32_t wcnt[kBucketWaves][256];  // per wavefront and digit: count, then the wavefront's prefix
    uint32_t dpre[256];                // per digit: first position in the chunk
    uint32_t dcnt[256];                // per digit: keys of the chunk
    uint32_t gbase[256];               // global path: per digit, next position in the bucket
    uint32_t scan[kBucketWaves];
};

XSG_DEV uint32_t block_exclusive_scan_bucket(uint32_t v, uint32_t* lds, uint32_t& total) {
    const uint32_t inc = wave_inclusive_scan(v);
    const int wave = threadIdx.x >> 6;
    if (__lane_id() == 63) lds[wave] = inc;
    __syncthreads();
    uint32_t before = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kBucketWaves; ++w) {
        const uint32_t x = lds[w];
        if (w < wave) before += x;
        tot += x;
    }
    __syncthreads();
    total = tot;
    return before + inc - v;
}

// Stable ranking of the chunk's n keys in L.key[src][0, n): wavefront w takes the contiguous segment
// [w seg, (w + 1) seg) in steps of 64 keys (seg a multiple of 64, at most kBucketSteps steps), equal
// digits inside a step are found with ballots over the digit bits and a wavefront counter per digit
// carries the rank across steps. pos[r] receives the step's key's position in the digit-sorted chunk,
// L.dpre / L.dcnt each digit's first position and count. Ends with a barrier.
XSG_DEV void bucket_rank(BucketLds& L, int src, int n, int seg, uint32_t kmin, int sh, int bits,
                         uint32_t (&dig)[kBucketSteps], uint32_t (&pos)[kBucketSteps]) {
    const int t = threadIdx.x, wave = t >> 6, lane = __lane_id();
    for (int i = t; i < kBucketWaves * 256; i += kBucketThreads) (&L.wcnt[0][0])[i] = 0u;
    __syncthreads();
    const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const int steps = seg >> 6;
#pragma unroll
    for (int r = 0; r < kBucketSteps; ++r) {
        dig[r] = 0u;
        pos[r] = 0u;
        if (r < steps) {  // uniform
            const int li = wave * seg + r * 64 + lane;
            const bool valid = li < n;
            const uint32_t d = valid ? ((L.key[src][li] - kmin) >> sh) & ((1u << bits) - 1u) : 0u;
            uint64_t peers = __ballot(valid);
            for (int b = 0; b < bits; ++b) {
                const uint64_t m = __ballot((d >> b) & 1u);
                peers &= ((d >> b) & 1u) ? m : ~m;
            }
            const uint32_t before = (uint32_t)__popcll(peers & lt_mask);
            const uint32_t base = valid ? L.wcnt[wave][d] : 0u;
            pos[r] = base + before;
            dig[r] = d;
            if (valid && before == 0) L.wcnt[wave][d] = base + (uint32_t)__popcll(peers);
        }
    }
    __syncthreads();
    uint32_t tot_d = 0;
    if (t < 256) {
#pragma unroll
        for (int w = 0; w < kBucketWaves; ++w) {
            const uint32_t c = L.wcnt[w][t];
            L.wcnt[w][t] = tot_d;
            tot_d += c;
        }
    }
    uint32_t total;
    const uint32_t ex = block_exclusive_scan_bucket(t < 256 ? tot_d : 0u, L.scan, total);
    if (t < 256) { L.dpre[t] = ex; L.dcnt[t] = tot_d; }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kBucketSteps; ++r)
        if (r < steps && wave * seg + r * 64 + lane < n) pos[r] += L.dpre[dig[r]] + L.wcnt[wave][dig[r]];
}

// segment per wavefront for n keys: a multiple of 64, the wavefronts covering n in order
XSG_DEV int bucket_seg(int n) { return min(kBucketCap / kBucketWaves, ((n + kBucketWaves * 64 - 1) / (kBucketWaves * 64)) * 64); }

template <int RB>
__global__ __launch_bounds__(kBucketThreads) void bucket_sort_kernel(
    const uint32_t* __restrict__ digit_total, const uint32_t* __restrict__ range, int range_parts,
    uint32_t* __restrict__ a_key, uint32_t* __restrict__ a_id, uint32_t* __restrict__ out_key,
    uint32_t* __restrict__ out_id) {
    __shared__ BucketLds L;
    const int t = threadIdx.x;
    const int b = blockIdx.x;
    // the bucket's first position: the counts of the buckets before it
    uint32_t acc = 0;
    for (int j = t; j < b; j += kBucketThreads) acc += digit_total[j];
    uint32_t start;
    block_exclusive_scan_bucket(acc, L.scan, start);
    const int n = (int)digit_total[b];
    if (n == 0) return;  // uniform
    const KeyRange kr = key_range(range, range_parts, RB);
    const int low = kr.shift;  // the key bits below the bucket digit
    if (low == 0 || n == 1) {  // equal keys (or one): already in order
        for (int i = t; i < n; i += kBucketThreads) { out_key[start + i] = a_key[start + i]; out_id[start + i] = a_id[start + i]; }
        return;
    }
    uint32_t dig[kBucketSteps], pos[kBucketSteps];
    if (n <= kBucketCap) {
        for (int i = t; i < n; i += kBucketThreads) { L.key[0][i] = a_key[start + i]; L.id[0][i] = a_id[start + i]; }
        __syncthreads();
        const int seg = bucket_seg(n);
        const int wave = t >> 6, lane = __lane_id();
        int cur = 0;
        for (int sh = 0; sh < low; sh += 8) {
            bucket_rank(L, cur, n, seg, kr.kmin, sh, min(8, low - sh), dig, pos);
#pragma unroll
            for (int r = 0; r < kBucketSteps; ++r) {
                const int li = wave * seg + r * 64 + lane;
                if (r < (seg >> 6) && li < n) {
                    L.key[cur ^ 1][pos[r]] = L.key[cur][li];
                    L.id[cur ^ 1][pos[r]] = L.id[cur][li];
                }
            }
            __syncthreads();
            cur ^= 1;
        }
        for (int i = t; i < n; i += kBucketThreads) { out_key[start + i] = L.key[cur][i]; out_id[start + i] = L.id[cur][i]; }
        return;
    }
    // larger than LDS: each pass counts the bucket's digits, then ranks it chunk by chunk in order and
    // writes every key to its place; the passes alternate between the bucket's ranges of the two arrays
    uint32_t* src_k = a_key; uint32_t* src_i = a_id;
    uint32_t* dst_k = out_key; uint32_t* dst_i = out_id;
    for (int sh = 0; sh < low; sh += 8) {
        const int bits = min(8, low - sh);
        if (t < 256) L.gbase[t] = 0u;
        __syncthreads();
        for (int i = t; i < n; i += kBucketThreads)
            atomicAdd(&L.gbase[((src_k[start + i] - kr.kmin) >> sh) & ((1u << bits) - 1u)], 1u);
        __syncthreads();
        uint32_t total;
        const uint32_t g = t < 256 ? L.gbase[t] : 0u;
        const uint32_t ex = block_exclusive_scan_bucket(g, L.scan, total);
        if (t < 256) L.gbase[t] = ex;
        __syncthreads();
        for (int c0 = 0; c0 < n; c0 += kBucketCap) {
            const int nc = min(kBucketCap, n - c0);
            for (int i = t; i < nc; i += kBucketThreads) { L.key[0][i] = src_k[start + c0 + i]; L.id[0][i] = src_i[start + c0 + i]; }
            __syncthreads();
            const int seg = bucket_seg(nc);
            bucket_rank(L, 0, nc, seg, kr.kmin, sh, bits, dig, pos);
            const int wave = t >> 6, lane = __lane_id();
#pragma unroll
            for (int r = 0; r < kBucketSteps; ++r) {
                const int li = wave * seg + r * 64 + lane;
                if (r < (seg >> 6) && li < nc) {
                    const uint32_t d = dig[r];
                    const uint32_t gp = L.gbase[d] + (pos[r] - L.dpre[d]);
                    dst_k[start + gp] = L.key[0][li];
                    dst_i[start + gp] = L.id[0][li];
                }
            }
            __syncthreads();
            if (t < 256) L.gbase[t] += L.dcnt[t];
            __syncthreads();
        }
        uint32_t* tk = src_k; src_k = dst_k; dst_k = tk;
        uint32_t* ti = src_i; src_i = dst_i; dst_i = ti;
    }
    if (src_k != out_key) {  // an even number of passes ends in the input arrays
        for (int i = t; i < n; i += kBucketThreads) { out_key[start + i] = src_k[start + i]; out_id[start + i] = src_i[start + i]; }
    }
}

// 64-bit key exactly as tiling_common.cuh:37,68 builds it: (tile << 32) | sign-extended depth bits
XSG_DEV int64_t make_key(uint32_t tile_hi, uint32_t depth_bits) {
    return (int64_t)(((uint64_t)tile_hi) << 32) | (int64_t)(int32_t)depth_bits;
}

struct FinalOut {  // unsorted output in the reference's fill order
    int64_t* keys;
    int32_t* ids;
    XSG_DEV void put(int64_t o, uint32_t tile_hi, uint32_t v, uint32_t dbits, int spans) const {
        keys[o] = make_key(tile_hi, dbits);
        ids[o] = (int32_t)(v / (uint32_t)spans);
    }
};

// Merge-path expansion: block b produces outputs [b * E, (b + 1) * E); the visible virtual
// instances overlapping that range (at most E, every count >= 1) are staged in LDS, each
// thread binary-searches its output's instance and decodes the tile from the rectangle.
template <typename Out>
__global__ __launch_bounds__(kBlock) void expand_kernel(
    int64_t n_out, const uint32_t* __restrict__ offs, const uint32_t* __restrict__ ids,
    const uint32_t* __restrict__ keys, int64_t m, const Rect* __restrict__ rects, int ntx, int tnb,
    int64_t n_per_cam, int spans, Out out) {
    __shared__ uint32_t s_off[kExpandPerBlock];
    __shared__ uint32_t s_id[kExpandPerBlock];
    __shared__ uint32_t s_dep[kExpandPerBlock];
    __shared__ Rect s_r[kExpandPerBlock];
    __shared__ int64_t s_range[2];
    const int64_t o0 = (int64_t)blockIdx.x * kExpandPerBlock;
    const int64_t o_end = min(n_out, o0 + kExpandPerBlock);
    if (threadIdx.x < 2) {
        const int64_t x = threadIdx.x == 0 ? o0 : o_end - 1;
        int64_t lo = 0, hi = m - 1;
        while (lo < hi) {
            const int64_t mid = (lo + hi + 1) >> 1;
            if ((int64_t)offs[mid] <= x) lo = mid; else hi = mid - 1;
        }
        s_range[threadIdx.x] = lo;
    }
    __syncthreads();
    const int64_t p_lo = s_range[0];
    const int cnt = (int)min<int64_t>(s_range[1] - p_lo + 1, kExpandPerBlock);
    for (int e = threadIdx.x; e < cnt; e += kBlock) {
        const int64_t p = p_lo + e;
        const uint32_t v = ids[p];
        s_off[e] = offs[p];
        s_id[e] = v;
        s_dep[e] = keys[p];
        s_r[e] = rects[v];
    }
    __syncthreads();
    for (int q = threadIdx.x; q < kExpandPerBlock; q += kBlock) {
        const int64_t o = o0 + q;
        if (o >= o_end) break;
        int lo = 0, hi = cnt - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if ((int64_t)s_off[mid] <= o) lo = mid; else hi = mid - 1;
        }
        const uint32_t l = (uint32_t)(o - (int64_t)s_off[lo]);
        const uint32_t v = s_id[lo];
        const Rect r = s_r[lo];
        const uint32_t wx = (uint32_t)(r.x1 - r.x0);
        const uint32_t yy = l / wx;
        const uint32_t tile = (r.y0 + yy) * (uint32_t)ntx + (r.x0 + (l - yy * wx));
        const uint32_t inst = v / (uint32_t)spans;
        const uint32_t cid = n_per_cam > 0 ? (uint32_t)(inst / (uint64_t)n_per_cam) : 0u;
        out.put(o, (cid << tnb) | tile, v, s_dep[lo], spans);
    }
}

// ---------------------------------------------------------------- sorted fill by tile rows
// The sorted fill without sorting the intersections themselves. The visible instances are in
// depth order (stable). Each instance's rectangle is cut into row runs, one per tile row it
// covers; the runs (about a ninth of the intersections) are sorted stably by row bucket
// (camera * n_tiles_y + row), so every row's runs are in depth order. A row's runs are then split
// into segments of kRunSeg; per segment, a difference array over the columns gives how many of
// its runs cover each column, and one exclusive scan over (row, column, segment) gives every
// segment the first output position of each of its columns. Finally a wavefront per (segment,
// group of 8 columns) walks the segment's runs in order and, per column, ballots the runs that
// cover it: they take consecutive positions, in depth order, so the stores of a column are
// contiguous. The order is (camera, tile, depth bits, Gaussian order): the reference's stable
// sort of its 64-bit keys. Entries of instances with a negative depth belong after every tile
// (their sign-extended keys saturate the tile bits); they form the last row bucket and are written
// in run order, which is depth order, then rows, then columns, as the reference orders them.
constexpr int kRunSeg = 512;          // runs per row segment
constexpr int kMaxSortedCols = 8192;  // tile columns (LDS difference array of seg_count_kernel)
constexpr int kColGroup = 4;    // columns per wavefront step in write_runs_kernel
constexpr int kBandCols = 8;    // columns whose runs write_runs_kernel lists together (a multiple of kColGroup)

// A rectangle as two words (x0 | y0 << 16, x1 | y1 << 16), for the depth-ordered copy that
// rows_reduce_kernel gathers once and the later passes read in order.
XSG_DEV Rect rect_of(uint32_t lo, uint32_t hi) {
    return Rect{(uint16_t)(lo & 0xffffu), (uint16_t)(lo >> 16), (uint16_t)(hi & 0xffffu), (uint16_t)(hi >> 16)};
}

// rows covered by each depth-ordered visible instance -> exclusive run offsets (reduce / scan).
// rows_reduce_kernel gathers each instance's rectangle (a random read per instance) and stores it in
// depth order (d_lo, d_hi), so that rows_scan_kernel and expand_runs_kernel read it sequentially.
__global__ __launch_bounds__(kBlock) void rows_reduce_kernel(int64_t m, const uint32_t* __restrict__ m_dev,
                                                             const uint32_t* __restrict__ ids,
                                                             const Rect* __restrict__ rects,
                                                             uint32_t* __restrict__ partials,
                                                             uint32_t* __restrict__ d_lo,
                                                             uint32_t* __restrict__ d_hi) {
    __shared__ uint32_t lds[kWaves];
    m = min(m, (int64_t)*m_dev);
    uint32_t acc = 0;
    const int64_t base = (int64_t)blockIdx.x * kCountTile;
    for (int k = 0; k < kCountItems; ++k) {
        const int64_t p = base + (int64_t)k * kBlock + threadIdx.x;
        if (p < m) {
            const Rect r = rects[ids[p]];
            d_lo[p] = (uint32_t)r.x0 | ((uint32_t)r.y0 << 16);
            d_hi[p] = (uint32_t)r.x1 | ((uint32_t)r.y1 << 16);
            acc += (uint32_t)(r.y1 - r.y0);
        }
    }
    acc = block_reduce_sum<uint32_t>(acc, lds);
    if (threadIdx.x == 0) partials[blockIdx.x] = acc;
}

__global__ __launch_bounds__(kBlock) void rows_scan_kernel(int64_t m, const uint32_t* __restrict__ m_dev,
                                                           const uint32_t* __restrict__ d_lo,
                                                           const uint32_t* __restrict__ d_hi,
                                                           const uint32_t* __restrict__ partials,
                                                           const uint32_t* __restrict__ slice_sum,
                                                           uint32_t* __restrict__ roff) {
    __shared__ uint32_t lds[kWaves];
    m = min(m, (int64_t)*m_dev);
    const int64_t base = (int64_t)blockIdx.x * kCountTile;
    if (base >= m) return;  // block-uniform
    // the block's first offset: the slices before it, then its place in its slice (slice_scan_kernel)
    uint32_t carry = slice_offset<uint32_t>(slice_sum, blockIdx.x / kSlice, lds) + partials[blockIdx.x];
    for (int k = 0; k < kCountItems; ++k) {
        if (base + (int64_t)k * kBlock >= m) break;
        const int64_t p = base + (int64_t)k * kBlock + threadIdx.x;
        uint32_t h = 0;
        if (p < m) h = (d_hi[p] >> 16) - (d_lo[p] >> 16);
        uint32_t tot;
        const uint32_t ex = block_exclusive_scan<uint32_t>(h, lds, tot);
        if (p < m) roff[p] = carry + ex;
        carry += tot;
    }
}

// Every expansion block's first and last instance (the instances holding its first and last run): each
// instance marks the blocks whose first or last run it holds. Every visible instance has at least one
// run, so a block of kExpandPerBlock runs spans at most that many instances.
__global__ __launch_bounds__(kBlock) void run_block_bounds_kernel(int64_t m, const uint32_t* __restrict__ roff,
                                                                  int64_t n_runs, uint32_t* __restrict__ first,
                                                                  uint32_t* __restrict__ last) {
    const int64_t p = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (p >= m) return;
    const int64_t o0 = roff[p], o1 = p + 1 < m ? (int64_t)roff[p + 1] : n_runs;  // the instance's runs [o0, o1)
    for (int64_t b = o0 / kExpandPerBlock; b * kExpandPerBlock < o1; ++b) {
        if (b * kExpandPerBlock >= o0) first[b] = (uint32_t)p;
        const int64_t end = min(n_runs, (b + 1) * kExpandPerBlock) - 1;
        if (end < o1) last[b] = (uint32_t)p;
    }
}

// Merge-path expansion of the depth-ordered instances into row runs: run r gets its row bucket
// and its record for the writers (flatten id, depth bits, column range x0 | x1 << 16, row bucket),
// which the row sort then carries. A block writes one tile of the run sort (kExpandPerBlock runs),
// so it also stores the tile's histogram of the sort's first digit (the low RB bits of the row
// bucket) into hist, digit-major as radix_upsweep would.
static_assert(kExpandPerBlock == kSortBlock * kRunSortItems, "an expansion block is one tile of the run sort");
template <int RB>
__global__ __launch_bounds__(kBlock) void expand_runs_kernel(int64_t n_runs, const uint32_t* __restrict__ roff,
                                                             const uint32_t* __restrict__ ids,
                                                             const uint32_t* __restrict__ keys, int64_t m,
                                                             const uint32_t* __restrict__ d_lo,
                                                             const uint32_t* __restrict__ d_hi, int nty,
                                                             int64_t n_per_cam, int spans, uint32_t neg_row,
                                                             uint32_t* __restrict__ out_row,
                                                             uint4* __restrict__ out_rec,
                                                             uint32_t* __restrict__ hist, unsigned nb,
                                                             const uint32_t* __restrict__ first,
                                                             const uint32_t* __restrict__ last) {
    __shared__ uint32_t s_off[kExpandPerBlock];
    __shared__ uint32_t s_row[kExpandPerBlock];  // first row bucket of the instance, or neg_row
    __shared__ uint32_t s_fid[kExpandPerBlock];
    __shared__ uint32_t s_key[kExpandPerBlock];
    __shared__ uint32_t s_cols[kExpandPerBlock];
    __shared__ int32_t s_inst[kExpandPerBlock];  // per run slot: the staged instance holding it
    __shared__ int32_t s_wmax[kWaves];
    constexpr int R = 1 << RB;
    __shared__ uint32_t s_hist[R];
    for (int d = threadIdx.x; d < R; d += kBlock) s_hist[d] = 0;
    for (int q = threadIdx.x; q < kExpandPerBlock; q += kBlock) s_inst[q] = 0;
    // each XCD takes a contiguous range of blocks, so that the histogram words of neighbouring blocks
    // (consecutive words of each digit's row) meet in one L2
    const unsigned blk = (unsigned)xcd_tile((int)blockIdx.x, (int)gridDim.x);
    const int64_t o0 = (int64_t)blk * kExpandPerBlock;
    const int64_t o_end = min(n_runs, o0 + kExpandPerBlock);
    // the instances holding the block's first and last run (run_block_bounds_kernel)
    const int64_t p_lo = first[blk];
    const int cnt = (int)min<int64_t>((int64_t)last[blk] - p_lo + 1, kExpandPerBlock);
    for (int e = threadIdx.x; e < cnt; e += kBlock) {
        const int64_t p = p_lo + e;
        const uint32_t v = ids[p];
        const uint32_t inst = v / (uint32_t)spans;
        const uint32_t cid = n_per_cam > 0 ? (uint32_t)(inst / (uint64_t)n_per_cam) : 0u;
        const uint32_t key = keys[p];
        const Rect r = rect_of(d_lo[p], d_hi[p]);
        s_off[e] = roff[p];
        s_row[e] = ((int32_t)key < 0) ? neg_row : cid * (uint32_t)nty + r.y0;
        s_fid[e] = inst;
        s_key[e] = key;
        s_cols[e] = (uint32_t)r.x0 | ((uint32_t)r.x1 << 16);
    }
    __syncthreads();
    // every staged instance after the first marks the slot of its first run; a running maximum over
    // the slots then gives each run its instance (the staged instances start in increasing order)
    for (int e = threadIdx.x + 1; e < cnt; e += kBlock) s_inst[s_off[e] - o0] = e;
    __syncthreads();
    {
        constexpr int kPer = kExpandPerBlock / kBlock;  // consecutive slots per thread
        const int q0 = threadIdx.x * kPer;
        int32_t v[kPer];
        int32_t run = 0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            run = max(run, s_inst[q0 + j]);
            v[j] = run;
        }
        // maximum over the threads before this one
        int32_t inc = run;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int32_t t = __shfl_up(inc, off, 64);
            if (__lane_id() >= off) inc = max(inc, t);
        }
        const int wave = threadIdx.x >> 6;
        if (__lane_id() == 63) s_wmax[wave] = inc;
        __syncthreads();
        int32_t before = __shfl_up(inc, 1, 64);
        if (__lane_id() == 0) before = 0;
        for (int w = 0; w < wave; ++w) before = max(before, s_wmax[w]);
#pragma unroll
        for (int j = 0; j < kPer; ++j) s_inst[q0 + j] = max(before, v[j]);
    }
    __syncthreads();
    for (int q = threadIdx.x; q < kExpandPerBlock; q += kBlock) {
        const int64_t o = o0 + q;
        if (o >= o_end) break;
        const int lo = s_inst[q];
        const uint32_t row0 = s_row[lo];
        const uint32_t row = row0 == neg_row ? neg_row : row0 + (uint32_t)(o - (int64_t)s_off[lo]);
        out_row[o] = row;
        out_rec[o] = make_uint4(s_fid[lo], s_key[lo], s_cols[lo], row);
        atomicAdd(&s_hist[row & (R - 1)], 1u);
    }
    __syncthreads();
    for (int d = threadIdx.x; d < R; d += kBlock) hist[(int64_t)d * nb + blk] = s_hist[d];
}

// Scan of the per-group counts of every bucket over its first ceil(m / 64) groups, in slices of
// `slice` groups, grid (buckets, slices): group_slice_sum_kernel sums each slice, then
// group_slice_scan_kernel scans each slice in place (exclusive) from the sum of the bucket's slices
// before it, and slice 0 stores the bucket total. Up to kGroupOneSlice groups (the host's bound) are
// one slice, whose sums are not needed: part is null and slice 0's own total is the bucket's. More
// groups take slices of one chunk each, so that the grid has several workgroups per bucket (a lidar
// frame's 17 buckets and 31 k groups: 272 instead of 34).
constexpr int kGroupItems = 8;                           // consecutive groups per thread and chunk
constexpr int kGroupChunk = kBlock * kGroupItems;        // groups per block scan
constexpr int kGroupOneSlice = kGroupChunk * 8;
inline int64_t group_slice(int64_t n_groups) { return n_groups <= kGroupOneSlice ? kGroupOneSlice : kGroupChunk; }

__global__ __launch_bounds__(kBlock) void group_slice_sum_kernel(const uint32_t* __restrict__ hist, int64_t n_groups,
                                                                 int64_t slice, const uint32_t* __restrict__ m_dev,
                                                                 uint32_t* __restrict__ part) {
    __shared__ uint32_t lds[kWaves];
    const int64_t ng = min(n_groups, ((int64_t)*m_dev + 63) / 64);
    const int64_t s0 = (int64_t)blockIdx.y * slice;
    if (s0 >= ng) return;  // block-uniform
    const uint32_t* h = hist + (int64_t)blockIdx.x * n_groups;
    uint32_t sum = 0;
    for (int64_t i = s0 + threadIdx.x; i < min(ng, s0 + slice); i += kBlock) sum += h[i];
    sum = block_reduce_sum<uint32_t>(sum, lds);
    if (threadIdx.x == 0) part[(int64_t)blockIdx.x * gridDim.y + blockIdx.y] = sum;
}

__global__ __launch_bounds__(kBlock) void group_slice_scan_kernel(uint32_t* __restrict__ hist, int64_t n_groups,
                                                                  int64_t slice, const uint32_t* __restrict__ m_dev,
                                                                  const uint32_t* __restrict__ part,
                                                                  uint32_t* __restrict__ total) {
    __shared__ uint32_t lds[kWaves];
    const int64_t ng = min(n_groups, ((int64_t)*m_dev + 63) / 64);
    const unsigned n_slices = (unsigned)((ng + slice - 1) / slice);
    const unsigned k = blockIdx.y;
    const uint32_t* pr = part ? part + (int64_t)blockIdx.x * gridDim.y : nullptr;
    if (k == 0 && pr) {  // block-uniform
        uint32_t acc = 0;
        for (unsigned j = threadIdx.x; j < n_slices; j += kBlock) acc += pr[j];
        acc = block_reduce_sum<uint32_t>(acc, lds);
        if (threadIdx.x == 0) total[blockIdx.x] = acc;
    }
    if (k >= max(n_slices, 1u)) return;  // block-uniform
    uint32_t run = 0;
    if (pr) {
        uint32_t acc = 0;
        for (unsigned j = threadIdx.x; j < k; j += kBlock) acc += pr[j];
        run = block_reduce_sum<uint32_t>(acc, lds);
    }
    uint32_t* h = hist + (int64_t)blockIdx.x * n_groups;
    const int n_chunks = (int)(slice / kGroupChunk);
    for (int c = 0; c < n_chunks; ++c) {
        const int64_t c0 = (int64_t)k * slice + (int64_t)c * kGroupChunk;
        if (c0 >= ng) break;  // block-uniform
        const int64_t i0 = c0 + (int64_t)threadIdx.x * kGroupItems;
        uint32_t v[kGroupItems], sum = 0;
#pragma unroll
        for (int j = 0; j < kGroupItems; ++j) {
            v[j] = i0 + j < ng ? h[i0 + j] : 0u;
            sum += v[j];
        }
        uint32_t tot;
        uint32_t at = run + block_exclusive_scan<uint32_t>(sum, lds, tot);
#pragma unroll
        for (int j = 0; j < kGroupItems; ++j) {
            if (i0 + j < ng) h[i0 + j] = at;
            at += v[j];
        }
        run += tot;
    }
    if (!pr && threadIdx.x == 0) total[blockIdx.x] = run;  // the only slice
}

// Direct placement of the row runs, for at most kDirectRows row buckets (camera rows plus the
// negative-depth bucket): instead of expanding the runs in depth order and sorting them stably by row
// bucket, every group of 64 depth-ordered instances (one wavefront step) counts its runs per row
// bucket (rows_hist_kernel, which also gathers the rectangles in depth order), one scan per bucket
// over the groups gives each (bucket, group) its first position (radix_scan_hist), and
// place_runs_kernel, one wavefront per group, writes each run straight to its place, bucket by bucket
// in lane order. Every bucket thus holds its runs in depth order: the order the stable sort gave.
constexpr int kDirectRows = 256;
constexpr int kGroupsPerCountBlock = kCountTile / 64;

XSG_DEV void run_rows(uint32_t key, Rect r, uint32_t v, int spans, int64_t n_per_cam, int nty, uint32_t& lo,
                      uint32_t& hi, uint32_t& n_neg) {
    // non-negative keys: buckets [lo, hi), one run each; a negative key: n_neg runs in the last bucket
    if ((int32_t)key < 0) {
        lo = hi = 0u;
        n_neg = (uint32_t)(r.y1 - r.y0);
        return;
    }
    const uint32_t inst = v / (uint32_t)spans;
    const uint32_t cid = n_per_cam > 0 ? (uint32_t)(inst / (uint64_t)n_per_cam) : 0u;
    lo = cid * (uint32_t)nty + r.y0;
    hi = cid * (uint32_t)nty + r.y1;
    n_neg = 0u;
}

// Per group of 64 depth-ordered instances (one wavefront, four per workgroup): their rectangles to
// d_lo / d_hi, and the group's runs per bucket, hist[bucket * n_groups + group]. The group's counts
// are kept in a wavefront-private LDS row (the LDS instructions of one wavefront complete in order).
__global__ __launch_bounds__(kBlock) void rows_hist_kernel(int64_t m, const uint32_t* __restrict__ m_dev,
                                                           const uint32_t* __restrict__ ids,
                                                           const uint32_t* __restrict__ keys,
                                                           const Rect* __restrict__ rects, int nty, int64_t n_per_cam,
                                                           int spans, int n_rows, int64_t n_groups,
                                                           uint32_t* __restrict__ hist, uint32_t* __restrict__ d_lo,
                                                           uint32_t* __restrict__ d_hi) {
    __shared__ uint32_t s_h[kWaves][kDirectRows];
    m = min(m, (int64_t)*m_dev);
    const int wave = threadIdx.x >> 6, lane = __lane_id();
    const int64_t grp = (int64_t)blockIdx.x * kWaves + wave;
    if (grp * 64 >= m) return;  // wave-uniform; the scan reads the active groups only
    const int64_t p = grp * 64 + lane;
    uint32_t v = 0u, key = 0u;
    if (p < m) { v = ids[p]; key = keys[p]; }
    uint32_t* h = s_h[wave];
    for (int i = lane; i < n_rows; i += 64) h[i] = 0u;
    wave_lds_sync();
    if (p < m) {
        const Rect r = rects[v];
        d_lo[p] = (uint32_t)r.x0 | ((uint32_t)r.y0 << 16);
        d_hi[p] = (uint32_t)r.x1 | ((uint32_t)r.y1 << 16);
        uint32_t lo, hi, n_neg;
        run_rows(key, r, v, spans, n_per_cam, nty, lo, hi, n_neg);
        if (n_neg) atomicAdd(&h[n_rows - 1], n_neg);
        for (uint32_t b = lo; b < hi; ++b) atomicAdd(&h[b], 1u);
    }
    wave_lds_sync();
    for (int i = lane; i < n_rows; i += 64) hist[(int64_t)i * n_groups + grp] = h[i];
}

XSG_DEV uint32_t wave_min_u32(uint32_t x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x = min(x, (uint32_t)__shfl_xor((int)x, off, 64));
    return x;
}
XSG_DEV uint32_t wave_max_u32(uint32_t x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x = max(x, (uint32_t)__shfl_xor((int)x, off, 64));
    return x;
}

// One wavefront per group of 64 instances: each bucket's first position for the group (the bucket's
// base, an exclusive scan of the bucket totals, plus the group's scanned count), then the runs,
// bucket by bucket, at consecutive positions in lane order. Lane l holds the positions of buckets
// l + 64 j in registers, and the loop over a bucket reads its position from that lane (a scalar
// read; no LDS round trip per bucket).
__global__ __launch_bounds__(64) void place_runs_kernel(int64_t m, const uint32_t* __restrict__ ids,
                                                        const uint32_t* __restrict__ keys,
                                                        const uint32_t* __restrict__ d_lo,
                                                        const uint32_t* __restrict__ d_hi, int nty, int64_t n_per_cam,
                                                        int spans, int n_rows, int64_t n_groups,
                                                        const uint32_t* __restrict__ hist,
                                                        const uint32_t* __restrict__ row_tot,
                                                        uint4* __restrict__ out_rec) {
    constexpr int kPer = kDirectRows / 64;
    const int lane = __lane_id();
    const int64_t grp = blockIdx.x;
    const int64_t p = grp * 64 + lane;
    uint32_t v = 0u, key = 0u, lo_w = 0u, hi_w = 0u;
    if (p < m) { v = ids[p]; key = keys[p]; lo_w = d_lo[p]; hi_w = d_hi[p]; }
    uint32_t c[kPer], at[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int b = lane + 64 * j;
        c[j] = b < n_rows ? row_tot[b] : 0u;
        at[j] = b < n_rows ? hist[(int64_t)b * n_groups + grp] : 0u;
    }
    // bucket b = lane + 64 j starts after every bucket of the lower j and the lanes below it in this j
    uint32_t before = 0u;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const uint32_t inc = wave_inclusive_scan<uint32_t>(c[j]);
        at[j] += before + inc - c[j];
        before += (uint32_t)__shfl((int)inc, 63, 64);
    }
    uint32_t lo = 0u, hi = 0u, n_neg = 0u;
    uint4 rec = make_uint4(0u, 0u, 0u, 0u);
    if (p < m) {
        const Rect r = rect_of(lo_w, hi_w);
        run_rows(key, r, v, spans, n_per_cam, nty, lo, hi, n_neg);
        rec = make_uint4(v / (uint32_t)spans, key, (uint32_t)r.x0 | ((uint32_t)r.x1 << 16), 0u);
    }
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    // the wave's bucket range, in scalar registers (a uniform loop)
    const uint32_t b0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)wave_min_u32(lo < hi ? lo : 0xffffffffu));
    const uint32_t b1 = (uint32_t)__builtin_amdgcn_readfirstlane((int)wave_max_u32(hi));
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const uint32_t jb0 = max(b0, (uint32_t)(64 * j)), jb1 = min(b1, (uint32_t)(64 * j + 64));
        for (uint32_t b = jb0; b < jb1; ++b) {  // wave-uniform
            const bool cov = lo <= b && b < hi;
            const uint64_t mk = __ballot(cov);
            const uint32_t base = (uint32_t)__builtin_amdgcn_readlane((int)at[j], (int)(b - 64 * j));
            if (cov) {
                rec.w = b;
                out_rec[base + (uint32_t)__popcll(mk & lt)] = rec;
            }
        }
    }
    if (__ballot(n_neg > 0)) {  // negative keys: n_neg identical runs each, in lane order
        const int neg = n_rows - 1;
        uint32_t nb = 0u;
#pragma unroll
        for (int j = 0; j < kPer; ++j)
            if (neg >> 6 == j) nb = (uint32_t)__builtin_amdgcn_readlane((int)at[j], neg & 63);
        const uint32_t at_neg = nb + wave_inclusive_scan<uint32_t>(n_neg) - n_neg;
        rec.w = (uint32_t)neg;
        for (uint32_t q = 0; q < n_neg; ++q) out_rec[at_neg + q] = rec;
    }
}

// row_start[r] = first sorted run of row bucket r (r in [0, n_rows]) from the sorted row buckets, one
// thread per boundary between runs i - 1 and i: it starts the rows (rows[i - 1], rows[i]] (from row 0
// before the first run, to n_rows after the last), so every row is written once.
__global__ __launch_bounds__(kBlock) void row_start_kernel(const uint32_t* __restrict__ rows, int64_t n_runs,
                                                           int n_rows, uint32_t* __restrict__ row_start) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i > n_runs) return;
    const int lo = i == 0 ? 0 : (int)rows[i - 1] + 1;
    const int hi = i == n_runs ? n_rows : min((int)rows[i], n_rows);
    for (int r = lo; r <= hi; ++r) row_start[r] = (uint32_t)i;
}

// single block: segments of kRunSeg runs per real row: seg_base = exclusive prefix of the segment
// counts (total at seg_base[n_real]) and seg_row[s] = row of segment s. When the row sort was a
// single pass, `row_count` holds its digit totals -- the runs per row bucket -- and row_start is
// their exclusive scan, written here; otherwise row_start_kernel has written row_start.
__global__ __launch_bounds__(kBlock) void row_segments_kernel(int n_rows, const uint32_t* __restrict__ row_count,
                                                              uint32_t* __restrict__ row_start,
                                                              uint32_t* __restrict__ seg_base,
                                                              uint32_t* __restrict__ seg_row) {
    __shared__ uint32_t lds[kWaves];
    if (row_count) {  // the single pass's digit totals: n_rows <= 1 << RB (at most 1024)
        const int per = (n_rows + kBlock - 1) / kBlock;  // consecutive rows per thread
        const int q0 = threadIdx.x * per, q1 = min(n_rows, q0 + per);
        uint32_t c = 0;
        for (int r = q0; r < q1; ++r) c += row_count[r];
        uint32_t tot;
        uint32_t run = block_exclusive_scan<uint32_t>(c, lds, tot);
        for (int r = q0; r < q1; ++r) {
            row_start[r] = run;
            run += row_count[r];
        }
        if (threadIdx.x == 0) row_start[n_rows] = tot;
    }
    __syncthreads();
    const int n_real = n_rows - 1;
    const int per = (n_real + kBlock - 1) / kBlock;
    const int r0 = threadIdx.x * per, r1 = min(n_real, r0 + per);
    uint32_t sum = 0;
    for (int r = r0; r < r1; ++r) sum += (row_start[r + 1] - row_start[r] + kRunSeg - 1) / kRunSeg;
    uint32_t tot;
    uint32_t run = block_exclusive_scan<uint32_t>(sum, lds, tot);
    // the bases also go to LDS when they fit, for the searches below
    __shared__ uint32_t s_base[kMaxLdsRows];
    const bool in_lds = n_real <= kMaxLdsRows;  // block-uniform
    for (int r = r0; r < r1; ++r) {
        seg_base[r] = run;
        if (in_lds) s_base[r] = run;
        run += (row_start[r + 1] - row_start[r] + kRunSeg - 1) / kRunSeg;
    }
    if (threadIdx.x == 0) seg_base[n_real] = tot;
    // every thread a contiguous share of the segments: the row of its first one is the last r with
    // seg_base[r] <= segment (rows without segments share a base with the next row, and the search
    // takes the later one); the following ones advance the row as they pass its segments
    __syncthreads();  // s_base, and the global seg_base of this block, are complete
    const uint32_t* base = in_lds ? s_base : seg_base;
    const uint32_t share = (tot + kBlock - 1) / kBlock;
    const uint32_t s0 = threadIdx.x * share, s1 = min(tot, s0 + share);
    if (s0 < s1) {
        int lo = 0, hi = n_real - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (base[mid] <= s0) lo = mid; else hi = mid - 1;
        }
        for (uint32_t sg = s0; sg < s1; ++sg) {
            while (lo + 1 < n_real && base[lo + 1] <= sg) ++lo;
            seg_row[sg] = (uint32_t)lo;
        }
    }
}

// One workgroup per segment: how many of its runs cover each column, from a difference array in
// LDS (+1 at x0, -1 at x1, then a prefix over the columns), stored at slot (row, column, segment).
__global__ __launch_bounds__(kBlock) void seg_count_kernel(int n_real, const uint4* __restrict__ rec,
                                                           const uint32_t* __restrict__ row_start,
                                                           const uint32_t* __restrict__ seg_base,
                                                           const uint32_t* __restrict__ seg_row, int ntx,
                                                           uint32_t* __restrict__ slots) {
    extern __shared__ int32_t s_diff[];  // ntx + 1
    __shared__ int32_t lds[kWaves];
    const int64_t sg = blockIdx.x;
    if (sg >= (int64_t)seg_base[n_real]) return;
    const uint32_t row = seg_row[sg];
    const uint32_t sb = seg_base[row], nseg = seg_base[row + 1] - sb;
    const uint32_t k = (uint32_t)sg - sb;
    const int64_t b = (int64_t)row_start[row] + (int64_t)k * kRunSeg;
    const int64_t e = min((int64_t)row_start[row + 1], b + kRunSeg);
    for (int c = threadIdx.x; c <= ntx; c += kBlock) s_diff[c] = 0;
    __syncthreads();
    for (int64_t i = b + threadIdx.x; i < e; i += kBlock) {
        const uint32_t x01 = rec[i].z;
        atomicAdd(&s_diff[x01 & 0xffffu], 1);
        atomicAdd(&s_diff[x01 >> 16], -1);
    }
    __syncthreads();
    // each thread a run of consecutive columns; block scan of the runs' sums
    const int per = (ntx + kBlock - 1) / kBlock;
    const int c0 = threadIdx.x * per, c1 = min(ntx, c0 + per);
    int32_t sum = 0;
    for (int c = c0; c < c1; ++c) sum += s_diff[c];
    int32_t tot;
    int32_t run = block_exclusive_scan<int32_t>(sum, lds, tot);
    uint32_t* out = slots + (int64_t)sb * ntx + k;
    for (int c = c0; c < c1; ++c) {
        run += s_diff[c];
        out[(int64_t)c * nseg] = (uint32_t)run;
    }
}

// seg_count_kernel with row_segments_kernel's work done by every workgroup, for up to kFusedRows row
// buckets: each derives the row starts (from the run sort's digit totals when given, else from
// row_start) and the segment bases, and each of its wavefronts then counts one segment (workgroup w,
// wavefront v: segment kWaves w + v) as seg_count_kernel does, in a wavefront-private LDS difference
// array (the LDS instructions of one wavefront complete in order, so no barrier follows the set-up);
// workgroup 0 stores the row starts and bases and each wavefront its segment's row, for the kernels
// after it. One launch fewer per fill, and the set-up shared by four segments.
constexpr int kFusedRows = 1024;

__global__ __launch_bounds__(kBlock) void seg_count_rows_kernel(int n_rows, const uint32_t* __restrict__ row_count,
                                                                const uint4* __restrict__ rec,
                                                                uint32_t* __restrict__ row_start,
                                                                uint32_t* __restrict__ seg_base,
                                                                uint32_t* __restrict__ seg_row, int ntx,
                                                                uint32_t* __restrict__ slots) {
    extern __shared__ int32_t s_diff[];  // kWaves rows of ntx + 1
    __shared__ uint32_t s_rs[kFusedRows + 1], s_sb[kFusedRows + 1];
    __shared__ uint32_t s_lds[kWaves];
    const int n_real = n_rows - 1;
    {
        // row starts: consecutive rows per thread, one block scan
        const int per = (n_rows + kBlock - 1) / kBlock;
        const int q0 = threadIdx.x * per, q1 = min(n_rows, q0 + per);
        if (row_count) {
            uint32_t c = 0;
            for (int r = q0; r < q1; ++r) c += row_count[r];
            uint32_t tot;
            uint32_t run = block_exclusive_scan<uint32_t>(c, s_lds, tot);
            for (int r = q0; r < q1; ++r) {
                s_rs[r] = run;
                run += row_count[r];
            }
            if (threadIdx.x == 0) s_rs[n_rows] = tot;
        } else {
            for (int r = threadIdx.x; r <= n_rows; r += kBlock) s_rs[r] = row_start[r];
        }
    }
    __syncthreads();
    {
        // segments per real row, one block scan
        const int per = (n_real + kBlock - 1) / kBlock;
        const int r0 = threadIdx.x * per, r1 = min(n_real, r0 + per);
        uint32_t sum = 0;
        for (int r = r0; r < r1; ++r) sum += (s_rs[r + 1] - s_rs[r] + kRunSeg - 1) / kRunSeg;
        uint32_t tot;
        uint32_t run = block_exclusive_scan<uint32_t>(sum, s_lds, tot);
        for (int r = r0; r < r1; ++r) {
            s_sb[r] = run;
            run += (s_rs[r + 1] - s_rs[r] + kRunSeg - 1) / kRunSeg;
        }
        if (threadIdx.x == 0) s_sb[n_real] = tot;
    }
    __syncthreads();
    if (blockIdx.x == 0) {
        if (row_count)
            for (int r = threadIdx.x; r <= n_rows; r += kBlock) row_start[r] = s_rs[r];
        for (int r = threadIdx.x; r <= n_real; r += kBlock) seg_base[r] = s_sb[r];
    }
    const int wave = threadIdx.x >> 6, lane = __lane_id();
    // each XCD a contiguous range of segments: a column's counts of consecutive segments share lines
    const uint32_t sg = (uint32_t)xcd_tile((int)blockIdx.x, (int)gridDim.x) * kWaves + wave;
    if (sg >= s_sb[n_real]) return;  // wave-uniform; no barrier follows
    // the segment's row: the last r with s_sb[r] <= sg (rows without segments share a base with the
    // next row, and the search takes the later one)
    int lo = 0, hi = n_real - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_sb[mid] <= sg) lo = mid; else hi = mid - 1;
    }
    const uint32_t row = (uint32_t)lo;
    if (lane == 0) seg_row[sg] = row;
    const uint32_t sb = s_sb[row], nseg = s_sb[row + 1] - sb;
    const uint32_t k = sg - sb;
    const int64_t b = (int64_t)s_rs[row] + (int64_t)k * kRunSeg;
    const int n_seg = (int)(min((int64_t)s_rs[row + 1], b + kRunSeg) - b);
    // every run's column range loaded before any is counted
    constexpr int kPer = kRunSeg / 64;
    uint32_t z[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) z[j] = 64 * j + lane < n_seg ? rec[b + 64 * j + lane].z : 0u;
    int32_t* d = s_diff + wave * (ntx + 1);
    for (int c = lane; c <= ntx; c += 64) d[c] = 0;
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        if (64 * j + lane < n_seg) {
            atomicAdd(&d[z[j] & 0xffffu], 1);
            atomicAdd(&d[z[j] >> 16], -1);
        }
    }
    wave_lds_sync();
    // columns per lane: a run of consecutive ones, one wavefront scan of the runs' sums
    const int per = (ntx + 63) / 64;
    const int c0 = lane * per, c1 = min(ntx, c0 + per);
    int32_t sum = 0;
    for (int c = c0; c < c1; ++c) sum += d[c];
    int32_t run = wave_inclusive_scan<int32_t>(sum) - sum;
    uint32_t* out = slots + (int64_t)sb * ntx + k;
    for (int c = c0; c < c1; ++c) {
        run += d[c];
        out[(int64_t)c * nseg] = (uint32_t)run;
    }
}

// Per tile (real row, column): exclusive prefix of its segments' counts in place (the slots of a
// tile are consecutive), and the tile's total into tile_tot. One wavefront per tile, lanes over the
// tile's segments, kPrefixChunks chunks of 64 loaded before any is scanned (a lidar frame's rows hold
// hundreds of segments: one memory round trip per group of chunks instead of one per chunk).
constexpr int kPrefixChunks = 8;

__global__ __launch_bounds__(kBlock) void tile_prefix_kernel(uint32_t* __restrict__ slots,
                                                             const uint32_t* __restrict__ seg_base, int n_real,
                                                             int ntx, uint32_t* __restrict__ tile_tot) {
    const int64_t t = ((int64_t)blockIdx.x * kBlock + threadIdx.x) >> 6;
    if (t >= (int64_t)n_real * ntx) return;  // wave-uniform
    const int lane = __lane_id();
    const int row = (int)(t / ntx), c = (int)(t - (int64_t)row * ntx);
    const uint32_t sb = seg_base[row], nseg = seg_base[row + 1] - sb;
    uint32_t* sl = slots + (int64_t)sb * ntx + (int64_t)c * nseg;
    uint32_t carry = 0;
    for (uint32_t k0 = 0; k0 < nseg; k0 += 64 * kPrefixChunks) {
        const int nc = (int)min<uint32_t>(kPrefixChunks, (nseg - k0 + 63) / 64);  // wave-uniform
        uint32_t x[kPrefixChunks];
#pragma unroll
        for (int j = 0; j < kPrefixChunks; ++j) {
            const uint32_t k = k0 + 64u * j + (uint32_t)lane;
            x[j] = (j < nc && k < nseg) ? sl[k] : 0u;
        }
#pragma unroll
        for (int j = 0; j < kPrefixChunks; ++j) {
            if (j >= nc) break;
            const uint32_t k = k0 + 64u * j + (uint32_t)lane;
            const uint32_t inc = wave_inclusive_scan(x[j]);
            if (k < nseg) sl[k] = carry + inc - x[j];
            carry += (uint32_t)__shfl((int)inc, 63, 64);
        }
    }
    if (lane == 0) tile_tot[t] = carry;
}

// single block of 1024 threads: exclusive scan of tile_tot[0, n) in place (the first position of
// every tile of the real rows), the total -- where the negative-depth entries start -- at tile_tot[n];
// with `offsets`, the same positions as int32 (the tile offsets). Each wavefront owns a contiguous
// range: it sums its range (coalesced 64-entry chunks, all loads in flight), one barrier gives every
// wavefront the sum of the ranges before it, and it then scans its range chunk by chunk from the
// registers that hold it (a range past kScanHeld chunks is read again, from the cache). Reading the
// range again for the scan took 7.7 µs at cfg2's 8160 tiles and 21 µs at the six-camera rig's 34 k;
// chunks of 1024 entries across the block, two barriers per chunk, 9 and 23-31 µs; eight consecutive
// entries per thread, 11.9 µs at cfg2.
constexpr int kScanThreads = 1024;
constexpr int kScanHeld = 40;  // chunks of 64 a wavefront keeps in registers between its sum and its scan
__global__ __launch_bounds__(kScanThreads) void tile_scan_kernel(uint32_t* __restrict__ a, int64_t n,
                                                                 int32_t* __restrict__ offsets) {
    constexpr int NW = kScanThreads / 64;
    __shared__ uint32_t s_tot[NW];
    const int wave = threadIdx.x >> 6, lane = __lane_id();
    const int64_t per = ((n + NW - 1) / NW + 63) / 64 * 64;  // whole chunks per wavefront
    const int64_t w0 = min(n, (int64_t)wave * per), w1 = min(n, w0 + per);
    // up to kScanHeld chunks per wavefront (40 k tiles in all) are read once and scanned from registers
    const bool held = per <= 64 * kScanHeld;  // block-uniform
    uint32_t x[kScanHeld];
    uint32_t sum = 0;
    if (held) {
#pragma unroll
        for (int j = 0; j < kScanHeld; ++j) {
            const int64_t i = w0 + 64 * j + lane;
            x[j] = i < w1 ? a[i] : 0u;
            sum += x[j];
        }
    } else {
        for (int64_t i = w0 + lane; i < w1; i += 64) sum += a[i];
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += (uint32_t)__shfl_xor((int)sum, off, 64);
    if (lane == 0) s_tot[wave] = sum;
    __syncthreads();
    uint32_t carry = 0, total = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const uint32_t t = s_tot[w];
        if (w < wave) carry += t;
        total += t;
    }
    auto put = [&](int64_t i, uint32_t v, uint32_t inc) {
        if (i < w1) {
            a[i] = carry + inc - v;
            if (offsets) offsets[i] = (int32_t)(carry + inc - v);
        }
    };
    if (held) {
#pragma unroll
        for (int j = 0; j < kScanHeld; ++j) {
            if (w0 + 64 * j >= w1) break;  // wave-uniform
            const uint32_t inc = wave_inclusive_scan(x[j]);
            put(w0 + 64 * j + lane, x[j], inc);
            carry += (uint32_t)__shfl((int)inc, 63, 64);
        }
    } else {
        for (int64_t c0 = w0; c0 < w1; c0 += 64) {
            const int64_t i = c0 + lane;
            const uint32_t v = i < w1 ? a[i] : 0u;
            const uint32_t inc = wave_inclusive_scan(v);
            put(i, v, inc);
            carry += (uint32_t)__shfl((int)inc, 63, 64);
        }
    }
    if (threadIdx.x == 0) a[n] = total;
}

// Runs of negative-depth instances, after every tile, in run order; each run's entries consecutive
// (their keys' tile bits are saturated by the sign extension). One workgroup. KEYS false writes the
// flatten ids only (a fill whose caller takes the tile offsets instead of the keys).
template <bool KEYS>
XSG_DEV void write_neg_runs(const uint4* __restrict__ rec, int64_t b, int64_t n_runs, uint32_t base, int64_t n_out,
                            int64_t* __restrict__ out_keys, int32_t* __restrict__ out_ids) {
    __shared__ uint32_t lds[kWaves];
    uint32_t carry = base;
    for (int64_t i0 = b; i0 < n_runs; i0 += kBlock) {
        const int64_t i = i0 + threadIdx.x;
        const uint4 rr = i < n_runs ? rec[i] : make_uint4(0, 0, 0, 0);
        const uint32_t w = i < n_runs ? (rr.z >> 16) - (rr.z & 0xffffu) : 0u;
        uint32_t tot;
        const uint32_t ex = block_exclusive_scan<uint32_t>(w, lds, tot);
        for (uint32_t q = 0; q < w; ++q) {
            const uint64_t pos = (uint64_t)carry + ex + q;
            if (pos < (uint64_t)n_out) {
                if constexpr (KEYS) out_keys[pos] = make_key(0u, rr.y);
                out_ids[pos] = (int32_t)rr.x;
            }
        }
        carry += tot;
    }
}

// One workgroup per segment: its runs are read once into LDS, and each wavefront takes bands of
// kBandCols columns in turn. For a band, the runs touching it are first listed in run (depth) order
// (a stable ballot compaction into a wavefront-private LDS list: a run covers about a tenth of a
// row's columns, so most runs touch few bands); then, per group of kColGroup columns, the runs of
// the list covering each column are found by ballot and take consecutive positions from the
// column's slot, in run order. They are staged in a wavefront-private LDS buffer of 64 entries per
// column and stored 64 at a time, so that every global store of a column is a full, contiguous
// wavefront. Workgroup s_max writes the negative-depth runs instead.
template <bool KEYS>
__global__ __launch_bounds__(kBlock) void write_runs_kernel(
    int n_real, const uint4* __restrict__ rec, const uint32_t* __restrict__ row_start,
    const uint32_t* __restrict__ seg_base, const uint32_t* __restrict__ seg_row, const uint32_t* __restrict__ slots,
    const uint32_t* __restrict__ tile_base, int64_t s_max, int64_t n_runs, int ntx, int nty, int tnb,
    int64_t n_out, int64_t* __restrict__ out_keys, int32_t* __restrict__ out_ids) {
    __shared__ uint4 s_rec[kRunSeg];
    __shared__ uint16_t s_list[kWaves][kRunSeg];       // per wavefront: the band's runs, in run order
    __shared__ uint32_t s_dep[kWaves][kColGroup][64];  // staged depth bits (low key word)
    __shared__ int32_t s_gid[kWaves][kColGroup][64];   // staged Gaussian ids
    extern __shared__ uint32_t s_first[];              // [ntx]: first output position per column
    // consecutive segments of a row write the two sides of the cache lines at their column
    // boundaries: on one XCD those partial lines meet in its L2
    const int64_t sg = xcd_tile((int)blockIdx.x, (int)(s_max + 1));
    if (sg == s_max) {
        write_neg_runs<KEYS>(rec, row_start[n_real], n_runs, tile_base[(int64_t)n_real * ntx], n_out, out_keys,
                             out_ids);
        return;
    }
    if (sg >= (int64_t)seg_base[n_real]) return;
    const int lane = __lane_id(), wave = threadIdx.x >> 6;
    const uint32_t row = seg_row[sg];
    const uint32_t sb = seg_base[row], nseg = seg_base[row + 1] - sb;
    const uint32_t k = (uint32_t)sg - sb;
    const int64_t b = (int64_t)row_start[row] + (int64_t)k * kRunSeg;
    const int n_seg = (int)(min((int64_t)row_start[row + 1], b + kRunSeg) - b);
    for (int i = threadIdx.x; i < n_seg; i += kBlock) s_rec[i] = rec[b + i];
    for (int c = threadIdx.x; c < ntx; c += kBlock)
        s_first[c] = tile_base[(int64_t)row * ntx + c] + slots[(int64_t)sb * ntx + (int64_t)c * nseg + k];
    __syncthreads();
    const uint32_t cid = row / (uint32_t)nty, y = row - cid * (uint32_t)nty;
    const uint32_t tile_row = (cid << tnb) | (y * (uint32_t)ntx);
    for (int band = wave; band * kBandCols < ntx; band += kWaves) {
        const int b0 = band * kBandCols, b1 = min(ntx, b0 + kBandCols);
        // the segment's runs that cover a column of [b0, b1), in run order (n_list is wave-uniform)
        int n_list = 0;
        for (int i0 = 0; i0 < n_seg; i0 += 64) {
            const int i = i0 + lane;
            bool hit = false;
            if (i < n_seg) {
                const uint32_t z = s_rec[i].z;
                hit = (int)(z & 0xffffu) < b1 && (int)(z >> 16) > b0;
            }
            const uint64_t mk = __builtin_amdgcn_ballot_w64(hit);
            if (hit)
                s_list[wave][n_list + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32),
                                                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0u))] =
                    (uint16_t)i;
            n_list += __popcll(mk);
        }
        for (int c0 = b0; c0 < b1; c0 += kColGroup) {
            const int nc = min(kColGroup, b1 - c0);
            // per column: global position of the next flushed entry and entries staged in LDS (< 64),
            // both wave-uniform
            uint32_t out[kColGroup], fill[kColGroup];
#pragma unroll
            for (int j = 0; j < kColGroup; ++j) {
                out[j] = j < nc ? (uint32_t)__builtin_amdgcn_readfirstlane((int)s_first[c0 + j]) : 0u;
                fill[j] = 0;
            }
            for (int i0 = 0; i0 < n_list; i0 += 64) {
                const int li = i0 + lane;
                const uint4 rr = li < n_list ? s_rec[s_list[wave][li]] : make_uint4(0, 0, 0, 0);  // width 0 past the end
                const uint32_t x0 = rr.z & 0xffffu, w = (rr.z >> 16) - x0;
                const uint32_t d0 = (uint32_t)c0 - x0;  // column offset in the run; covered iff below w
#pragma unroll
                for (int j = 0; j < kColGroup; ++j) {
                    if (j >= nc) break;
                    const bool cov = d0 + (uint32_t)j < w;
                    const uint64_t mk = __builtin_amdgcn_ballot_w64(cov);
                    const uint32_t cnt = (uint32_t)__popcll(mk);
                    const uint32_t slot = __builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32),
                                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)mk, fill[j]));
                    if (cov && slot < 64) {
                        if constexpr (KEYS) s_dep[wave][j][slot] = rr.y;
                        s_gid[wave][j][slot] = (int32_t)rr.x;
                    }
                    const uint32_t f = (uint32_t)__builtin_amdgcn_readfirstlane((int)(fill[j] + cnt));
                    if (f >= 64) {  // the column's buffer is full: store it, then stage the overflow
                        const uint64_t pos = (uint64_t)out[j] + (uint64_t)lane;
                        if (pos < (uint64_t)n_out) {
                            if constexpr (KEYS)
                                out_keys[pos] = make_key(tile_row + (uint32_t)(c0 + j), s_dep[wave][j][lane]);
                            out_ids[pos] = s_gid[wave][j][lane];
                        }
                        out[j] = (uint32_t)__builtin_amdgcn_readfirstlane((int)(out[j] + 64));
                        if (cov && slot >= 64) {
                            if constexpr (KEYS) s_dep[wave][j][slot - 64] = rr.y;
                            s_gid[wave][j][slot - 64] = (int32_t)rr.x;
                        }
                        fill[j] = f - 64;
                    } else {
                        fill[j] = f;
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < kColGroup; ++j) {
                const uint64_t pos = (uint64_t)out[j] + (uint64_t)lane;
                if (j < nc && (uint32_t)lane < fill[j] && pos < (uint64_t)n_out) {
                    if constexpr (KEYS) out_keys[pos] = make_key(tile_row + (uint32_t)(c0 + j), s_dep[wave][j][lane]);
                    out_ids[pos] = s_gid[wave][j][lane];
                }
            }
        }
    }
}

// Tile offsets of sorted keys by binary search: offsets[t] = first index whose key bits above 32,
// read as unsigned, are >= t's (camera, tile) id -- what the reference's encoder
// (tiling_common.cu:25-71) writes for sorted keys of non-negative depth. A negative depth's
// sign-extended bits set the key's whole upper half, so such entries sort after every tile and lie
// outside every tile's range here; the reference's encoder races on them (its last thread writes
// n_isects over the tiles after 2^tile_bits - 1 - n_tiles while other threads write their starts).
__global__ __launch_bounds__(kBlock) void offset_search_kernel(const int64_t* __restrict__ ids, int64_t n,
                                                               int n_tiles, int tnb, int64_t total,
                                                               int32_t* __restrict__ offsets) {
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= total) return;
    const uint32_t cam = (uint32_t)(t / n_tiles), tile = (uint32_t)(t - (int64_t)cam * n_tiles);
    const uint32_t target = (cam << tnb) | tile;
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((uint32_t)((uint64_t)ids[mid] >> 32) < target) lo = mid + 1; else hi = mid;
    }
    offsets[t] = (int32_t)lo;
}

__global__ __launch_bounds__(kBlock) void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i < n) p[i] = v;
}

// mask_radii_kernel / mask_radii_packed_kernel (mask_radii.cu:10-58)
__global__ __launch_bounds__(kBlock) void mask_radii_kernel(int64_t n, const uint8_t* __restrict__ mask,
                                                            const uint32_t* __restrict__ packed,
                                                            float2* __restrict__ radii) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const bool keep = packed ? ((packed[i / 32] & (1u << (i % 32))) != 0) : (mask[i] != 0);
    if (!keep) radii[i] = make_float2(0.f, 0.f);
}

int tile_n_bits_of(int n_tiles) {  // regular_tiling.cu:96-97
    return (int)floorf(log2f((float)n_tiles)) + 1;
}

int geometry_of(const xsg_isect_desc* d, Geometry& g) {
    if (!d) return xsg_fail(XSG_ERR_INVALID, "null isect descriptor");
    if (d->n < 0 || d->n_cams < 1 || d->tile_w <= 0 || d->tile_h <= 0)
        return xsg_fail(XSG_ERR_INVALID, "invalid isect descriptor (n=%lld cams=%d tile=%dx%d)",
                        (long long)d->n, d->n_cams, d->tile_w, d->tile_h);
    g.kind = d->kind;
    g.sort = d->sort ? 1 : 0;
    g.n_cams = d->n_cams;
    g.n = d->n;
    g.spans = 1;
    switch (d->kind) {
        case XSG_TILING_REGULAR: {
            const int w = (int)d->img_width, h = (int)d->img_height;
            g.ntx = (w + d->tile_w - 1) / d->tile_w;
            g.nty = (h + d->tile_h - 1) / d->tile_h;
            break;
        }
        case XSG_TILING_LIDAR:
            if (d->n_cams != 1) return xsg_fail(XSG_ERR_UNSUPPORTED, "lidar tiling takes one camera");
            if (!d->elev_boundaries || d->n_elev <= 0)
                return xsg_fail(XSG_ERR_INVALID, "lidar tiling needs elevation boundaries");
            g.ntx = ((int)d->img_width + d->tile_w - 1) / d->tile_w;
            g.nty = d->n_elev;
            g.spans = 2;
            break;
        case XSG_TILING_SPHERICAL:
            if (d->n_cams != 1) return xsg_fail(XSG_ERR_UNSUPPORTED, "spherical tiling takes one camera");
            g.ntx = (int)ceilf(d->img_width / (float)d->tile_w);
            g.nty = (int)ceilf(d->img_height / (float)d->tile_h);
            g.spans = 2;
            break;
        default: return xsg_fail(XSG_ERR_INVALID, "unknown tiling kind %d", d->kind);
    }
    if (g.ntx <= 0 || g.nty <= 0 || g.ntx > 65535 || g.nty > 65535)
        return xsg_fail(XSG_ERR_INVALID, "tile grid %d x %d out of range", g.ntx, g.nty);
    g.n_tiles = g.ntx * g.nty;
    g.tnb = tile_n_bits_of(g.n_tiles);
    g.cam_bits = 0;
    while ((1 << g.cam_bits) < d->n_cams) ++g.cam_bits;
    if (g.tnb + g.cam_bits > 31) return xsg_fail(XSG_ERR_INVALID, "too many tiles / cameras for 64-bit keys");
    if (g.n * g.n_cams * g.spans >= (1ll << 31)) return xsg_fail(XSG_ERR_INVALID, "too many Gaussians");
    return XSG_OK;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// The depth pre-order sorts the visible instances' depth bits. Below kPresortLargeAt virtual
// instances (the count sizes the launches on the host; the visible count is known only on the
// device when they are queued), in two stages: a stable most-significant-digit pass over the top 8
// bits of each key's offset from the smallest visible key (the compaction finds the key range)
// splits them into buckets of consecutive key values, and bucket_sort_kernel sorts each bucket by its
// remaining bits: four launches, where four LSD passes over 32 bits take twelve, whose fixed cost
// dominates at these counts; the same stable order. From kPresortLargeAt on (a lidar frame, a camera
// rig: millions of visible instances), four LSD passes in tiles of 2048 keys, where buckets would
// outgrow the LDS or need a wider first digit whose scatter coalesces poorly. One call's launches
// depend on its own arguments only.
constexpr int kPresortItems = 4;
constexpr int kPresortItemsLarge = 8;
constexpr int kPresortRB = 8;  // digit bits of both schemes
constexpr int64_t kPresortLargeAt = 3000000;  // virtual instances (Gaussians x cameras x spans)
constexpr unsigned kPresortGrid = 2048;

// count workspace: per virtual instance rectangle / count / depth bits, block partials, compaction
struct CountWs {
    Rect* rects; uint32_t* vcnt; uint32_t* vkey; uint64_t* partials; uint64_t* cpart;
    uint32_t* comp_id; uint32_t* comp_off; uint32_t* comp_key;
    // depth pre-order (sorted fills only): ping-pong, histograms, device-side count, run offsets
    uint32_t* alt_key; uint32_t* alt_id; uint32_t* hist; uint32_t* dtot; uint32_t* m_dev;
    uint32_t* key_range;  // per count block, then per slice of them: smallest and largest visible depth key
    uint32_t* slice_range;
    // after the pre-order: the depth-ordered instances (keys, ids) and the depth-ordered rectangles
    // (two words each), in whichever pair of the two ping-pong pairs the passes left free
    uint32_t* pre_key; uint32_t* pre_id; uint32_t* drect_lo; uint32_t* drect_hi;
    uint32_t* roff; uint32_t* rpart;
    uint32_t* seam_cnt; uint32_t* seam_ids;  // per count block: its seam Gaussians (two spans only)
    uint64_t* slice64; uint64_t* slice_extra; uint32_t* slice32;  // slice totals of the two-level scans
    // direct run placement (sorted fills of at most kDirectRows row buckets): per count block and
    // bucket the block's runs (scanned in place), and the bucket totals
    bool direct; int n_rows;
    uint32_t* row_hist; uint32_t* row_part; uint32_t* row_tot;
    int64_t n_virtual; unsigned nb;
    size_t bytes;
};

int row_buckets(const Geometry& g) { return g.n_cams * g.nty + 1; }  // camera rows + the negative bucket

CountWs count_ws_layout(const Geometry& g, void* base) {
    CountWs w;
    w.n_virtual = g.n * g.n_cams * g.spans;
    const int64_t nv = w.n_virtual;
    w.nb = (unsigned)(((nv > 0 ? nv : 1) + kCountTile - 1) / kCountTile);
    char* p = (char*)base;
    size_t off = 0;
    w.rects = (Rect*)(p + off); off += align256(sizeof(Rect) * nv);
    const size_t nv2 = g.spans == 2 ? (size_t)nv : 0;  // regular tiling compacts from its inputs
    w.vcnt = (uint32_t*)(p + off); off += align256(4 * nv2);
    w.vkey = (uint32_t*)(p + off); off += align256(4 * nv2);
    w.partials = (uint64_t*)(p + off); off += align256(sizeof(uint64_t) * (w.nb + 3));
    w.cpart = (uint64_t*)(p + off); off += align256(sizeof(uint64_t) * 2 * w.nb);
    w.comp_id = (uint32_t*)(p + off); off += align256(4 * nv);
    w.comp_off = (uint32_t*)(p + off); off += align256(4 * nv);
    w.comp_key = (uint32_t*)(p + off); off += align256(4 * nv);
    const size_t ns = g.sort ? (size_t)nv : 0;
    w.alt_key = (uint32_t*)(p + off); off += align256(4 * ns);
    w.alt_id = (uint32_t*)(p + off); off += align256(4 * ns);
    // the bucket pass scatters the compacted pairs into the alt pair and the bucket sort writes them
    // back in order; the rectangles in depth order then go to the alt pair
    w.pre_key = w.comp_key;
    w.pre_id = w.comp_id;
    w.drect_lo = w.alt_key;
    w.drect_hi = w.alt_id;
    w.roff = (uint32_t*)(p + off); off += align256(4 * ns);
    w.hist = (uint32_t*)(p + off);
    const size_t nv1 = nv > 0 ? (size_t)nv : 1;
    const size_t hist_words = ((size_t)1 << kPresortRB) * sort_blocks<kPresortItems>(nv1);
    off += align256(g.sort ? 4 * hist_words : 0);
    w.dtot = (uint32_t*)(p + off); off += align256(4 * ((size_t)1 << kPresortRB));
    w.rpart = (uint32_t*)(p + off); off += align256(4 * ((size_t)w.nb + 1));
    w.m_dev = (uint32_t*)(p + off); off += align256(4);
    const size_t n_slices = ((size_t)w.nb + kSlice - 1) / kSlice;
    w.key_range = (uint32_t*)(p + off); off += align256(8 * (size_t)w.nb);
    w.slice_range = (uint32_t*)(p + off); off += align256(8 * n_slices);
    w.seam_cnt = (uint32_t*)(p + off); off += align256(g.spans == 2 ? 4 * (size_t)w.nb : 0);
    w.seam_ids = (uint32_t*)(p + off); off += align256(g.spans == 2 ? 4 * (size_t)w.nb * (kCountTile / 2) : 0);
    w.slice64 = (uint64_t*)(p + off); off += align256(8 * n_slices);
    w.slice_extra = (uint64_t*)(p + off); off += align256(16 * n_slices);
    w.slice32 = (uint32_t*)(p + off); off += align256(4 * n_slices);
    w.n_rows = row_buckets(g);
    w.direct = g.sort && w.n_rows <= kDirectRows;
    const size_t nr = w.direct ? (size_t)w.n_rows : 0;
    w.row_hist = (uint32_t*)(p + off); off += align256(4 * nr * w.nb * kGroupsPerCountBlock);
    w.row_part = (uint32_t*)(p + off);
    const int64_t n_groups = (int64_t)w.nb * kGroupsPerCountBlock;
    off += align256(4 * nr * (size_t)((n_groups + group_slice(n_groups) - 1) / group_slice(n_groups)));
    w.row_tot = (uint32_t*)(p + off); off += align256(4 * nr);
    w.bytes = off;
    return w;
}

struct FillWs {
    uint32_t* row_a; uint32_t* row_b;               // run row buckets and ping-pong [n_runs]
    uint4* rec_a; uint4* rec_b;                     // run records and ping-pong [n_runs]
    uint32_t* row_start; uint32_t* seg_base; uint32_t* seg_row;
    uint32_t* slots; uint32_t* tile_tot;
    uint32_t* hist; uint32_t* dtot;
    uint32_t* blk_first; uint32_t* blk_last;       // each expansion block's first and last instance
    int n_rows;                                     // row buckets incl. the negative one
    int row_bits, rb, passes;                       // row bucket bits, run sort digit width and passes
    int64_t s_max;                                  // segment bound
    int64_t n_slots;
    size_t bytes;
};

FillWs fill_ws_layout(const Geometry& g, int64_t n_runs, void* base) {
    char* p = (char*)base;
    FillWs w{};
    size_t off = 0;
    w.n_rows = row_buckets(g);
    const bool direct = w.n_rows <= kDirectRows;  // the runs are placed, not sorted: one record array
    w.row_bits = 1;
    while ((1u << w.row_bits) <= (uint32_t)(w.n_rows - 1)) ++w.row_bits;
    w.rb = run_sort_rb(w.row_bits);
    w.passes = (w.row_bits + w.rb - 1) / w.rb;
    w.s_max = n_runs / kRunSeg + w.n_rows;
    w.n_slots = w.s_max * g.ntx;
    const unsigned nb_r = sort_blocks<kRunSortItems>(n_runs > 0 ? n_runs : 1);
    auto take = [&](size_t bytes) { void* q = p + off; off += align256(bytes); return q; };
    const size_t n_sorted = direct ? 0 : (size_t)n_runs;
    w.row_a = (uint32_t*)take(4 * n_sorted);
    w.row_b = (uint32_t*)take(4 * n_sorted);
    w.rec_a = (uint4*)take(16 * n_runs);
    w.rec_b = (uint4*)take(16 * n_sorted);
    w.row_start = (uint32_t*)take(4 * ((size_t)w.n_rows + 1));
    w.seg_base = (uint32_t*)take(4 * ((size_t)w.n_rows + 1));
    w.seg_row = (uint32_t*)take(4 * (size_t)w.s_max);
    w.slots = (uint32_t*)take(4 * (size_t)w.n_slots);
    w.tile_tot = (uint32_t*)take(4 * ((size_t)(w.n_rows - 1) * g.ntx + 1));
    w.hist = (uint32_t*)take(direct ? 0 : 4 * ((size_t)1 << w.rb) * nb_r);
    w.dtot = (uint32_t*)take(direct ? 0 : 4 * ((size_t)1 << w.rb));
    w.blk_first = (uint32_t*)take(direct ? 0 : 4 * (size_t)nb_r);
    w.blk_last = (uint32_t*)take(direct ? 0 : 4 * (size_t)nb_r);
    w.bytes = off;
    return w;
}

// The runs' expansion (which stores the first digit's per-tile histogram) and their stable sort by
// row bucket, RB bits per pass; the result ends in (out_row, out_rec), the b buffers for an odd
// number of passes.
template <int RB>
void expand_and_sort_runs(const FillWs& fw, const CountWs& cw, int64_t n_runs, int64_t m, int nty, int64_t n_per_cam,
                          int spans, uint32_t neg_row, uint32_t* out_row, uint4* out_rec, hipStream_t s) {
    const unsigned nb_runs = sort_blocks<kRunSortItems>(n_runs);
    run_block_bounds_kernel<<<xsg_blocks(m, kBlock), kBlock, 0, s>>>(m, cw.roff, n_runs, fw.blk_first, fw.blk_last);
    expand_runs_kernel<RB><<<nb_runs, kBlock, 0, s>>>(n_runs, cw.roff, cw.pre_id, cw.pre_key, m, cw.drect_lo,
                                                      cw.drect_hi, nty, n_per_cam, spans, neg_row, fw.row_a, fw.rec_a,
                                                      fw.hist, nb_runs, fw.blk_first, fw.blk_last);
    radix_sort_passes<uint32_t, uint4, PlainOut<uint32_t, uint4>, kRunSortItems, RB>(
        fw.row_a, fw.rec_a, fw.row_b, fw.rec_b, n_runs, 0, fw.row_bits, fw.hist, fw.dtot,
        PlainOut<uint32_t, uint4>{out_row, out_rec}, s, nullptr, /*first_hist_ready=*/true);
}

}  // namespace

extern "C" int xsg_isect_geometry(const xsg_isect_desc* d, int* ntw, int* nth, int* tnb, int* bits_above) {
    Geometry g;
    const int rc = geometry_of(d, g);
    if (rc) return rc;
    if (ntw) *ntw = g.ntx;
    if (nth) *nth = g.nty;
    if (tnb) *tnb = g.tnb;
    if (bits_above) *bits_above = g.tnb + g.cam_bits;
    return XSG_OK;
}

extern "C" size_t xsg_isect_count_workspace_bytes(const xsg_isect_desc* d) {
    Geometry g;
    if (geometry_of(d, g)) return 0;
    return count_ws_layout(g, nullptr).bytes;
}

// Per host thread and device: a mapped pinned host buffer that the count phase writes its totals to,
// and the event that marks the write. Allocated on a thread's first count on a device and kept until
// the thread calls xsg_release_thread_resources (64 bytes of pinned memory and one event per device).
struct CountReadback {
    uint64_t* host = nullptr;  // host view
    uint64_t* dev = nullptr;   // device view of the same memory
    hipEvent_t ev = nullptr;
};

static thread_local std::vector<CountReadback> tl_readbacks;

extern "C" int xsg_release_thread_resources(void) {
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return xsg_launch_status("release_thread_resources device");
    int rc = XSG_OK;
    for (size_t d = 0; d < tl_readbacks.size(); ++d) {
        CountReadback& rb = tl_readbacks[d];
        if (!rb.host) continue;
        // xsg_isect_count waited for the event before it returned, so no queued work still writes here
        if (hipSetDevice((int)d) != hipSuccess || hipEventDestroy(rb.ev) != hipSuccess ||
            hipHostFree(rb.host) != hipSuccess)
            rc = xsg_launch_status("release_thread_resources");
        rb = CountReadback{};
    }
    tl_readbacks.clear();
    if (hipSetDevice(cur) != hipSuccess && rc == XSG_OK) rc = xsg_launch_status("release_thread_resources device");
    return rc;
}

static int count_readback(CountReadback*& out) {
    std::vector<CountReadback>& per_device = tl_readbacks;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return xsg_launch_status("isect_count readback device");
    if ((int)per_device.size() <= dev) per_device.resize(dev + 1);
    CountReadback& rb = per_device[dev];
    if (!rb.host) {
        void* h = nullptr;
        if (hipHostMalloc(&h, 64, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess)
            return xsg_launch_status("isect_count readback buffer");
        void* d = nullptr;
        if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess) return xsg_launch_status("isect_count readback map");
        hipEvent_t ev = nullptr;
        if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess)
            return xsg_launch_status("isect_count readback event");
        rb.host = static_cast<uint64_t*>(h);
        rb.dev = static_cast<uint64_t*>(d);
        rb.ev = ev;
    }
    out = &rb;
    return XSG_OK;
}

// The depth pre-order: the bucket pass (compacted pairs -> alt pair, by the top RB bits of each key's
// offset in the visible key range) and the per-bucket sort (alt pair -> pre pair).
template <int ITEMS, int RB>
void presort_buckets(const CountWs& w, int range_parts, hipStream_t s) {
    const unsigned nb = sort_blocks<ITEMS>(w.n_virtual);
    const unsigned grid = min(nb, kPresortGrid);
    radix_upsweep<uint32_t, ITEMS, RB, true><<<grid, kSortBlock, 0, s>>>(w.comp_key, w.n_virtual, 0, RB, w.hist, nb,
                                                                        w.m_dev, w.slice_range, range_parts);
    radix_scan_hist<ITEMS><<<1u << RB, kSortBlock, 0, s>>>(w.hist, nb, w.dtot, w.n_virtual, w.m_dev);
    radix_downsweep<uint32_t, uint32_t, PlainOut<uint32_t, uint32_t>, ITEMS, RB, true><<<grid, kSortBlock, 0, s>>>(
        w.comp_key, w.comp_id, w.n_virtual, 0, RB, w.hist, w.dtot, nb, PlainOut<uint32_t, uint32_t>{w.alt_key, w.alt_id},
        w.m_dev, w.slice_range, range_parts);
    bucket_sort_kernel<RB><<<1u << RB, kBucketThreads, 0, s>>>(w.dtot, w.slice_range, range_parts, w.alt_key, w.alt_id,
                                                               w.pre_key, w.pre_id);
}

extern "C" int xsg_isect_count(const xsg_isect_desc* d, int32_t* tpg, void* workspace, int64_t* n_isects,
                               int64_t* n_visible, int64_t* n_runs, xsg_stream_t stream) {
    Geometry g;
    int rc = geometry_of(d, g);
    if (rc) return rc;
    const int64_t nt = g.n * g.n_cams;
    if (n_isects) *n_isects = 0;
    if (n_visible) *n_visible = 0;
    if (n_runs) *n_runs = 0;
    if (nt == 0) return XSG_OK;
    if (!workspace || !tpg || !d->means2d || !d->radii || !d->depths)
        return xsg_fail(XSG_ERR_INVALID, "xsg_isect_count: null pointer");
    if (const int rc2 = xsg_check_workspace(workspace, "xsg_isect_count")) return rc2;
    const hipStream_t s = (hipStream_t)stream;
    const CountWs w = count_ws_layout(g, workspace);
    // the bucketed depth pre-order takes its first digit from the visible keys' range: every count
    // block records its own, each slice scan workgroup reduces its blocks' (no atomics)
    const bool large_presort = w.n_virtual >= kPresortLargeAt;
    uint32_t* key_range = g.sort && !large_presort ? w.key_range : nullptr;
    if (g.kind == XSG_TILING_REGULAR) {
        count_regular_kernel<<<w.nb, kBlock, 0, s>>>(nt, (const float2*)d->means2d, (const float2*)d->radii,
                                                     (float)d->tile_w, (float)d->tile_h, g.ntx, g.nty, tpg,
                                                     w.rects, w.partials, w.cpart, d->depths, key_range);
    } else {
        if (!d->camera_pack || !d->flags || !d->points || !d->scales || !d->quats)
            return xsg_fail(XSG_ERR_INVALID, "lidar / spherical tiling needs camera and Gaussian tensors");
        const UtWeights ut = xsg_ut_weights(d->ut_alpha, d->ut_beta, d->ut_kappa);
        const f2 img = mk2(d->img_width, d->img_height);
        const float u_per_tile = (float)d->tile_w / d->img_width;
        const float v_per_tile = (float)d->tile_h / d->img_height;
        const unsigned seam_grid = (w.nb + kSeamBlocks - 1) / kSeamBlocks;
        if (g.kind == XSG_TILING_LIDAR) {
            count_spherical_kernel<XSG_CAM_LIDAR, true><<<w.nb, kBlock, 0, s>>>(
                nt, d->camera_pack, img, d->flags, (const float2*)d->means2d, (const float2*)d->radii, d->depths,
                d->elev_boundaries, d->n_elev, u_per_tile, v_per_tile, g.ntx, g.nty, tpg, w.rects, w.vcnt, w.vkey,
                w.partials, w.cpart, w.seam_cnt, w.seam_ids, key_range);
            seam_span_kernel<XSG_CAM_LIDAR, true><<<seam_grid, kBlock, 0, s>>>(
                w.nb, w.seam_cnt, w.seam_ids, d->camera_pack, ut, img, d->points, d->velocity, d->scales,
                (const float4*)d->quats, d->opacity, d->elev_boundaries, d->n_elev, u_per_tile, v_per_tile, g.ntx,
                g.nty, tpg, w.rects, w.vcnt, w.vkey, w.partials, w.cpart, key_range);
        } else {
            count_spherical_kernel<XSG_CAM_SPHERICAL, false><<<w.nb, kBlock, 0, s>>>(
                nt, d->camera_pack, img, d->flags, (const float2*)d->means2d, (const float2*)d->radii, d->depths,
                nullptr, 0, u_per_tile, v_per_tile, g.ntx, g.nty, tpg, w.rects, w.vcnt, w.vkey, w.partials, w.cpart,
                w.seam_cnt, w.seam_ids, key_range);
            seam_span_kernel<XSG_CAM_SPHERICAL, false><<<seam_grid, kBlock, 0, s>>>(
                w.nb, w.seam_cnt, w.seam_ids, d->camera_pack, ut, img, d->points, d->velocity, d->scales,
                (const float4*)d->quats, d->opacity, nullptr, 0, u_per_tile, v_per_tile, g.ntx, g.nty, tpg, w.rects,
                w.vcnt, w.vkey, w.partials, w.cpart, key_range);
        }
    }
    // the totals are final after the compaction, which publishes them to pinned host memory; an event
    // marks that write, so that the host reads them while the depth pre-order and row offsets below
    // still run
    CountReadback* rb = nullptr;
    rc = count_readback(rb);
    if (rc) return rc;
    const unsigned n_slices = (w.nb + kSlice - 1) / kSlice;
    slice_scan_kernel<uint64_t><<<n_slices, kBlock, 0, s>>>(w.nb, w.partials, w.slice64, w.cpart, w.slice_extra,
                                                            key_range, w.slice_range);
    // regular tiling has one span per instance: its counts are tiles_per_gauss and its depth bits the
    // depths themselves
    const bool regular = g.kind == XSG_TILING_REGULAR;
    compact_kernel<<<w.nb, kBlock, 0, s>>>(w.n_virtual, regular ? reinterpret_cast<const uint32_t*>(tpg) : w.vcnt,
                                           regular ? reinterpret_cast<const uint32_t*>(d->depths) : w.vkey,
                                           w.partials, w.slice64, w.slice_extra,
                                           n_slices, w.comp_id, w.comp_off, w.comp_key,
                                           g.sort ? w.m_dev : nullptr, rb->dev);
    if (hipEventRecord(rb->ev, s) != hipSuccess) return xsg_launch_status("isect_count readback event");
    if (g.sort) {
        // queued ahead of the readback, sized on the device: the visible spans in depth order
        // (stable; result in pre_key / pre_id), then their row-run offsets
        if (large_presort)  // four LSD passes over the 32 depth bits (an even count: the result is back in pre)
            radix_sort_passes<uint32_t, uint32_t, PlainOut<uint32_t, uint32_t>, kPresortItemsLarge, kPresortRB>(
                w.comp_key, w.comp_id, w.alt_key, w.alt_id, w.n_virtual, 0, 32, w.hist, w.dtot,
                PlainOut<uint32_t, uint32_t>{w.pre_key, w.pre_id}, s, w.m_dev, false, kPresortGrid);
        else
            presort_buckets<kPresortItems, kPresortRB>(w, (int)n_slices, s);
        // the depth-ordered rectangles go to the bucket pass's output pair (free after the bucket sort)
        if (w.direct) {  // per count block and row bucket, the block's runs; their scans
            const int64_t n_per_cam = g.n_cams > 1 ? g.n : 0;
            const int64_t n_groups = (int64_t)w.nb * kGroupsPerCountBlock;
            rows_hist_kernel<<<w.nb * (kGroupsPerCountBlock / kWaves), kBlock, 0, s>>>(
                w.n_virtual, w.m_dev, w.pre_id, w.pre_key, w.rects, g.nty, n_per_cam, g.spans, w.n_rows, n_groups,
                w.row_hist, w.drect_lo, w.drect_hi);
            const int64_t slice = group_slice(n_groups);
            const dim3 sgrid((unsigned)w.n_rows, (unsigned)((n_groups + slice - 1) / slice));
            const bool one_slice = sgrid.y == 1;
            if (!one_slice)
                group_slice_sum_kernel<<<sgrid, kBlock, 0, s>>>(w.row_hist, n_groups, slice, w.m_dev, w.row_part);
            group_slice_scan_kernel<<<sgrid, kBlock, 0, s>>>(w.row_hist, n_groups, slice, w.m_dev,
                                                             one_slice ? nullptr : w.row_part, w.row_tot);
        } else {
            rows_reduce_kernel<<<w.nb, kBlock, 0, s>>>(w.n_virtual, w.m_dev, w.pre_id, w.rects, w.rpart, w.drect_lo,
                                                       w.drect_hi);
            slice_scan_kernel<uint32_t><<<n_slices, kBlock, 0, s>>>(w.nb, w.rpart, w.slice32, nullptr, nullptr);
            rows_scan_kernel<<<w.nb, kBlock, 0, s>>>(w.n_virtual, w.m_dev, w.drect_lo, w.drect_hi, w.rpart,
                                                     w.slice32, w.roff);
        }
    }
    XSG_TRY_LAUNCH("isect_count");
    // packed (visible << 32 | count) total, exact intersection total, exact row-run total; poll the
    // event rather than block on it (waking from a blocking wait costs more than the short wait)
    hipError_t q;
    while ((q = hipEventQuery(rb->ev)) == hipErrorNotReady) {
    }
    if (q != hipSuccess) return xsg_launch_status("isect_count readback");
    const volatile uint64_t* hv = rb->host;
    const uint64_t total[3] = {hv[0], hv[1], hv[2]};
    // below 2^31 intersections the packed count field never carried, so its visible count is exact
    if (total[1] >= (1ull << 31))
        return xsg_fail(XSG_ERR_INVALID, "%llu intersections exceed the int32 range of flatten ids",
                        (unsigned long long)total[1]);
    if (n_isects) *n_isects = (int64_t)total[1];
    if (n_visible) *n_visible = (int64_t)(total[0] >> 32);
    if (n_runs) *n_runs = (int64_t)total[2];
    return XSG_OK;
}

extern "C" size_t xsg_isect_fill_workspace_bytes(const xsg_isect_desc* d, int64_t n_isects, int64_t n_visible,
                                                 int64_t n_runs) {
    Geometry g;
    if (geometry_of(d, g) || n_isects < 0 || n_visible < 0 || n_runs < 0) return 0;
    return fill_ws_layout(g, n_runs, nullptr).bytes;
}

extern "C" int xsg_isect_fill(const xsg_isect_desc* d, int64_t n_isects, int64_t n_visible, int64_t n_runs,
                              int sort, void* count_workspace, void* fill_workspace, int64_t* isect_ids,
                              int32_t* flatten_ids, int32_t* tile_offsets, int64_t n_tile_offsets,
                              xsg_stream_t stream) {
    Geometry g;
    int rc = geometry_of(d, g);
    if (rc) return rc;
    if (tile_offsets) {
        if (!sort) return xsg_fail(XSG_ERR_INVALID, "xsg_isect_fill: tile offsets come with a sorted fill");
        if (n_tile_offsets != (int64_t)g.n_cams * g.n_tiles)
            return xsg_fail(XSG_ERR_INVALID, "xsg_isect_fill: %lld tile offsets for a grid of %d x %d x %d tiles",
                            (long long)n_tile_offsets, g.n_cams, g.nty, g.ntx);
    }
    if (!isect_ids && !(sort && tile_offsets))
        return xsg_fail(XSG_ERR_INVALID, "xsg_isect_fill: the keys may be left out only by a sorted fill that writes "
                                         "the tile offsets");
    if (n_isects == 0) {  // tiling_common.cu:86-88: every offset 0
        if (tile_offsets)
            fill_i32_kernel<<<xsg_blocks(n_tile_offsets, kBlock), kBlock, 0, (hipStream_t)stream>>>(tile_offsets,
                                                                                                   n_tile_offsets, 0);
        XSG_TRY_LAUNCH("isect_fill");
        return XSG_OK;
    }
    const CountWs cw = count_ws_layout(g, count_workspace);
    if (n_isects < 0 || n_visible <= 0 || n_visible > cw.n_virtual || n_runs <= 0 || n_runs > n_isects ||
        !count_workspace || !flatten_ids)
        return xsg_fail(XSG_ERR_INVALID, "xsg_isect_fill: bad arguments");
    if (const int rc2 = xsg_check_workspace(count_workspace, "xsg_isect_fill")) return rc2;
    const hipStream_t s = (hipStream_t)stream;
    const int64_t m = n_visible;
    const int64_t n_per_cam = g.n_cams > 1 ? g.n : 0;
    if (!sort) {
        if (g.sort) return xsg_fail(XSG_ERR_INVALID, "xsg_isect_fill: unsorted fill of a descriptor counted with sort = 1");
        const unsigned nb_expand = (unsigned)((n_isects + kExpandPerBlock - 1) / kExpandPerBlock);
        expand_kernel<FinalOut><<<nb_expand, kBlock, 0, s>>>(n_isects, cw.comp_off, cw.comp_id, cw.comp_key, m,
                                                             cw.rects, g.ntx, g.tnb, n_per_cam, g.spans,
                                                             FinalOut{isect_ids, flatten_ids});
        XSG_TRY_LAUNCH("isect_fill (unsorted)");
        return XSG_OK;
    }
    if (!fill_workspace) return xsg_fail(XSG_ERR_INVALID, "xsg_isect_fill: null fill workspace");
    if (const int rc2 = xsg_check_workspace(fill_workspace, "xsg_isect_fill")) return rc2;
    if (!g.sort) return xsg_fail(XSG_ERR_INVALID, "xsg_isect_fill: sorted fill of a descriptor counted with sort = 0");
    if (g.ntx > kMaxSortedCols)
        return xsg_fail(XSG_ERR_UNSUPPORTED, "sorted binning supports at most %d tile columns (got %d)", kMaxSortedCols,
                        g.ntx);
    const FillWs fw = fill_ws_layout(g, n_runs, fill_workspace);
    const uint32_t neg_row = (uint32_t)(fw.n_rows - 1);
    const int n_real = fw.n_rows - 1;
    const uint4* rec;
    const uint32_t* row_count;  // with one pass or direct placement: the bucket totals (else row_start)
    if (cw.direct) {
        // every run written to its place in (row bucket, depth) order
        place_runs_kernel<<<(unsigned)((m + 63) / 64), 64, 0, s>>>(
            m, cw.pre_id, cw.pre_key, cw.drect_lo, cw.drect_hi, g.nty, n_per_cam, g.spans, fw.n_rows,
            (int64_t)cw.nb * kGroupsPerCountBlock, cw.row_hist, cw.row_tot, fw.rec_a);
        rec = fw.rec_a;
        row_count = cw.row_tot;
    } else {
        // stable sort of the runs (row bucket, record) by row bucket, ping-ponging between the a and b
        // buffers: an odd number of passes ends in b
        const bool odd = fw.passes % 2 == 1;
        uint32_t* rows_sorted = odd ? fw.row_b : fw.row_a;
        uint4* rec_sorted = odd ? fw.rec_b : fw.rec_a;
        rec = rec_sorted;
        row_count = fw.passes == 1 ? fw.dtot : nullptr;
        switch (fw.rb) {
            case 9: expand_and_sort_runs<9>(fw, cw, n_runs, m, g.nty, n_per_cam, g.spans, neg_row, rows_sorted,
                                            rec_sorted, s); break;
            case 10: expand_and_sort_runs<10>(fw, cw, n_runs, m, g.nty, n_per_cam, g.spans, neg_row, rows_sorted,
                                              rec_sorted, s); break;
            default: expand_and_sort_runs<8>(fw, cw, n_runs, m, g.nty, n_per_cam, g.spans, neg_row, rows_sorted,
                                             rec_sorted, s); break;
        }
        if (fw.passes > 1)
            row_start_kernel<<<xsg_blocks(n_runs + 1, kBlock), kBlock, 0, s>>>(rows_sorted, n_runs, fw.n_rows,
                                                                             fw.row_start);
    }
    // column counts per segment; per tile, the exclusive prefix over its segments and the tile total;
    // one exclusive scan over the tile totals
    if (fw.n_rows <= kFusedRows) {
        seg_count_rows_kernel<<<(unsigned)((fw.s_max + kWaves - 1) / kWaves), kBlock,
                                sizeof(int32_t) * kWaves * (g.ntx + 1), s>>>(
            fw.n_rows, row_count, rec, fw.row_start, fw.seg_base, fw.seg_row, g.ntx, fw.slots);
    } else {
        row_segments_kernel<<<1, kBlock, 0, s>>>(fw.n_rows, row_count, fw.row_start, fw.seg_base, fw.seg_row);
        seg_count_kernel<<<(unsigned)fw.s_max, kBlock, sizeof(int32_t) * (g.ntx + 1), s>>>(
            n_real, rec, fw.row_start, fw.seg_base, fw.seg_row, g.ntx, fw.slots);
    }
    const int64_t n_tile_slots = (int64_t)n_real * g.ntx;
    tile_prefix_kernel<<<xsg_blocks(n_tile_slots * 64, kBlock), kBlock, 0, s>>>(fw.slots, fw.seg_base, n_real,
                                                                               g.ntx, fw.tile_tot);
    // the exclusive scan over the tiles is each tile's first output position: the reference's
    // offsets of the sorted keys (negative-depth runs follow every tile)
    tile_scan_kernel<<<1, kScanThreads, 0, s>>>(fw.tile_tot, n_tile_slots, tile_offsets);
    // the writers (one extra workgroup for the negative-depth runs)
    auto writer = isect_ids ? write_runs_kernel<true> : write_runs_kernel<false>;
    writer<<<(unsigned)fw.s_max + 1, kBlock, sizeof(uint32_t) * g.ntx, s>>>(n_real, rec, fw.row_start, fw.seg_base,
                                                                         fw.seg_row, fw.slots, fw.tile_tot, fw.s_max,
                                                                         n_runs, g.ntx, g.nty, g.tnb, n_isects,
                                                                         isect_ids, flatten_ids);
    XSG_TRY_LAUNCH("isect_fill");
    return XSG_OK;
}

extern "C" int xsg_isect_offset_encode(const int64_t* isect_ids, int64_t n_isects, int n_tiles_w, int n_tiles_h,
                                       int n_cams, int32_t* offsets, xsg_stream_t stream) {
    if (n_tiles_w <= 0 || n_tiles_h <= 0 || n_cams < 1 || !offsets || n_isects < 0)
        return xsg_fail(XSG_ERR_INVALID, "xsg_isect_offset_encode: bad arguments");
    const hipStream_t s = (hipStream_t)stream;
    const int n_tiles = n_tiles_w * n_tiles_h;
    const int64_t total = (int64_t)n_tiles * n_cams;
    if (n_isects == 0) {  // tiling_common.cu:86-88
        fill_i32_kernel<<<xsg_blocks(total, kBlock), kBlock, 0, s>>>(offsets, total, 0);
    } else {
        offset_search_kernel<<<xsg_blocks(total, kBlock), kBlock, 0, s>>>(isect_ids, n_isects, n_tiles,
                                                                          tile_n_bits_of(n_tiles), total, offsets);
    }
    XSG_TRY_LAUNCH("isect_offset_encode");
    return XSG_OK;
}

extern "C" int xsg_mask_radii(int64_t n, const uint8_t* mask, float* radii, xsg_stream_t stream) {
    if (n < 0 || (!mask && n) || (!radii && n)) return xsg_fail(XSG_ERR_INVALID, "xsg_mask_radii: bad arguments");
    if (n == 0) return XSG_OK;
    mask_radii_kernel<<<xsg_blocks(n, kBlock), kBlock, 0, (hipStream_t)stream>>>(n, mask, nullptr, (float2*)radii);
    XSG_TRY_LAUNCH("mask_radii");
    return XSG_OK;
}

extern "C" int xsg_mask_radii_packed(int64_t n, const uint32_t* packed, float* radii, xsg_stream_t stream) {
    if (n < 0 || (!packed && n) || (!radii && n))
        return xsg_fail(XSG_ERR_INVALID, "xsg_mask_radii_packed: bad arguments");
    if (n == 0) return XSG_OK;
    mask_radii_kernel<<<xsg_blocks(n, kBlock), kBlock, 0, (hipStream_t)stream>>>(n, nullptr, packed, (float2*)radii);
    XSG_TRY_LAUNCH("mask_radii_packed");
    return XSG_OK;
}

// ------------------------------------------------------------------ generic sort (C-ABI)
extern "C" size_t xsg_radix_sort_workspace_bytes(int64_t n) {
    return align256(4 * (size_t)kRadix * sort_blocks(n > 0 ? n : 1)) + align256(4 * kRadix);
}

extern "C" int xsg_radix_sort_pairs_u64_i32(int64_t* keys, int32_t* vals, int64_t* keys_alt, int32_t* vals_alt,
                                            int64_t n, int begin_bit, int end_bit, void* workspace, int* selector,
                                            xsg_stream_t stream) {
    if (n < 0 || begin_bit < 0 || end_bit > 64 || begin_bit > end_bit || !selector)
        return xsg_fail(XSG_ERR_INVALID, "xsg_radix_sort_pairs_u64_i32: bad arguments");
    *selector = 0;
    if (n == 0 || begin_bit == end_bit) return XSG_OK;
    if (!workspace || !keys || !vals || !keys_alt || !vals_alt)
        return xsg_fail(XSG_ERR_INVALID, "xsg_radix_sort_pairs_u64_i32: null pointer");
    if (const int rc = xsg_check_workspace(workspace, "xsg_radix_sort_pairs_u64_i32")) return rc;
    uint32_t* hist = (uint32_t*)workspace;
    uint32_t* dtot = (uint32_t*)((char*)workspace + align256(4 * (size_t)kRadix * sort_blocks(n)));
    using K = uint64_t;
    using V = uint32_t;
    K* k0 = (K*)keys; V* v0 = (V*)vals; K* k1 = (K*)keys_alt; V* v1 = (V*)vals_alt;
    const int passes = (end_bit - begin_bit + 7) / 8;
    const bool in_alt = (passes % 2) == 1;
    PlainOut<K, V> fin{in_alt ? k1 : k0, in_alt ? v1 : v0};
    radix_sort_passes<K, V, PlainOut<K, V>>(k0, v0, k1, v1, n, begin_bit, end_bit, hist, dtot, fin,
                                            (hipStream_t)stream);
    *selector = in_alt ? 1 : 0;
    XSG_TRY_LAUNCH("radix_sort_pairs");
    return XSG_OK;
}
