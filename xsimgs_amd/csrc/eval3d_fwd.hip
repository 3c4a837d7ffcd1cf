// Forward eval3d compositing: rasterize_eval3d_[dynamic_]fwd_kernel (eval3d_fwd.cu:34-166,
// eval3d_dynamic_fwd.cu:37-173).
#include <type_traits>

#include "xsg_eval3d.h"

namespace xsg {
namespace {

// NT threads per workgroup, one per pixel: 256 for tiles of up to 256 pixels, 1024 for larger ones
// (the reference launches tile_w * tile_h threads, eval3d_fwd.cu:204-221). The 1024-thread variant
// stages up to 8 colour channels in LDS, so that its batch of 1024 Gaussians fits.
template <int CDIM, bool DYN, int NT, bool COUNT>
__global__ __launch_bounds__(NT) void eval3d_fwd_kernel(Eval3dParams p) {
    constexpr int kLdsColors = NT > kTileThreads ? 8 : kColorLdsMax;
    constexpr int CL = (CDIM > 0 && CDIM <= kLdsColors) ? CDIM : 0;   // channels staged in LDS
    constexpr int C4 = (CL + 3) / 4;                                   // float4 slots of them
    constexpr int CS = CDIM > 0 ? CDIM : 1;
    constexpr int NW = NT / 64;
    // The opacity rides in the last colour float4's first free component when there is one, so that a
    // pair reads four float4s (M rows with gro or the mean, colours with opacity)
    constexpr bool OP_IN_COL = CL > 0 && (CL & 3) != 0;
    // Every per-Gaussian slot is a float4 indexed by the batch position, so one address register
    // serves all reads of a pair. The M rows' fourth components hold gro = M (o - mu) when the tile's
    // rays share one origin, else the mean.
    __shared__ float4 s_m0[NT], s_m1[NT], s_m2[NT];  // M rows | gro or mean
    __shared__ float s_op[OP_IN_COL ? 1 : NT];       // opacity, when no colour slot has room
    __shared__ float4 s_vel[DYN ? NT : 1];
    __shared__ float4 s_col[C4 > 0 ? C4 : 1][NT];
    __shared__ int32_t s_id[CL > 0 ? 1 : NT];
    __shared__ float s_origin[3];
    __shared__ RayBundle s_bundle[NW];
    __shared__ uint64_t s_mask[NW][NW];  // [wavefront][staging wavefront]: Gaussians it evaluates

    const TileGrid& g = p.g;
    const PixelCtx c = pixel_ctx(g, p.offsets);
    const int bs = g.tile_w * g.tile_h;
    const int nw = (bs + 63) >> 6;  // the workgroup is nw whole wavefronts; threads >= bs own no pixel
    const int wave = c.tr >> 6, lane = c.tr & 63;
    bool done = !c.inside;
    const f3 rd = c.inside ? ld3(p.ray_d + 3 * c.pix) : mk3(0.f, 0.f, 0.f);
    const f3 ro = c.inside ? ld3(p.ray_o + 3 * c.pix) : mk3(0.f, 0.f, 0.f);
    float rt = 0.f;
    if constexpr (DYN) rt = (c.inside && p.rtd) ? p.rtd[c.pix] : 0.0f;

    {
        const bool in1[1] = {c.inside};
        const f3 ro1[1] = {ro}, rd1[1] = {rd};
        const float rt1[1] = {rt};
        const RayBundle bun = wave_bundle<1>(in1, ro1, rd1, rt1);
        if (lane == 0) s_bundle[wave] = bun;
    }
    // shared ray origin across the tile (thread 0's pixel is always inside the image)
    if (c.tr == 0) { s_origin[0] = ro.x; s_origin[1] = ro.y; s_origin[2] = ro.z; }
    __syncthreads();
    const f3 o0 = mk3(s_origin[0], s_origin[1], s_origin[2]);
    const bool same = !c.inside || (__float_as_uint(ro.x) == __float_as_uint(o0.x) &&
                                    __float_as_uint(ro.y) == __float_as_uint(o0.y) &&
                                    __float_as_uint(ro.z) == __float_as_uint(o0.z));
    const bool fixed = !DYN && __syncthreads_and(same);
    constexpr bool counting = COUNT;  // the pair counters (a variant of its own: their scalar work per pair)

    float depth = 0.0f, T = 1.0f;
    uint32_t cur_idx = 0;
    uint64_t n_eval = 0, n_contrib = 0;  // wave totals (uniform) when counting
    float pix[CS];
#pragma unroll
    for (int k = 0; k < CS; ++k) pix[k] = 0.f;

    const int32_t n_range = c.range_end - c.range_start;
    const int num_batches = n_range > 0 ? (n_range + bs - 1) / bs : 0;
    // the flatten id a thread stages in the next batch, loaded one batch ahead (its latency then
    // overlaps the pair loop instead of preceding the Gaussian's own loads)
    int32_t fid_next = 0;
    {
        const uint32_t idx0 = (uint32_t)c.range_start + (uint32_t)c.tr;
        if (num_batches > 0 && c.tr < bs && idx0 < (uint32_t)c.range_end) fid_next = p.flatten[idx0];
    }
    for (int b = 0; b < num_batches; ++b) {
        if (__syncthreads_count(done) >= (int)blockDim.x) break;
        const uint32_t batch_start = (uint32_t)c.range_start + (uint32_t)(bs * b);
        const uint32_t idx = batch_start + c.tr;
        bool staged = false;
        CullGauss cg;
        const int32_t fid_cur = fid_next;
        if (c.tr < bs && idx + (uint32_t)bs < (uint32_t)c.range_end) fid_next = p.flatten[idx + bs];
        if (c.tr < bs && idx < (uint32_t)c.range_end) {
            staged = true;
            const int32_t fid = fid_cur;
            const int64_t gid = fid - (int64_t)c.cam * g.n;
            const f3 mu = ld3(p.means + 3 * gid);
            const float op = p.opac[gid];
            const float4 q = p.quats[gid];
            const f3 sc = ld3(p.scales + 3 * gid);
            f3 r0, r1, r2;
            iscl_rot_rows(q, sc, r0, r1, r2);
            const f3 fourth = fixed ? rows_mul(r0, r1, r2, o0 - mu) : mu;
            s_m0[c.tr] = make_float4(r0.x, r0.y, r0.z, fourth.x);
            s_m1[c.tr] = make_float4(r1.x, r1.y, r1.z, fourth.y);
            s_m2[c.tr] = make_float4(r2.x, r2.y, r2.z, fourth.z);
            if constexpr (!OP_IN_COL) s_op[c.tr] = op;
            f3 vel = mk3(0.f, 0.f, 0.f);
            if constexpr (DYN) {
                if (p.velocity) vel = ld3(p.velocity + 3 * gid);
                s_vel[c.tr] = make_float4(vel.x, vel.y, vel.z, 0.f);
            }
            if constexpr (CL > 0) {
                const float* cp = p.colors + ((int64_t)fid * CDIM - (int64_t)c.cam * p.col_shift);
#pragma unroll
                for (int k4 = 0; k4 < C4; ++k4) {
                    float v[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        v[j] = (4 * k4 + j < CL) ? cp[4 * k4 + j] : (OP_IN_COL && 4 * k4 + j == CL) ? op : 0.f;
                    s_col[k4][c.tr] = make_float4(v[0], v[1], v[2], v[3]);
                }
            } else {
                s_id[c.tr] = fid;
            }
            cg = cull_gauss(mu, r0, r1, r2, sc, q, op, vel);
        }
        // which wavefronts evaluate this Gaussian: one ballot per wavefront
        for (int k = 0; k < nw; ++k) {
            const bool keep = staged && cull_keep<DYN>(s_bundle[k], cg);
            const uint64_t m = __ballot(keep);
            if (lane == 0) s_mask[k][wave] = m;
        }
        __syncthreads();

        // Branch-free per pair: a finished lane keeps evaluating with its results selected away,
        // and the wave leaves the batch once all its lanes are finished (`alive`, uniform). The
        // loop is instantiated for both origin modes so that neither branches per pair.
        uint64_t alive = __ballot(!done);
        auto pairs = [&](auto fixed_c) {
            constexpr bool FIXED = decltype(fixed_c)::value;
            for (int w2 = 0; w2 < nw && alive != 0; ++w2) {
                uint64_t m = uniform_u64(s_mask[wave][w2]);
                for (; m != 0 && alive != 0; m &= m - 1) {
                    const int t = (w2 << 6) + (int)__builtin_ctzll(m);
                    const float4 a = s_m0[t], bq = s_m1[t], cq = s_m2[t];
                    const f3 r0 = mk3(a.x, a.y, a.z), r1 = mk3(bq.x, bq.y, bq.z), r2 = mk3(cq.x, cq.y, cq.z);
                    float4 cl[C4 > 0 ? C4 : 1];
#pragma unroll
                    for (int k4 = 0; k4 < C4; ++k4) cl[k4] = s_col[k4][t];
                    float op;
                    if constexpr (OP_IN_COL) {
                        const float4 last = cl[C4 - 1];
                        op = (CL & 3) == 1 ? last.y : (CL & 3) == 2 ? last.z : last.w;
                    } else {
                        op = s_op[t];
                    }
                    f3 gro;
                    if constexpr (FIXED) {
                        gro = mk3(a.w, bq.w, cq.w);
                    } else {
                        f3 mu = mk3(a.w, bq.w, cq.w);
                        if constexpr (DYN) mu = mu + rt * mk3(s_vel[t].x, s_vel[t].y, s_vel[t].z);
                        gro = rows_mul(r0, r1, r2, ro - mu);
                    }
                    const f3 grd = rows_mul(r0, r1, r2, rd);
                    // 1/|grd|^2, capped so that grd = 0 gives power 0 as safe_normalize does
                    const float inv_dd = fminf(__builtin_amdgcn_rcpf(dot(grd, grd)), 3.40282347e38f);
                    // |n x gro|^2 = |grd x gro|^2 / |grd|^2; exp(-x/2) = exp2(x * -log2(e)/2)
                    const f3 cr = cross(grd, gro);
                    const float e = __builtin_amdgcn_exp2f(dot(cr, cr) * (inv_dd * -0.72134752f));
                    const float alpha = fminf(0.999f, op * e);
                    const float next_T = T * (1.0f - alpha);
                    // lane masks of this pair; termination is exclusive (eval3d_fwd.cu:135-139)
                    const uint64_t pass_m = __ballot(alpha >= 1.f / 255.f) & alive;
                    const uint64_t low_m = __ballot(next_T <= 1e-4f);
                    const bool take = __builtin_amdgcn_inverse_ballot_w64(pass_m & ~low_m);
                    const float hit_t = -dot(gro, grd) * inv_dd;
                    const float vis = take ? alpha * T : 0.0f;
                    depth += vis * hit_t;
                    if constexpr (CDIM > 0) {
                        if constexpr (CL > 0) {
#pragma unroll
                            for (int k4 = 0; k4 < C4; ++k4) {
                                const float4 cv = cl[k4];
                                const float cc[4] = {cv.x, cv.y, cv.z, cv.w};
#pragma unroll
                                for (int j = 0; j < 4; ++j)
                                    if (4 * k4 + j < CDIM) pix[4 * k4 + j] += cc[j] * vis;
                            }
                        } else {
                            const float* cp = p.colors + ((int64_t)s_id[t] * CDIM - (int64_t)c.cam * p.col_shift);
#pragma unroll
                            for (int k = 0; k < CDIM; ++k) pix[k] += cp[k] * vis;
                        }
                    }
                    cur_idx = take ? batch_start + t : cur_idx;
                    T = take ? next_T : T;
                    if (counting) {  // wave totals, scalar
                        n_eval += (uint64_t)__popcll(alive);
                        n_contrib += (uint64_t)__popcll(pass_m & ~low_m);
                    }
                    alive &= ~(pass_m & low_m);
                }
            }
        };
        if (fixed) pairs(std::true_type{});
        else pairs(std::false_type{});
        done = !__builtin_amdgcn_inverse_ballot_w64(alive);
    }
    if (counting && lane == 0) {  // one atomic per wave and counter
        atomicAdd(p.pair_counts, (unsigned long long)n_eval);
        atomicAdd(p.pair_counts + 1, (unsigned long long)n_contrib);
    }
    if (c.inside) {
        p.out_alpha[c.pix] = 1.0f - T;
        p.out_depth[c.pix] = depth;
#pragma unroll
        for (int k = 0; k < CDIM; ++k) p.out_rgb[c.pix * CDIM + k] = pix[k];
        p.out_last[c.pix] = (int32_t)cur_idx;
    }
    if (p.tile_work) {  // the tile's backward work: its intersections up to the largest last id
        __shared__ int s_last[NW];
        int m = c.inside ? (int)cur_idx : -1;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) m = max(m, __shfl_xor(m, off, 64));
        if (lane == 0) s_last[wave] = m;
        __syncthreads();
        if (c.tr == 0) {
            for (int k = 1; k < nw; ++k) m = max(m, s_last[k]);
            p.tile_work[c.cam * g.n_tiles_w * g.n_tiles_h + c.tile] = max(0, min(c.range_end - 1, m) - c.range_start + 1);
        }
    }
}

template <int CDIM>
int launch_cdim(bool dyn, const Eval3dParams& p, hipStream_t s) {
    const int n_blocks = p.g.n_tiles_w * p.g.n_tiles_h * p.g.n_cams;
    const int tile_px = p.g.tile_w * p.g.tile_h;
    const int nt = (tile_px + 63) / 64 * 64;  // whole wavefronts
    auto go = [&](auto count_c) {
        constexpr bool C = decltype(count_c)::value;
        if (tile_px <= kTileThreads) {
            if (dyn) eval3d_fwd_kernel<CDIM, true, kTileThreads, C><<<n_blocks, nt, 0, s>>>(p);
            else eval3d_fwd_kernel<CDIM, false, kTileThreads, C><<<n_blocks, nt, 0, s>>>(p);
        } else {
            if (dyn) eval3d_fwd_kernel<CDIM, true, kMaxTilePixels, C><<<n_blocks, nt, 0, s>>>(p);
            else eval3d_fwd_kernel<CDIM, false, kMaxTilePixels, C><<<n_blocks, nt, 0, s>>>(p);
        }
    };
    if (p.pair_counts) go(std::true_type{});
    else go(std::false_type{});
    return XSG_OK;
}

}  // namespace

int eval3d_fwd_launch(int cdim, bool dyn, const Eval3dParams& p, hipStream_t s) {
    switch (cdim) {
#define XSG_CASE(C) case C: return launch_cdim<C>(dyn, p, s);
        XSG_CDIM_LIST(XSG_CASE)
#undef XSG_CASE
        default: return xsg_fail(XSG_ERR_INVALID, "Unsupported number of channels: %d", cdim);
    }
}

}  // namespace xsg
