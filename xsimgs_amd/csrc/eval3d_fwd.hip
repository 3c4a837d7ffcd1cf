// Forward eval3d compositing: rasterize_eval3d_[dynamic_]fwd_kernel (eval3d_fwd.cu:34-166,
// eval3d_dynamic_fwd.cu:37-173).
#include "xsg_eval3d.h"

namespace xsg {
namespace {

template <int CDIM, bool DYN>
__global__ __launch_bounds__(kTileThreads) void eval3d_fwd_kernel(Eval3dParams p) {
    constexpr int CL = (CDIM > 0 && CDIM <= kColorLdsMax) ? CDIM : 0;  // channels staged in LDS
    constexpr int CS = CDIM > 0 ? CDIM : 1;
    __shared__ int32_t s_id[kTileThreads];
    __shared__ float4 s_m0[kTileThreads], s_m1[kTileThreads], s_m2[kTileThreads];  // M rows | gro
    __shared__ float4 s_xo[kTileThreads];                                            // mean | opacity
    __shared__ float4 s_vel[DYN ? kTileThreads : 1];
    __shared__ float s_col[CL > 0 ? kTileThreads * CL : 1];
    __shared__ float s_origin[3];

    const TileGrid& g = p.g;
    const PixelCtx c = pixel_ctx(g, p.offsets);
    const int bs = g.tile_w * g.tile_h;
    bool done = !c.inside;
    const f3 rd = c.inside ? ld3(p.ray_d + 3 * c.pix) : mk3(0.f, 0.f, 0.f);
    const f3 ro = c.inside ? ld3(p.ray_o + 3 * c.pix) : mk3(0.f, 0.f, 0.f);
    float rt = 0.f;
    if constexpr (DYN) rt = (c.inside && p.rtd) ? p.rtd[c.pix] : 0.0f;

    // shared ray origin across the tile (thread 0's pixel is always inside the image)
    if (c.tr == 0) { s_origin[0] = ro.x; s_origin[1] = ro.y; s_origin[2] = ro.z; }
    __syncthreads();
    const f3 o0 = mk3(s_origin[0], s_origin[1], s_origin[2]);
    const bool same = !c.inside || (__float_as_uint(ro.x) == __float_as_uint(o0.x) &&
                                    __float_as_uint(ro.y) == __float_as_uint(o0.y) &&
                                    __float_as_uint(ro.z) == __float_as_uint(o0.z));
    const bool fixed = !DYN && __syncthreads_and(same);

    float depth = 0.0f, T = 1.0f;
    uint32_t cur_idx = 0;
    uint32_t n_eval = 0, n_contrib = 0;
    float pix[CS];
#pragma unroll
    for (int k = 0; k < CS; ++k) pix[k] = 0.f;

    const int32_t n_range = c.range_end - c.range_start;
    const int num_batches = n_range > 0 ? (n_range + bs - 1) / bs : 0;
    for (int b = 0; b < num_batches; ++b) {
        if (__syncthreads_count(done) >= bs) break;
        const uint32_t batch_start = (uint32_t)c.range_start + (uint32_t)(bs * b);
        const uint32_t idx = batch_start + c.tr;
        if (idx < (uint32_t)c.range_end) {
            const int32_t fid = p.flatten[idx];
            const int64_t gid = fid - (int64_t)c.cam * g.n;
            s_id[c.tr] = fid;
            const f3 mu = ld3(p.means + 3 * gid);
            const float op = p.opac[gid];
            f3 r0, r1, r2;
            iscl_rot_rows(p.quats[gid], ld3(p.scales + 3 * gid), r0, r1, r2);
            f3 gro = mk3(0.f, 0.f, 0.f);
            if (fixed) gro = rows_mul(r0, r1, r2, o0 - mu);
            s_m0[c.tr] = make_float4(r0.x, r0.y, r0.z, gro.x);
            s_m1[c.tr] = make_float4(r1.x, r1.y, r1.z, gro.y);
            s_m2[c.tr] = make_float4(r2.x, r2.y, r2.z, gro.z);
            s_xo[c.tr] = make_float4(mu.x, mu.y, mu.z, op);
            if constexpr (DYN) {
                const f3 v = p.velocity ? ld3(p.velocity + 3 * gid) : mk3(0.f, 0.f, 0.f);
                s_vel[c.tr] = make_float4(v.x, v.y, v.z, 0.f);
            }
            if constexpr (CL > 0) {
#pragma unroll
                for (int k = 0; k < CL; ++k) s_col[c.tr * CL + k] = p.colors[(int64_t)fid * CDIM + k];
            }
        }
        __syncthreads();
        const int batch_size = min(bs, c.range_end - (int32_t)batch_start);
        // Branch-free per pair: a finished lane keeps evaluating with its results selected away,
        // and the wave leaves the batch once all its lanes are finished.
        for (int t = 0; t < batch_size; ++t) {
            if (__ballot(!done) == 0) break;  // wave-uniform
            const float4 a = s_m0[t], bq = s_m1[t], cq = s_m2[t];
            const f3 r0 = mk3(a.x, a.y, a.z), r1 = mk3(bq.x, bq.y, bq.z), r2 = mk3(cq.x, cq.y, cq.z);
            const float op = s_xo[t].w;
            f3 gro;
            if (fixed) {
                gro = mk3(a.w, bq.w, cq.w);
            } else {
                f3 mu = mk3(s_xo[t].x, s_xo[t].y, s_xo[t].z);
                if constexpr (DYN) mu = mu + rt * mk3(s_vel[t].x, s_vel[t].y, s_vel[t].z);
                gro = rows_mul(r0, r1, r2, ro - mu);
            }
            const f3 grd = rows_mul(r0, r1, r2, rd);
            const float dd = dot(grd, grd);
            const float il = inv_len(dd);
            const f3 gcrod = cross(grd * il, gro);
            const float power = -0.5f * dot(gcrod, gcrod);
            const float alpha = fminf(0.999f, op * __expf(power));
            const bool live = !done;
            const bool pass = live && alpha >= 1.f / 255.f;
            const float next_T = T * (1.0f - alpha);
            const bool term = pass && next_T <= 1e-4f;  // exclusive termination (eval3d_fwd.cu:135-139)
            const bool take = pass && !term;
            done = done || term;
            const float hit_t = -dot(gro, grd) * (il * il);
            const float vis = take ? alpha * T : 0.0f;
            depth += vis * hit_t;
            if constexpr (CDIM > 0) {
                if constexpr (CL > 0) {
#pragma unroll
                    for (int k = 0; k < CDIM; ++k) pix[k] += s_col[t * CL + k] * vis;
                } else {
                    const float* cp = p.colors + (int64_t)s_id[t] * CDIM;
#pragma unroll
                    for (int k = 0; k < CDIM; ++k) pix[k] += cp[k] * vis;
                }
            }
            cur_idx = take ? batch_start + t : cur_idx;
            T = take ? next_T : T;
            n_eval += live ? 1u : 0u;
            n_contrib += take ? 1u : 0u;
        }
    }
    if (p.pair_counts) {  // one atomic per wave and counter
        unsigned long long e = n_eval, k = n_contrib;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            e += __shfl_xor(e, off, 64);
            k += __shfl_xor(k, off, 64);
        }
        if (__lane_id() == 0) {
            atomicAdd(p.pair_counts, e);
            atomicAdd(p.pair_counts + 1, k);
        }
    }
    if (c.inside) {
        p.out_alpha[c.pix] = 1.0f - T;
        p.out_depth[c.pix] = depth;
#pragma unroll
        for (int k = 0; k < CDIM; ++k) p.out_rgb[c.pix * CDIM + k] = pix[k];
        p.out_last[c.pix] = (int32_t)cur_idx;
    }
}

template <int CDIM>
int launch_cdim(bool dyn, const Eval3dParams& p, hipStream_t s) {
    const int n_blocks = p.g.n_tiles_w * p.g.n_tiles_h * p.g.n_cams;
    const int bs = p.g.tile_w * p.g.tile_h;
    if (dyn) eval3d_fwd_kernel<CDIM, true><<<n_blocks, bs, 0, s>>>(p);
    else eval3d_fwd_kernel<CDIM, false><<<n_blocks, bs, 0, s>>>(p);
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
