// Backward eval3d compositing: rasterize_eval3d_[dynamic_]bwd_kernel (eval3d_bwd.cu:66-294,
// eval3d_dynamic_bwd.cu kernel before :312).
//
// Differences in structure (not in what is computed):
//  * batches start at the largest last_id of the tile instead of the end of the tile's list; the
//    reference loads and skips those trailing batches (every index there exceeds every pixel's
//    last_id, eval3d_bwd.cu:155-159);
//  * dL/dM (M = S^-1 R^T) is accumulated per Gaussian and turned into quaternion / scale gradients
//    once per Gaussian by eval3d_bwd_epilogue: quat_scale_to_preci_half_vjp (utils.h:232-263) is
//    linear in dL/dM, so the sum of per-pair vjps equals the vjp of the sum;
//  * per-pair gradients are summed over the 64 lanes of a wavefront by a reduce-scatter that
//    leaves each component's total on its own lane, and one atomic instruction per 16
//    components adds them (one lane per component);
//  * divisions in the per-pair math are reciprocal-multiplies (v_rcp_f32, 1 ulp) and 1/|grd|^2 is
//    the square of the normalisation's reciprocal square root;
//  * with a shared ray origin, the staged Gaussian carries o - mu instead of mu.
#include "xsg_eval3d.h"

namespace xsg {
namespace {

constexpr float kMaxAlpha = 0.99f;  // eval3d_bwd.cu:38

XSG_DEV int wave_max(int v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
    return v;
}

template <int CDIM, bool DYN, bool RG>
__global__ __launch_bounds__(kTileThreads) void eval3d_bwd_kernel(Eval3dParams p) {
    constexpr int CL = (CDIM > 0 && CDIM <= kColorLdsMax) ? CDIM : 0;
    constexpr int CS = CDIM > 0 ? CDIM : 1;
    constexpr int K = CDIM + 3 + 9 + 1 + (DYN ? 3 : 0);  // colours, mean, M, opacity, velocity
    __shared__ int32_t s_id[kTileThreads];
    __shared__ float4 s_m0[kTileThreads], s_m1[kTileThreads], s_m2[kTileThreads];  // M rows | M (o - mu)
    __shared__ float4 s_xo[kTileThreads];  // o - mu (fixed origin) or mu, and opacity
    __shared__ float4 s_vel[DYN ? kTileThreads : 1];
    __shared__ float s_col[CL > 0 ? kTileThreads * CL : 1];
    __shared__ float s_origin[3];
    __shared__ int s_max;

    const TileGrid& g = p.g;
    const PixelCtx c = pixel_ctx(g, p.offsets);
    const int bs = g.tile_w * g.tile_h;
    const int lane = __lane_id();
    const f3 rd = c.inside ? ld3(p.ray_d + 3 * c.pix) : mk3(0.f, 0.f, 0.f);
    const f3 ro = c.inside ? ld3(p.ray_o + 3 * c.pix) : mk3(0.f, 0.f, 0.f);
    float rt = 0.f;
    if constexpr (DYN) rt = c.inside ? p.rtd[c.pix] : 0.0f;

    if (c.tr == 0) { s_origin[0] = ro.x; s_origin[1] = ro.y; s_origin[2] = ro.z; s_max = -1; }
    __syncthreads();
    const f3 o0 = mk3(s_origin[0], s_origin[1], s_origin[2]);
    const bool same = !c.inside || (__float_as_uint(ro.x) == __float_as_uint(o0.x) &&
                                    __float_as_uint(ro.y) == __float_as_uint(o0.y) &&
                                    __float_as_uint(ro.z) == __float_as_uint(o0.z));
    const bool fixed = !DYN && __syncthreads_and(same);

    const float T_final = 1.0f - p.render_alpha[c.pix];
    float T = T_final;
    float buffer[CS];
    float v_c[CS];
#pragma unroll
    for (int k = 0; k < CS; ++k) { buffer[k] = 0.f; v_c[k] = 0.f; }
#pragma unroll
    for (int k = 0; k < CDIM; ++k) v_c[k] = c.inside ? p.v_rgb[c.pix * CDIM + k] : 0.0f;
    const float v_d = c.inside ? p.v_depth[c.pix] : 0.0f;
    const float v_a = c.inside ? p.v_alpha[c.pix] : 0.0f;
    const int32_t bin_final = c.inside ? p.last_ids[c.pix] : 0;
    const int32_t wave_bin_final = wave_max(bin_final);
    if (lane == 0) atomicMax(&s_max, wave_bin_final);
    f3 v_ro = mk3(0.f, 0.f, 0.f), v_rd = mk3(0.f, 0.f, 0.f);
    float depth_buffer = 0.0f, v_t = 0.0f;
    // The lane that adds component k of a chunk (k = lane / 4, lanes 4k) writes to
    // dst_base[chunk] + gid * dst_stride[chunk]; both are fixed per lane.
    constexpr int kChunks = (K + 15) / 16;
    float* dst_base[kChunks];
    int dst_stride[kChunks];
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
        const int kk = 16 * ch + (lane >> 2);
        if (kk < CDIM) {  // colours are [n_cams, n, CDIM]: flatten id = cam * n + gid
            dst_base[ch] = p.v_colors + ((int64_t)c.cam * g.n) * CDIM + kk;
            dst_stride[ch] = CDIM;
        } else if (kk < CDIM + 3) {
            dst_base[ch] = p.v_means + (kk - CDIM); dst_stride[ch] = 3;
        } else if (kk < CDIM + 12) {
            dst_base[ch] = p.v_mt + (kk - CDIM - 3); dst_stride[ch] = 9;
        } else if (kk == CDIM + 12) {
            dst_base[ch] = p.v_opac; dst_stride[ch] = 1;
        } else if (kk < K) {
            dst_base[ch] = p.v_velocity + (kk - CDIM - 13); dst_stride[ch] = 3;
        } else {
            dst_base[ch] = nullptr; dst_stride[ch] = 0;
        }
    }
    __syncthreads();
    const int32_t eff_end = min(c.range_end - 1, s_max);
    const int32_t n_eff = eff_end - c.range_start + 1;
    const int num_batches = n_eff > 0 ? (n_eff + bs - 1) / bs : 0;

    for (int b = 0; b < num_batches; ++b) {
        __syncthreads();
        const int32_t batch_end = eff_end - bs * b;
        const int32_t batch_size = min(bs, batch_end + 1 - c.range_start);
        const int32_t idx = batch_end - c.tr;
        if (idx >= c.range_start) {
            const int32_t fid = p.flatten[idx];
            const int64_t gid = fid - (int64_t)c.cam * g.n;
            s_id[c.tr] = fid;
            const f3 mu = ld3(p.means + 3 * gid);
            f3 r0, r1, r2;
            iscl_rot_rows(p.quats[gid], ld3(p.scales + 3 * gid), r0, r1, r2);
            f3 gro = mk3(0.f, 0.f, 0.f), xo = mu;
            if (fixed) {
                xo = o0 - mu;
                gro = rows_mul(r0, r1, r2, xo);
            }
            s_m0[c.tr] = make_float4(r0.x, r0.y, r0.z, gro.x);
            s_m1[c.tr] = make_float4(r1.x, r1.y, r1.z, gro.y);
            s_m2[c.tr] = make_float4(r2.x, r2.y, r2.z, gro.z);
            s_xo[c.tr] = make_float4(xo.x, xo.y, xo.z, p.opac[gid]);
            if constexpr (DYN) {
                const f3 v = ld3(p.velocity + 3 * gid);
                s_vel[c.tr] = make_float4(v.x, v.y, v.z, 0.f);
            }
            if constexpr (CL > 0) {
#pragma unroll
                for (int k = 0; k < CL; ++k) s_col[c.tr * CL + k] = p.colors[(int64_t)fid * CDIM + k];
            }
        }
        __syncthreads();
        for (int t = max(0, batch_end - wave_bin_final); t < batch_size; ++t) {
            const float4 a = s_m0[t], bq = s_m1[t], cq = s_m2[t];
            const f3 r0 = mk3(a.x, a.y, a.z), r1 = mk3(bq.x, bq.y, bq.z), r2 = mk3(cq.x, cq.y, cq.z);
            const float4 xo = s_xo[t];
            const float op = xo.w;
            f3 vel = mk3(0.f, 0.f, 0.f);
            f3 omm, gro;  // o - mu and M (o - mu)
            if (fixed) {
                omm = mk3(xo.x, xo.y, xo.z);
                gro = mk3(a.w, bq.w, cq.w);
            } else {
                f3 mu = mk3(xo.x, xo.y, xo.z);
                if constexpr (DYN) {
                    vel = mk3(s_vel[t].x, s_vel[t].y, s_vel[t].z);
                    mu = mu + rt * vel;
                }
                omm = ro - mu;
                gro = rows_mul(r0, r1, r2, omm);
            }
            const f3 grd = rows_mul(r0, r1, r2, rd);
            const float dd = dot(grd, grd);
            const float il = inv_len(dd);
            const f3 grd_n = grd * il;
            const f3 gcrod = cross(grd_n, gro);
            const float power = -0.5f * dot(gcrod, gcrod);
            const float vis = __expf(power);
            const float alpha = fminf(kMaxAlpha, op * vis);
            const bool valid = c.inside && (batch_end - t <= bin_final) && alpha >= 1.f / 255.f;
            if (__ballot(valid) == 0) continue;  // wave-uniform (eval3d_bwd.cu:209-212)

            // Every lane runs the same instructions; a lane whose pair is not valid contributes
            // exact zeros (its fac and gated upstream gradients are selected to 0, and every
            // gradient below is linear in them) and keeps its transmittance and buffers.
            const float inv_dd = il * il;
            const float od = dot(gro, grd);
            const float last_hit_T = -od * inv_dd;
            const float ra = __builtin_amdgcn_rcpf(fmaxf(1e-6f, 1.0f - alpha));
            T = valid ? T * ra : T;
            const float fac = valid ? alpha * T : 0.0f;
            float rgb[CS];
#pragma unroll
            for (int k = 0; k < CS; ++k) rgb[k] = 0.f;
            if constexpr (CDIM > 0) {
                if constexpr (CL > 0) {
#pragma unroll
                    for (int k = 0; k < CDIM; ++k) rgb[k] = s_col[t * CL + k];
                } else {
                    const float* cp = p.colors + (int64_t)s_id[t] * CDIM;
#pragma unroll
                    for (int k = 0; k < CDIM; ++k) rgb[k] = cp[k];
                }
            }
            float acc[K];
            // grad_alpha (eval3d_bwd.cu:42-63)
            float v_alpha = 0.0f;
#pragma unroll
            for (int k = 0; k < CDIM; ++k) {
                acc[k] = v_c[k] * fac;
                v_alpha += (rgb[k] * T - buffer[k] * ra) * v_c[k];
            }
            v_alpha += (last_hit_T * T - depth_buffer * ra) * v_d;
            v_alpha += T_final * ra * v_a;
            // geometry and opacity only below the clamp (eval3d_bwd.cu:243)
            const bool geo = valid && op * vis <= kMaxAlpha;
            const float v_alpha_g = geo ? v_alpha : 0.0f;
            const float dL_dhitT = geo ? v_d * fac : 0.0f;

            f3 v_gro = grd * (-dL_dhitT * inv_dd);
            f3 v_grd = (2.0f * od * grd - dd * gro) * (dL_dhitT * inv_dd * inv_dd);
            const float v_gd = -0.5f * vis * (op * v_alpha_g);
            const f3 v_gcrod = (2.0f * v_gd) * gcrod;
            const f3 v_grd_n = -cross(v_gcrod, gro);
            v_gro = v_gro + cross(v_gcrod, grd_n);
            v_grd = v_grd + safe_normalize_bwd_il(grd, il, v_grd_n);
            const f3 v_omm = rows_tmul(r0, r1, r2, v_gro);
            acc[CDIM + 0] = -v_omm.x;
            acc[CDIM + 1] = -v_omm.y;
            acc[CDIM + 2] = -v_omm.z;
            // dL/dM^T (math rows): v_grd (x) ray_d + v_gro (x) (o - mu)
            acc[CDIM + 3] = v_grd.x * rd.x + v_gro.x * omm.x;
            acc[CDIM + 4] = v_grd.x * rd.y + v_gro.x * omm.y;
            acc[CDIM + 5] = v_grd.x * rd.z + v_gro.x * omm.z;
            acc[CDIM + 6] = v_grd.y * rd.x + v_gro.y * omm.x;
            acc[CDIM + 7] = v_grd.y * rd.y + v_gro.y * omm.y;
            acc[CDIM + 8] = v_grd.y * rd.z + v_gro.y * omm.z;
            acc[CDIM + 9] = v_grd.z * rd.x + v_gro.z * omm.x;
            acc[CDIM + 10] = v_grd.z * rd.y + v_gro.z * omm.y;
            acc[CDIM + 11] = v_grd.z * rd.z + v_gro.z * omm.z;
            acc[CDIM + 12] = vis * v_alpha_g;
            if constexpr (DYN) {
                acc[CDIM + 13] = -v_omm.x * rt;
                acc[CDIM + 14] = -v_omm.y * rt;
                acc[CDIM + 15] = -v_omm.z * rt;
                v_t += -dot(v_omm, vel);
            }
            if constexpr (RG) {
                v_ro = v_ro + v_omm;
                v_rd = v_rd + rows_tmul(r0, r1, r2, v_grd);
            }
#pragma unroll
            for (int k = 0; k < CDIM; ++k) buffer[k] += rgb[k] * fac;
            depth_buffer += fac * last_hit_T;

            // wave totals by reduce-scatter: lane l ends with component 16 * chunk + (l >> 2); the
            // first lane of each quad adds it, one atomic instruction per chunk of 16 components
            const int64_t gid = s_id[t] - (int64_t)c.cam * g.n;
#pragma unroll
            for (int ch = 0; ch < kChunks; ++ch) {
                float chunk[16];
#pragma unroll
                for (int k = 0; k < 16; ++k) chunk[k] = (16 * ch + k < K) ? acc[16 * ch + k] : 0.f;
                const float tot = wave_reduce_scatter16(chunk);
                if ((lane & 3) == 0 && 16 * ch + (lane >> 2) < K)
                    unsafeAtomicAdd(dst_base[ch] + gid * dst_stride[ch], tot);
            }
        }
    }
    if (c.inside) {
        if constexpr (RG) {
            st3(p.v_ray_o + 3 * c.pix, v_ro);
            st3(p.v_ray_d + 3 * c.pix, v_rd);
        }
        if constexpr (DYN) p.v_time[c.pix] = v_t;
    }
}

// Variants without per-pixel ray gradients exist for CDIM <= kColorLdsMax; larger CDIMs always
// compute them (the C-ABI then needs the ray-gradient buffers).
template <int CDIM>
int launch_cdim(bool dyn, bool ray_grads, const Eval3dParams& p, hipStream_t s) {
    const int n_blocks = p.g.n_tiles_w * p.g.n_tiles_h * p.g.n_cams;
    const int bs = p.g.tile_w * p.g.tile_h;
    if constexpr (CDIM <= kColorLdsMax) {
        if (!ray_grads) {
            if (dyn) eval3d_bwd_kernel<CDIM, true, false><<<n_blocks, bs, 0, s>>>(p);
            else eval3d_bwd_kernel<CDIM, false, false><<<n_blocks, bs, 0, s>>>(p);
            return XSG_OK;
        }
    }
    if (!p.v_ray_o || !p.v_ray_d) return xsg_fail(XSG_ERR_INVALID, "ray gradient buffers are required for cdim %d", CDIM);
    if (dyn) eval3d_bwd_kernel<CDIM, true, true><<<n_blocks, bs, 0, s>>>(p);
    else eval3d_bwd_kernel<CDIM, false, true><<<n_blocks, bs, 0, s>>>(p);
    return XSG_OK;
}

}  // namespace

int eval3d_bwd_launch(int cdim, bool dyn, const Eval3dParams& p, hipStream_t s) {
    const bool ray_grads = p.v_ray_o != nullptr;
    switch (cdim) {
#define XSG_CASE(C) case C: return launch_cdim<C>(dyn, ray_grads, p, s);
        XSG_CDIM_LIST(XSG_CASE)
#undef XSG_CASE
        default: return xsg_fail(XSG_ERR_INVALID, "unsupported feature dimension: %d", cdim);
    }
}

}  // namespace xsg
