// Backward eval3d compositing: rasterize_eval3d_[dynamic_]bwd_kernel (eval3d_bwd.cu:66-294,
// eval3d_dynamic_bwd.cu kernel before :312).
//
// Differences in structure (not in what is computed):
//  * batches start at the largest last_id of the tile instead of the end of the tile's list; the
//    reference loads and skips those trailing batches (every index there exceeds every pixel's
//    last_id, eval3d_bwd.cu:155-159);
//  * the gradient of M = S^-1 R^T is accumulated per Gaussian, as the symmetric Q = sum of
//    v_grd (x) grd + v_gro (x) gro (dL/dM = Q S R^T, six entries), and turned into quaternion /
//    scale gradients once per Gaussian by the epilogue: quat_scale_to_preci_half_vjp
//    (utils.h:232-263) is linear in dL/dM, so the sum of per-pair vjps equals the vjp of the sum,
//    and the scale gradient is -Q_ii / s_i;
//  * per-pair gradients are summed over the 64 lanes of a wavefront by a reduce-scatter that
//    leaves each component's total on its own lane, and one atomic instruction per 16
//    components adds them (one lane per component);
//  * each thread owns two pixels (four in tiles of more than 128 pixels, which a single wavefront
//    then covers up to 256 pixels; tiles of up to 1024 pixels take up to four wavefronts), so the
//    staged Gaussian's LDS reads, the reduction and the atomics serve all of them;
//  * divisions in the per-pair math are reciprocal-multiplies (v_rcp_f32, 1 ulp);
//  * (wavefront, Gaussian) pairs that no pixel of the wavefront can take are skipped unevaluated
//    (cull_keep); they would add exact zeros.
//
// This header holds the kernel template and its per-CDIM launcher; eval3d_bwd_g*.hip instantiate the
// launcher for groups of colour dimensions in separate translation units (the variants compile in
// parallel) and eval3d_bwd.hip dispatches on the dimension.
#pragma once
#include <type_traits>

#include "xsg_eval3d.h"

namespace xsg {
namespace {

constexpr float kMaxAlpha = 0.99f;  // eval3d_bwd.cu:38

XSG_DEV int wave_max(int v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
    return v;
}

// Reduce-scatter of the first nv (<= 16) of 16 per-lane values over the 64 lanes of a wavefront through a
// wavefront-private LDS buffer: lane l stores value k at row k (rows of kRedRow floats, padded so that
// the four lanes reading one quarter-row each fall in different banks), then lane 4k + q adds lanes
// 16q .. 16q + 15 of row k with four 16-byte reads and the quad adds its four sums (DPP). Every lane of
// quad k ends with the wave total of value k. LDS instructions of one wavefront complete in order, so
// the reads see the stores and the next call's stores follow these reads. All 64 lanes active.
constexpr int kRedRow = 68;
XSG_DEV float wave_reduce_scatter16_lds(const float (&v)[16], int nv, float* __restrict__ buf) {
    const int lane = __lane_id();
#pragma unroll
    for (int k = 0; k < 16; ++k)
        if (k < nv) buf[k * kRedRow + lane] = v[k];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int k = lane >> 2, q = lane & 3;
    float s = 0.0f;
    if (k < nv) {
        const float4* row = reinterpret_cast<const float4*>(buf + k * kRedRow + 16 * q);
        const float4 a = row[0], b = row[1], c = row[2], d = row[3];
        s = (((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w))) +
            (((c.x + c.y) + (c.z + c.w)) + ((d.x + d.y) + (d.z + d.w)));
    }
    s += dpp_mov<kDppQuadSwap2>(s);
    s += dpp_mov<kDppQuadSwap1>(s);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    return s;
}

// Per-pixel state of the backward sweep. The ray origin is not kept: the tiles whose rays share one
// origin never read it per pair, the others reload it (keeping it live would cost the registers
// that decide the kernel's occupancy).
template <int CS>
struct BwdPixel {
    f3 rd;
    float rt;
    float T, v_t;
    float buf;  // sum over composited pairs of fac (rgb . v_rgb + hit_t v_depth), minus T_final v_alpha
    float v_c[CS];
    float v_d;
    int32_t bin_final;
    bool inside;
    f3 v_ro, v_rd;
};

// The staged Gaussian of one loop step.
struct BwdGauss {
    f3 r0, r1, r2;   // rows of M
    f3 mu;
    f3 gro_fixed;    // M (o - mu) (shared origin)
    f3 vel;
    float op;
};

// alpha evaluation of one (pixel, Gaussian) pair (eval3d_bwd.cu:172-205) in the forward kernel's
// arithmetic: |n x gro|^2 = |grd x gro|^2 / |grd|^2, so that the transmittance this sweep divides
// out is the one the forward pass multiplied in.
struct BwdEval {
    f3 gro, grd, c;                  // c = grd x gro
    float inv_dd, vis, araw, alpha;  // araw = op * vis, before the clamp
    bool valid;
};

template <bool DYN, bool FIXED>
XSG_DEV BwdEval bwd_eval(const BwdGauss& gs, const f3 ro, const f3 rd, float rt, bool in_range) {
    BwdEval e;
    if constexpr (FIXED) {
        e.gro = gs.gro_fixed;
    } else {
        f3 mu = gs.mu;
        if constexpr (DYN) mu = mu + rt * gs.vel;
        e.gro = rows_mul(gs.r0, gs.r1, gs.r2, ro - mu);
    }
    e.grd = rows_mul(gs.r0, gs.r1, gs.r2, rd);
    e.inv_dd = fminf(__builtin_amdgcn_rcpf(dot(e.grd, e.grd)), 3.40282347e38f);
    e.c = cross(e.grd, e.gro);
    e.vis = __builtin_amdgcn_exp2f(dot(e.c, e.c) * (e.inv_dd * -0.72134752f));
    e.araw = gs.op * e.vis;
    e.alpha = fminf(kMaxAlpha, e.araw);
    e.valid = in_range && e.alpha >= 1.f / 255.f;
    e.alpha = e.valid ? e.alpha : 0.0f;  // an invalid pair then leaves T (1 / (1 - 0) is exact) and fac at 0
    return e;
}

// acc[k] = v for the lane's first pixel, += v for the second (no addition to a zero start)
template <bool FIRST>
XSG_DEV void put(float& a, float v) {
    if constexpr (FIRST) a = v;
    else a += v;
}

// acc = x y - z w for the first pixel; acc += x y, then acc -= z w (two FMAs) for the others
template <bool FIRST>
XSG_DEV void put_diff(float& a, float x, float y, float z, float w) {
    if constexpr (FIRST) {
        a = fmaf(x, y, -(z * w));
    } else {
        a = fmaf(x, y, a);
        a = fmaf(-z, w, a);
    }
}

// Gradient contribution of one pair into acc (eval3d_bwd.cu:206-271). A pair that is not valid
// adds exact zeros (its alpha is 0, so fac = 0 and T / (1 - 0) = T; its gated upstream gradients
// are selected to 0, and every gradient is linear in them) and leaves the pixel's transmittance
// and buffer unchanged.
//
// The reference's dL/dalpha sums, per channel, rgb T - buffer / (1 - alpha) and the depth and
// alpha terms; here one running buffer carries all of them, so dL/dalpha = T u - buf / (1 - alpha)
// with u = rgb . v_rgb + hit_t v_depth. Its chain through gcrod = n x gro, n = grd / |grd|, and
// safe_normalize_bwd collapses to one vector w = (grd x gro) x grd (= |grd|^2 (gcrod x n)):
// with A = -op vis dL/dalpha / |grd|^2 it adds A w to dL/dgro and -A (grd . gro) / |grd|^2 w to
// dL/dgrd. The hit-distance terms are k1 = dL/dhit_t / |grd|^2 times -grd (gro) and
// 2 (grd . gro) / |grd|^2 grd - gro (grd). With hit_t = -(grd . gro) / |grd|^2 the whole of
// dL/dgrd is hit_t (dL/dgro - k1 grd) - k1 gro. Without per-pixel ray or time gradients the mean
// gradient -M^T dL/dgro is applied once to the sum over the lane's pixels (vg_sum).
//
// Q: with p = gro + hit_t grd = w / |grd|^2 (the Gaussian's offset from the ray, perpendicular to
// it, in the normalised frame), dL/dgrd = hit_t dL/dgro - k1 p and gro = p - hit_t grd, so the
// hit_t terms of Q = dL/dgrd (x) grd + dL/dgro (x) gro cancel exactly and
//   Q = dL/dgro (x) p - p (x) k1 grd = A |grd|^2 p (x) p - k1 (grd (x) p + p (x) grd),
// which is symmetric (the loss depends on M only through rotation invariants of gro and grd).
// Accumulating it in this form skips the two products of size |hit_t| |grd| that cancel (the
// far-from-the-Gaussian part of the ray), which in float32 lose the scale gradient of thin
// Gaussians seen from far away.
template <int CDIM, int CS, int K, bool DYN, bool RG, bool FIRST>
XSG_DEV void bwd_pair(BwdPixel<CS>& px, const BwdGauss& gs, const BwdEval& e, const float (&rgb)[CS],
                      float (&acc)[K], f3& vg_sum) {
    const float od = dot(e.gro, e.grd);
    const float hit_t = -od * e.inv_dd;
    // 1 / max(1e-6, 1 - alpha) (eval3d_bwd.cu:221): alpha <= kMaxAlpha, so the max never applies
    const float ra = __builtin_amdgcn_rcpf(1.0f - e.alpha);
    px.T = px.T * ra;
    const float T = px.T;
    const float fac = e.alpha * T;
    float rv = 0.0f;
#pragma unroll
    for (int k = 0; k < CDIM; ++k) {
        put<FIRST>(acc[k], px.v_c[k] * fac);
        rv = (k == 0) ? rgb[0] * px.v_c[0] : fmaf(rgb[k], px.v_c[k], rv);
    }
    const float u = (CDIM > 0) ? fmaf(hit_t, px.v_d, rv) : hit_t * px.v_d;
    const float v_alpha = T * u - ra * px.buf;
    // geometry and opacity only below the clamp (eval3d_bwd.cu:243)
    const bool geo = e.valid && e.araw <= kMaxAlpha;
    const float v_alpha_g = geo ? v_alpha : 0.0f;
    const float k1 = geo ? px.v_d * fac * e.inv_dd : 0.0f;
    // A w = -op vis dL/dalpha p with p = w / |grd|^2 (the offset of the Gaussian from the ray).
    // p = gro + hit_t grd in exact arithmetic; from the cross product its float32 error is smaller
    // (the direct sum moved per-pixel ray gradients of the golden fixtures beyond tolerance).
    const float Ap = -e.araw * v_alpha_g;
    const f3 pp = cross(e.c, e.grd) * e.inv_dd;
    const f3 kg = k1 * e.grd;
    const f3 v_gro = Ap * pp - kg;
    if constexpr (RG || DYN) {
        const f3 v_omm = rows_tmul(gs.r0, gs.r1, gs.r2, v_gro);
        put<FIRST>(acc[CDIM + 0], -v_omm.x);
        put<FIRST>(acc[CDIM + 1], -v_omm.y);
        put<FIRST>(acc[CDIM + 2], -v_omm.z);
        if constexpr (DYN) {
            put<FIRST>(acc[CDIM + 10], -v_omm.x * px.rt);
            put<FIRST>(acc[CDIM + 11], -v_omm.y * px.rt);
            put<FIRST>(acc[CDIM + 12], -v_omm.z * px.rt);
            px.v_t -= dot(v_omm, gs.vel);
        }
        if constexpr (RG) {
            const f3 v_grd = hit_t * (v_gro - kg) - k1 * e.gro;
            px.v_ro = px.v_ro + v_omm;
            px.v_rd = px.v_rd + rows_tmul(gs.r0, gs.r1, gs.r2, v_grd);
        }
    } else {
        vg_sum = FIRST ? v_gro : vg_sum + v_gro;
    }
    // Q (upper triangle, row-major): Q_ij = dL/dgro_i p_j - p_i k1 grd_j
    put<FIRST>(acc[CDIM + 3], pp.x * (v_gro.x - kg.x));
    put_diff<FIRST>(acc[CDIM + 4], v_gro.x, pp.y, pp.x, kg.y);
    put_diff<FIRST>(acc[CDIM + 5], v_gro.x, pp.z, pp.x, kg.z);
    put<FIRST>(acc[CDIM + 6], pp.y * (v_gro.y - kg.y));
    put_diff<FIRST>(acc[CDIM + 7], v_gro.y, pp.z, pp.y, kg.z);
    put<FIRST>(acc[CDIM + 8], pp.z * (v_gro.z - kg.z));
    put<FIRST>(acc[CDIM + 9], e.vis * v_alpha_g);
    px.buf = fmaf(fac, u, px.buf);
}

// Waves per SIMD the compiler is asked to fit: four for the one-wavefront tiles of up to three colour
// channels without per-pixel ray or time gradients (evaluating and compositing one pixel slot at a
// time, they need about 139 registers; at 128 the few that do not fit are set-up values spilled
// outside the pair loop), else whatever the registers allow.
template <int CDIM, bool DYN, bool RG, int PX, int NT>
constexpr int kBwdWaves = (NT == 64 && PX == 4 && !RG && !DYN && CDIM <= 3) ? 4 : 1;

// PX pixels per thread: a workgroup of ceil(tile / PX) threads (rounded up to whole wavefronts) per
// tile, thread tr owning the pixels PX tr ... PX tr + PX - 1 of the tile in row-major order. The
// staged Gaussian's LDS reads, the wavefront reduction and the atomic adds are shared by the
// thread's pixels.
template <int CDIM, bool DYN, bool RG, int PX, int NT, bool COUNT>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(kBwdWaves<CDIM, DYN, RG, PX, NT>))) void eval3d_bwd_kernel(Eval3dParams p) {
    // NT: threads (and staged Gaussians per batch) at most
    constexpr int CL = (CDIM > 0 && CDIM <= kColorLdsMax) ? CDIM : 0;
    constexpr int CS = CDIM > 0 ? CDIM : 1;
    constexpr int K = CDIM + 3 + 6 + 1 + (DYN ? 3 : 0);  // colours, mean, Q, opacity, velocity
    __shared__ int32_t s_id[NT];
    __shared__ float4 s_m0[NT], s_m1[NT], s_m2[NT];  // M rows | M (o - mu)
    __shared__ float4 s_xo[NT];                      // mu and opacity
    __shared__ float4 s_vel[DYN ? NT : 1];
    __shared__ float s_col[CL > 0 ? NT * CL : 1];
    __shared__ float s_origin[3];
    __shared__ int s_max;
    constexpr int NWB = NT / 64;
    __shared__ RayBundle s_bundle[NWB];
    __shared__ int32_t s_wbf[NWB];       // largest last id of each wavefront's pixels
    __shared__ uint64_t s_mask[NWB][NWB];  // [wavefront][staging wavefront]: Gaussians it evaluates
    __shared__ __align__(16) float s_red[NWB][16 * kRedRow];  // per wavefront: the gradient reduction

    const TileGrid& g = p.g;
    const int n_tiles = g.n_tiles_w * g.n_tiles_h;
    const int nblocks = n_tiles * g.n_cams;
    const int slot = xcd_tile((int)blockIdx.x, nblocks);
    const int logical = p.tile_order ? p.tile_order[slot] : slot;
    const int cam = logical / n_tiles, tile = logical - cam * n_tiles;
    const int bs = g.tile_w * g.tile_h;
    const int nthr = (bs + PX - 1) / PX;
    const int tr = threadIdx.x;
    const int lane = __lane_id();
    const int trow = tile / g.n_tiles_w, tcol = tile - trow * g.n_tiles_w;
    const int gt = cam * n_tiles + tile;  // utils.h:48-58
    const int32_t range_start = p.offsets[gt];
    const int32_t range_end = (gt == nblocks - 1) ? (int32_t)g.n_isects : p.offsets[gt + 1];
    const int64_t hw = (int64_t)g.width * g.height;

    // a pixel's index in the [cams, H, W] images (utils.h:32-44), recomputed where needed rather than
    // kept in registers
    auto pixel_of = [&](int h) {
        const int qi = PX * tr + h;
        const int ty = qi / g.tile_w, tx = qi - ty * g.tile_w;
        const int i = trow * g.tile_h + ty, j = tcol * g.tile_w + tx;
        return (int64_t)cam * hw + min((int64_t)i * g.width + j, hw - 1);
    };
    BwdPixel<CS> px[PX];
    f3 ro0[PX];  // the pixels' ray origins, for the set-up only
#pragma unroll
    for (int h = 0; h < PX; ++h) {
        BwdPixel<CS>& q = px[h];
        const int qi = PX * tr + h;
        const int ty = qi / g.tile_w, tx = qi - ty * g.tile_w;
        const int i = trow * g.tile_h + ty, j = tcol * g.tile_w + tx;  // utils.h:32-44
        q.inside = qi < bs && i < g.height && j < g.width;
        const int64_t pix = pixel_of(h);
        q.rd = q.inside ? ld3(p.ray_d + 3 * pix) : mk3(0.f, 0.f, 0.f);
        ro0[h] = q.inside ? ld3(p.ray_o + 3 * pix) : mk3(0.f, 0.f, 0.f);
        q.rt = 0.f;
        if constexpr (DYN) q.rt = q.inside ? p.rtd[pix] : 0.0f;
        const float T_final = 1.0f - p.render_alpha[pix];
        q.T = T_final;
#pragma unroll
        for (int k = 0; k < CS; ++k) q.v_c[k] = 0.f;
#pragma unroll
        for (int k = 0; k < CDIM; ++k) q.v_c[k] = q.inside ? p.v_rgb[pix * CDIM + k] : 0.0f;
        q.v_d = q.inside ? p.v_depth[pix] : 0.0f;
        q.buf = q.inside ? -T_final * p.v_alpha[pix] : 0.0f;
        q.bin_final = q.inside ? p.last_ids[pix] : 0;
        q.v_t = 0.f;
        q.v_ro = mk3(0.f, 0.f, 0.f);
        q.v_rd = mk3(0.f, 0.f, 0.f);
    }

    if (tr == 0) { s_origin[0] = ro0[0].x; s_origin[1] = ro0[0].y; s_origin[2] = ro0[0].z; s_max = -1; }
    __syncthreads();
    const f3 o0 = mk3(s_origin[0], s_origin[1], s_origin[2]);
    bool same = true;
#pragma unroll
    for (int h = 0; h < PX; ++h)
        same = same && (!px[h].inside || (__float_as_uint(ro0[h].x) == __float_as_uint(o0.x) &&
                                          __float_as_uint(ro0[h].y) == __float_as_uint(o0.y) &&
                                          __float_as_uint(ro0[h].z) == __float_as_uint(o0.z)));
    const bool fixed = !DYN && __syncthreads_and(same);

    int32_t lane_bin_final = px[0].bin_final;
#pragma unroll
    for (int h = 1; h < PX; ++h) lane_bin_final = max(lane_bin_final, px[h].bin_final);
    const int32_t wave_bin_final = wave_max(lane_bin_final);
    const int wave = tr >> 6;
    const int nwb = (int)(blockDim.x >> 6);
    {
        bool in2[PX];
        f3 ro2[PX], rd2[PX];
        float rt2[PX];
#pragma unroll
        for (int h = 0; h < PX; ++h) {
            in2[h] = px[h].inside;
            ro2[h] = ro0[h];
            rd2[h] = px[h].rd;
            rt2[h] = px[h].rt;
        }
        const RayBundle bun = wave_bundle<PX>(in2, ro2, rd2, rt2);
        if (lane == 0) {
            s_bundle[wave] = bun;
            s_wbf[wave] = wave_bin_final;
        }
    }
    if (lane == 0) atomicMax(&s_max, wave_bin_final);
    // The lane that adds component k of a chunk (k = lane / 4, lanes 4k) writes to
    // dst_base[chunk] + gid * dst_stride[chunk]; both are fixed per lane.
    constexpr int kChunks = (K + 15) / 16;
    float* dst_base[kChunks];
    int dst_stride[kChunks];
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
        const int kk = 16 * ch + (lane >> 2);
        if (kk < CDIM) {  // colour gradients of camera cam start at cam * (n * CDIM - col_shift)
            dst_base[ch] = p.v_colors + (int64_t)cam * (g.n * CDIM - p.col_shift) + kk;
            dst_stride[ch] = CDIM;
        } else if (kk < CDIM + 3) {
            dst_base[ch] = p.v_means + (kk - CDIM); dst_stride[ch] = 3;
        } else if (kk < CDIM + 9) {
            dst_base[ch] = p.v_mt + (kk - CDIM - 3); dst_stride[ch] = 6;
        } else if (kk == CDIM + 9) {
            dst_base[ch] = p.v_opac; dst_stride[ch] = 1;
        } else if (kk < K) {
            dst_base[ch] = p.v_velocity + (kk - CDIM - 10); dst_stride[ch] = 3;
        } else {
            dst_base[ch] = nullptr; dst_stride[ch] = 0;
        }
    }
    __syncthreads();
    constexpr bool counting = COUNT;  // the pair counters (a variant of its own: their scalar work per pair)
    uint64_t n_eval = 0, n_contrib = 0;  // evaluated / composited pixel-pairs of the wave, when counting
    const int32_t eff_end = min(range_end - 1, s_max);
    const int32_t n_eff = eff_end - range_start + 1;
    const int num_batches = n_eff > 0 ? (n_eff + nthr - 1) / nthr : 0;
    // the flatten id a thread stages in the next batch, loaded one batch ahead (its latency then
    // overlaps the pair loop instead of preceding the Gaussian's own loads)
    int32_t fid_next = 0;
    if (num_batches > 0 && tr < nthr && eff_end - tr >= range_start) fid_next = p.flatten[eff_end - tr];

    for (int b = 0; b < num_batches; ++b) {
        __syncthreads();
        const int32_t batch_end = eff_end - nthr * b;
        const int32_t idx = batch_end - tr;
        bool staged = false;
        CullGauss cg;
        const int32_t fid_cur = fid_next;
        if (tr < nthr && idx - nthr >= range_start) fid_next = p.flatten[idx - nthr];
        if (tr < nthr && idx >= range_start) {
            staged = true;
            const int32_t fid = fid_cur;
            const int64_t gid = fid - (int64_t)cam * g.n;
            s_id[tr] = fid;
            const f3 mu = ld3(p.means + 3 * gid);
            const float4 q = p.quats[gid];
            const f3 sc = ld3(p.scales + 3 * gid);
            f3 r0, r1, r2;
            iscl_rot_rows(q, sc, r0, r1, r2);
            f3 gro = mk3(0.f, 0.f, 0.f);
            if (fixed) gro = rows_mul(r0, r1, r2, o0 - mu);
            s_m0[tr] = make_float4(r0.x, r0.y, r0.z, gro.x);
            s_m1[tr] = make_float4(r1.x, r1.y, r1.z, gro.y);
            s_m2[tr] = make_float4(r2.x, r2.y, r2.z, gro.z);
            const float op = p.opac[gid];
            s_xo[tr] = make_float4(mu.x, mu.y, mu.z, op);
            f3 vel = mk3(0.f, 0.f, 0.f);
            if constexpr (DYN) {
                vel = ld3(p.velocity + 3 * gid);
                s_vel[tr] = make_float4(vel.x, vel.y, vel.z, 0.f);
            }
            if constexpr (CL > 0) {
                const float* cp = p.colors + ((int64_t)fid * CDIM - (int64_t)cam * p.col_shift);
#pragma unroll
                for (int k = 0; k < CL; ++k) s_col[tr * CL + k] = cp[k];
            }
            cg = cull_gauss(mu, r0, r1, r2, sc, q, op, vel);
        }
        // which wavefronts evaluate this Gaussian: those with a pixel at or past it (last ids)
        // that the Gaussian can reach; one ballot per wavefront
        for (int k = 0; k < nwb; ++k) {
            const bool keep = staged && idx <= s_wbf[k] && cull_keep<DYN>(s_bundle[k], cg);
            const uint64_t m = __ballot(keep);
            if (lane == 0) s_mask[k][wave] = m;
        }
        __syncthreads();
        // the pair loop, instantiated for both origin modes so that neither branches per pair
        auto pairs = [&](auto fixed_c) {
            constexpr bool FIXED = decltype(fixed_c)::value;
            for (int w2 = 0; w2 < nwb; ++w2)
            for (uint64_t m = uniform_u64(s_mask[wave][w2]); m != 0; m &= m - 1) {
                const int t = (w2 << 6) + (int)__builtin_ctzll(m);
                BwdGauss gs;
                {
                    const float4 a = s_m0[t], bq = s_m1[t], cq = s_m2[t], xo = s_xo[t];
                    gs.r0 = mk3(a.x, a.y, a.z);
                    gs.r1 = mk3(bq.x, bq.y, bq.z);
                    gs.r2 = mk3(cq.x, cq.y, cq.z);
                    gs.gro_fixed = mk3(a.w, bq.w, cq.w);
                    gs.mu = mk3(xo.x, xo.y, xo.z);
                    gs.op = xo.w;
                    gs.vel = mk3(0.f, 0.f, 0.f);
                    if constexpr (DYN) gs.vel = mk3(s_vel[t].x, s_vel[t].y, s_vel[t].z);
                }
                const int32_t gidx = batch_end - t;
                float rgb[CS];
#pragma unroll
                for (int k = 0; k < CS; ++k) rgb[k] = 0.f;
                if constexpr (CDIM > 0) {
                    if constexpr (CL > 0) {
#pragma unroll
                        for (int k = 0; k < CDIM; ++k) rgb[k] = s_col[t * CL + k];
                    } else {
                        const float* cp = p.colors + ((int64_t)s_id[t] * CDIM - (int64_t)cam * p.col_shift);
#pragma unroll
                        for (int k = 0; k < CDIM; ++k) rgb[k] = cp[k];
                    }
                }
                // each pixel slot evaluated, then composited, in turn (one evaluation live at a time): the
                // first slot always (its gradients initialise the accumulators), the others only when a
                // lane of the wave takes the pair (eval3d_bwd.cu:209-212 skips pairs below the alpha
                // threshold; an invalid pair adds exact zeros, so skipping whole slots changes nothing)
                auto eval = [&](int h) {
                    f3 ro = mk3(0.f, 0.f, 0.f);
                    if constexpr (!FIXED) ro = px[h].inside ? ld3(p.ray_o + 3 * pixel_of(h)) : ro;
                    const BwdEval e = bwd_eval<DYN, FIXED>(gs, ro, px[h].rd, px[h].rt,
                                                           px[h].inside && gidx <= px[h].bin_final);
                    if (counting) {  // wave totals, scalar
                        n_eval += (uint64_t)__popcll(__builtin_amdgcn_ballot_w64(px[h].inside && gidx <= px[h].bin_final));
                        n_contrib += (uint64_t)__popcll(__builtin_amdgcn_ballot_w64(e.valid));
                    }
                    return e;
                };
                float acc[K];
                f3 vg_sum;
                bool any_valid;
                {
                    const BwdEval e = eval(0);
                    any_valid = __builtin_amdgcn_ballot_w64(e.valid) != 0;
                    bwd_pair<CDIM, CS, K, DYN, RG, true>(px[0], gs, e, rgb, acc, vg_sum);
                }
#pragma unroll
                for (int h = 1; h < PX; ++h) {
                    // a slot none of whose pixels reaches this Gaussian adds nothing: not evaluated
                    if (__builtin_amdgcn_ballot_w64(px[h].inside && gidx <= px[h].bin_final) == 0) continue;
                    const BwdEval e = eval(h);
                    if (__builtin_amdgcn_ballot_w64(e.valid) != 0) {  // wave-uniform
                        any_valid = true;
                        bwd_pair<CDIM, CS, K, DYN, RG, false>(px[h], gs, e, rgb, acc, vg_sum);
                    }
                }
                if (!any_valid) continue;  // nothing to reduce (wave-uniform)
                if constexpr (!(RG || DYN)) {
                    const f3 v_omm = rows_tmul(gs.r0, gs.r1, gs.r2, vg_sum);
                    acc[CDIM + 0] = -v_omm.x;
                    acc[CDIM + 1] = -v_omm.y;
                    acc[CDIM + 2] = -v_omm.z;
                }

                // wave totals by reduce-scatter: lane l ends with component 16 * chunk + (l >> 2);
                // the first lane of each quad adds it, one atomic instruction per chunk of 16
                // Gaussian index below 2^31 (flatten ids are int32): one 32 x 32 + 64-bit multiply-add
                const uint32_t gid = (uint32_t)(__builtin_amdgcn_readfirstlane(s_id[t]) - (int64_t)cam * g.n);
#pragma unroll
                for (int ch = 0; ch < kChunks; ++ch) {
                    float chunk[16];
#pragma unroll
                    for (int k = 0; k < 16; ++k) chunk[k] = (16 * ch + k < K) ? acc[16 * ch + k] : 0.f;
                    const float tot = wave_reduce_scatter16_lds(chunk, min(16, K - 16 * ch), s_red[wave]);
                    if ((lane & 3) == 0 && 16 * ch + (lane >> 2) < K)
                        unsafeAtomicAdd((float*)((char*)dst_base[ch] + (uint64_t)gid * (uint32_t)(4 * dst_stride[ch])),
                                        tot);
                }
            }
        };
        if (fixed) pairs(std::true_type{});
        else pairs(std::false_type{});
    }
    if (counting && lane == 0) {  // one atomic per wave and counter
        atomicAdd(p.pair_counts, (unsigned long long)n_eval);
        atomicAdd(p.pair_counts + 1, (unsigned long long)n_contrib);
    }
#pragma unroll
    for (int h = 0; h < PX; ++h) {
        if (px[h].inside) {
            const int64_t pix = pixel_of(h);
            if constexpr (RG) {
                st3(p.v_ray_o + 3 * pix, px[h].v_ro);
                st3(p.v_ray_d + 3 * pix, px[h].v_rd);
            }
            if constexpr (DYN) p.v_time[pix] = px[h].v_t;
        }
    }
}

// Variants without per-pixel ray gradients exist for CDIM <= kColorLdsMax, with two or (tiles of
// more than 128 pixels) four pixels per thread; larger CDIMs always compute them, two pixels per
// thread (the C-ABI then needs the ray-gradient buffers). Tiles of more than 256 pixels (up to
// kMaxTilePixels) take four pixels per thread in workgroups of up to 256 threads, with and without
// ray gradients.
constexpr int64_t kBwdFullGridWaves = 3 * 1024;

// one launch, with or without the pair counters
template <int CDIM, bool DYN, bool RG, int PX, int NT>
void launch_bwd(int n_blocks, int threads, const Eval3dParams& p, hipStream_t s) {
    if (p.pair_counts) eval3d_bwd_kernel<CDIM, DYN, RG, PX, NT, true><<<n_blocks, threads, 0, s>>>(p);
    else eval3d_bwd_kernel<CDIM, DYN, RG, PX, NT, false><<<n_blocks, threads, 0, s>>>(p);
}

}  // namespace

template <int CDIM>
int eval3d_bwd_cdim(bool dyn, bool ray_grads, const Eval3dParams& p, hipStream_t s) {
    const int n_blocks = p.g.n_tiles_w * p.g.n_tiles_h * p.g.n_cams;
    const int tile_px = p.g.tile_w * p.g.tile_h;
    // whole wavefronts (the reduction uses every lane)
    const int bs2 = ((tile_px + 1) / 2 + 63) / 64 * 64;
    const int bs4 = ((tile_px + 3) / 4 + 63) / 64 * 64;
    constexpr int T = kTileThreads;
    if (tile_px > T) {
        if (ray_grads || CDIM > kColorLdsMax) {
            if (!p.v_ray_o || !p.v_ray_d)
                return xsg_fail(XSG_ERR_INVALID, "ray gradient buffers are required for cdim %d", CDIM);
            if (dyn) launch_bwd<CDIM, true, true, 4, T>(n_blocks, bs4, p, s);
            else launch_bwd<CDIM, false, true, 4, T>(n_blocks, bs4, p, s);
        } else {
            if (dyn) launch_bwd<CDIM, true, false, 4, T>(n_blocks, bs4, p, s);
            else launch_bwd<CDIM, false, false, 4, T>(n_blocks, bs4, p, s);
        }
        return XSG_OK;
    }
    if constexpr (CDIM <= kColorLdsMax) {
        if (!ray_grads) {
            // four pixels per lane when the grid still fills the GPU's wave slots (three waves on each
            // of 1024 SIMDs); a small grid (cfg3's 1024 lidar tiles) runs two per lane on twice the
            // waves; the caller may fix either
            const bool px4 = p.px_hint == 4 ||
                             (p.px_hint == 0 && (int64_t)n_blocks * (bs4 / 64) >= kBwdFullGridWaves);
            if (tile_px > 128 && px4) {
                if (dyn) launch_bwd<CDIM, true, false, 4, T / 4>(n_blocks, bs4, p, s);
                else launch_bwd<CDIM, false, false, 4, T / 4>(n_blocks, bs4, p, s);
            } else {
                if (dyn) launch_bwd<CDIM, true, false, 2, T / 2>(n_blocks, bs2, p, s);
                else launch_bwd<CDIM, false, false, 2, T / 2>(n_blocks, bs2, p, s);
            }
            return XSG_OK;
        }
    }
    if (!p.v_ray_o || !p.v_ray_d) return xsg_fail(XSG_ERR_INVALID, "ray gradient buffers are required for cdim %d", CDIM);
    if (dyn) launch_bwd<CDIM, true, true, 2, T / 2>(n_blocks, bs2, p, s);
    else launch_bwd<CDIM, false, true, 2, T / 2>(n_blocks, bs2, p, s);
    return XSG_OK;
}

}  // namespace xsg
