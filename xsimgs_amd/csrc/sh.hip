// Spherical harmonics -> RGB (forward and backward), reference csrc/color/sh_fwd.cu, sh_bwd.cu.
//
// One thread per Gaussian: the basis is evaluated once and shared by the three channels (the
// reference runs one thread per (Gaussian, channel)). For the [N, K, 3] layout a 256-Gaussian
// block stages its coefficient rows through LDS with coalesced loads; rows are padded to an odd
// stride so that each thread's row reads hit distinct banks. The [3, K, N] layout is already
// coalesced per thread and is read directly. The backward writes every band of d_coeffs (zeros
// above the used degree), d_positions without atomics, and per-block d_origin partials that a
// second kernel sums in a fixed order.
#include <mutex>

#include "xsg_common.h"

namespace {

constexpr int kBlock = 256;

template <int DEG>
XSG_DEV void sh_basis(f3 d, float* Y) {
    const float x = d.x, y = d.y, z = d.z;
    Y[0] = 0.2820947917738781f;
    if constexpr (DEG >= 1) {
        Y[1] = -0.48860251190292f * y;
        Y[2] = 0.48860251190292f * z;
        Y[3] = -0.48860251190292f * x;
    }
    if constexpr (DEG >= 2) {
        const float z2 = z * z;
        const float fTmp0B = -1.092548430592079f * z;
        const float fC1 = x * x - y * y, fS1 = 2.f * x * y;
        Y[4] = 0.5462742152960395f * fS1;
        Y[5] = fTmp0B * y;
        Y[6] = 0.9461746957575601f * z2 - 0.3153915652525201f;
        Y[7] = fTmp0B * x;
        Y[8] = 0.5462742152960395f * fC1;
        if constexpr (DEG >= 3) {
            const float fTmp0C = -2.285228997322329f * z2 + 0.4570457994644658f;
            const float fTmp1B = 1.445305721320277f * z;
            const float fC2 = x * fC1 - y * fS1, fS2 = x * fS1 + y * fC1;
            Y[9] = -0.5900435899266435f * fS2;
            Y[10] = fTmp1B * fS1;
            Y[11] = fTmp0C * y;
            Y[12] = z * (1.865881662950577f * z2 - 1.119528997770346f);
            Y[13] = fTmp0C * x;
            Y[14] = fTmp1B * fC1;
            Y[15] = -0.5900435899266435f * fC2;
            if constexpr (DEG >= 4) {
                const float fTmp0D = z * (-4.683325804901025f * z2 + 2.007139630671868f);
                const float fTmp1C = 3.31161143515146f * z2 - 0.47308734787878f;
                const float fTmp2B = -1.770130769779931f * z;
                const float fC3 = x * fC2 - y * fS2, fS3 = x * fS2 + y * fC2;
                Y[16] = 0.6258357354491763f * fS3;
                Y[17] = fTmp2B * fS2;
                Y[18] = fTmp1C * fS1;
                Y[19] = fTmp0D * y;
                Y[20] = 1.984313483298443f * z * Y[12] - 1.006230589874905f * Y[6];
                Y[21] = fTmp0D * x;
                Y[22] = fTmp1C * fC1;
                Y[23] = fTmp2B * fC2;
                Y[24] = 0.6258357354491763f * fC3;
            }
        }
    }
}

// colour of one channel; `c(k)` returns band k of that channel. Summation grouped per degree as in
// sh_coeffs_to_color_fast (sh_fwd.cu:16-115).
template <int DEG, class CF>
XSG_DEV float sh_color(f3 d, const float* Y, CF c) {
    float r = Y[0] * c(0);
    if constexpr (DEG >= 1) r += 0.48860251190292f * (-d.y * c(1) + d.z * c(2) - d.x * c(3));
    if constexpr (DEG >= 2) r += Y[4] * c(4) + Y[5] * c(5) + Y[6] * c(6) + Y[7] * c(7) + Y[8] * c(8);
    if constexpr (DEG >= 3)
        r += Y[9] * c(9) + Y[10] * c(10) + Y[11] * c(11) + Y[12] * c(12) + Y[13] * c(13) +
             Y[14] * c(14) + Y[15] * c(15);
    if constexpr (DEG >= 4)
        r += Y[16] * c(16) + Y[17] * c(17) + Y[18] * c(18) + Y[19] * c(19) + Y[20] * c(20) +
             Y[21] * c(21) + Y[22] * c(22) + Y[23] * c(23) + Y[24] * c(24);
    return r;
}

// d(colour)/d(dir) contracted with g[k] = sum_c coeff[k][c] * d_out[c] (sh_bwd.cu:50-246).
template <int DEG>
XSG_DEV f3 sh_dir_grad(f3 d, const float* g) {
    const float x = d.x, y = d.y, z = d.z;
    f3 dd = mk3(0.f, 0.f, 0.f);
    if constexpr (DEG >= 1) {
        dd.x += -0.48860251190292f * g[3];
        dd.y += -0.48860251190292f * g[1];
        dd.z += 0.48860251190292f * g[2];
    }
    if constexpr (DEG >= 2) {
        const float z2 = z * z;
        const float fTmp0B = -1.092548430592079f * z;
        const float fC1 = x * x - y * y, fS1 = 2.f * x * y;
        const float fTmp0B_z = -1.092548430592079f;
        const float fC1_x = 2.f * x, fC1_y = -2.f * y, fS1_x = 2.f * y, fS1_y = 2.f * x;
        const float p6_z = 2.f * 0.9461746957575601f * z;
        const float p7_x = fTmp0B, p7_z = fTmp0B_z * x, p5_y = fTmp0B, p5_z = fTmp0B_z * y;
        const float p8_x = 0.5462742152960395f * fC1_x, p8_y = 0.5462742152960395f * fC1_y;
        const float p4_x = 0.5462742152960395f * fS1_x, p4_y = 0.5462742152960395f * fS1_y;
        dd.x += p4_x * g[4] + p8_x * g[8] + p7_x * g[7];
        dd.y += p4_y * g[4] + p8_y * g[8] + p5_y * g[5];
        dd.z += p6_z * g[6] + p7_z * g[7] + p5_z * g[5];
        if constexpr (DEG >= 3) {
            const float fTmp0C = -2.285228997322329f * z2 + 0.4570457994644658f;
            const float fTmp1B = 1.445305721320277f * z;
            const float fC2 = x * fC1 - y * fS1, fS2 = x * fS1 + y * fC1;
            const float fTmp0C_z = -2.285228997322329f * 2.f * z;
            const float fTmp1B_z = 1.445305721320277f;
            const float fC2_x = fC1 + x * fC1_x - y * fS1_x;
            const float fC2_y = x * fC1_y - fS1 - y * fS1_y;
            const float fS2_x = fS1 + x * fS1_x + y * fC1_x;
            const float fS2_y = x * fS1_y + fC1 + y * fC1_y;
            const float p12_z = 3.f * 1.865881662950577f * z2 - 1.119528997770346f;
            const float p13_x = fTmp0C, p13_z = fTmp0C_z * x, p11_y = fTmp0C, p11_z = fTmp0C_z * y;
            const float p14_x = fTmp1B * fC1_x, p14_y = fTmp1B * fC1_y, p14_z = fTmp1B_z * fC1;
            const float p10_x = fTmp1B * fS1_x, p10_y = fTmp1B * fS1_y, p10_z = fTmp1B_z * fS1;
            const float p15_x = -0.5900435899266435f * fC2_x, p15_y = -0.5900435899266435f * fC2_y;
            const float p9_x = -0.5900435899266435f * fS2_x, p9_y = -0.5900435899266435f * fS2_y;
            dd.x += p9_x * g[9] + p15_x * g[15] + p10_x * g[10] + p14_x * g[14] + p13_x * g[13];
            dd.y += p9_y * g[9] + p15_y * g[15] + p10_y * g[10] + p14_y * g[14] + p11_y * g[11];
            dd.z += p12_z * g[12] + p13_z * g[13] + p11_z * g[11] + p14_z * g[14] + p10_z * g[10];
            if constexpr (DEG >= 4) {
                const float p12 = z * (1.865881662950577f * z2 - 1.119528997770346f);
                const float p6 = 0.9461746957575601f * z2 - 0.3153915652525201f;
                (void)p6;
                const float fTmp0D = z * (-4.683325804901025f * z2 + 2.007139630671868f);
                const float fTmp1C = 3.31161143515146f * z2 - 0.47308734787878f;
                const float fTmp2B = -1.770130769779931f * z;
                const float fTmp0D_z = 3.f * -4.683325804901025f * z2 + 2.007139630671868f;
                const float fTmp1C_z = 2.f * 3.31161143515146f * z;
                const float fTmp2B_z = -1.770130769779931f;
                const float fC3_x = fC2 + x * fC2_x - y * fS2_x;
                const float fC3_y = x * fC2_y - fS2 - y * fS2_y;
                const float fS3_x = fS2 + y * fC2_x + x * fS2_x;
                const float fS3_y = x * fS2_y + fC2 + y * fC2_y;
                const float p20_z = 1.984313483298443f * (p12 + z * p12_z) + -1.006230589874905f * p6_z;
                const float p21_x = fTmp0D, p21_z = fTmp0D_z * x, p19_y = fTmp0D, p19_z = fTmp0D_z * y;
                const float p22_x = fTmp1C * fC1_x, p22_y = fTmp1C * fC1_y, p22_z = fTmp1C_z * fC1;
                const float p18_x = fTmp1C * fS1_x, p18_y = fTmp1C * fS1_y, p18_z = fTmp1C_z * fS1;
                const float p23_x = fTmp2B * fC2_x, p23_y = fTmp2B * fC2_y, p23_z = fTmp2B_z * fC2;
                const float p17_x = fTmp2B * fS2_x, p17_y = fTmp2B * fS2_y, p17_z = fTmp2B_z * fS2;
                const float p24_x = 0.6258357354491763f * fC3_x, p24_y = 0.6258357354491763f * fC3_y;
                const float p16_x = 0.6258357354491763f * fS3_x, p16_y = 0.6258357354491763f * fS3_y;
                dd.x += p16_x * g[16] + p24_x * g[24] + p17_x * g[17] + p23_x * g[23] + p18_x * g[18] +
                        p22_x * g[22] + p21_x * g[21];
                dd.y += p16_y * g[16] + p24_y * g[24] + p17_y * g[17] + p23_y * g[23] + p18_y * g[18] +
                        p22_y * g[22] + p19_y * g[19];
                dd.z += p20_z * g[20] + p21_z * g[21] + p19_z * g[19] + p22_z * g[22] + p18_z * g[18] +
                        p23_z * g[23] + p17_z * g[17];
            }
        }
    }
    return dd;
}

XSG_DEV bool mask_ok(const uint32_t* mask, int64_t i) {
    return mask ? ((mask[i / 32] & (1u << (i % 32))) != 0) : true;
}

constexpr int odd_stride(int n) { return (n % 2 == 0) ? n + 1 : n; }

// Cooperative copy of `rows` rows of ROW_LEN floats (global row pitch `pitch`) into LDS rows of
// stride S. A full tile of contiguous rows is copied with every thread's 16-byte loads issued
// before any LDS store, so each wavefront keeps ROW_LEN / 4 loads in flight; other tiles use a
// plain strided loop.
template <int ROW_LEN, int S>
XSG_DEV void stage_rows(float* lds, const float* __restrict__ src, int64_t pitch, int rows) {
    if constexpr (ROW_LEN % 4 == 0) {
        if (rows == kBlock && pitch == ROW_LEN && ((uintptr_t)src & 15) == 0) {
            constexpr int PER = ROW_LEN / 4;  // 16-byte vectors per thread
            typedef float v4f __attribute__((ext_vector_type(4)));
            const v4f* src4 = reinterpret_cast<const v4f*>(src);
            v4f v[PER];
#pragma unroll
            for (int k = 0; k < PER; ++k) v[k] = __builtin_nontemporal_load(src4 + k * kBlock + threadIdx.x);
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int e = 4 * (k * kBlock + (int)threadIdx.x);
                const int r = e / ROW_LEN, j = e - r * ROW_LEN;
                float* d = lds + r * S + j;
                d[0] = v[k].x; d[1] = v[k].y; d[2] = v[k].z; d[3] = v[k].w;
            }
            return;
        }
    }
    const int total = rows * ROW_LEN;
    for (int e = threadIdx.x; e < total; e += kBlock) {
        const int r = e / ROW_LEN, j = e - r * ROW_LEN;
        lds[r * S + j] = __builtin_nontemporal_load(src + (int64_t)r * pitch + j);
    }
}

// spherical_harmonics_fused_fwd_kernel (sh_fwd.cu:119-159), [N, K, 3] layout.
template <int DEG, bool HAS_DC>
__global__ __launch_bounds__(kBlock) void sh_fwd_nk3_kernel(
    int64_t n, int dim, const float* __restrict__ origin, const float* __restrict__ pos,
    const float* __restrict__ coeffs, const float* __restrict__ dc, const uint32_t* __restrict__ mask,
    int zero_masked, float* __restrict__ out) {
    constexpr int NB = (DEG + 1) * (DEG + 1) - (HAS_DC ? 1 : 0);  // bands read from `coeffs`
    constexpr int RL = NB * 3;
    constexpr int S = odd_stride(RL);
    __shared__ float lds[kBlock * S];
    const int64_t g0 = (int64_t)blockIdx.x * kBlock;
    const int rows = (int)min<int64_t>(kBlock, n - g0);
    const int t = threadIdx.x;
    const int64_t i = g0 + t;
    const bool active = t < rows;
    const bool valid = active && mask_ok(mask, i);
    // A block whose rows mostly pass the mask stages them all with wide loads; a sparse block (a mask
    // of the Gaussians some tile can hold, most of a frame's scene off screen) reads only its own rows,
    // straight from global memory (copying them to LDS first measured slower).
    bool staged = true;
    if constexpr (NB > 0) {
        staged = !mask || 4 * __syncthreads_count(valid) > rows;  // block-uniform
        if (staged) stage_rows<RL, S>(lds, coeffs + g0 * dim * 3, (int64_t)dim * 3, rows);
    }
    __syncthreads();
    if (!active) return;
    if (!valid) {
        if (zero_masked) { out[3 * i] = 0.f; out[3 * i + 1] = 0.f; out[3 * i + 2] = 0.f; }
        return;
    }
    const f3 diff = ld3(pos + 3 * i) - ld3(origin);
    const f3 dir = diff * (1.0f / sqrtf(dot(diff, diff)));
    float Y[(DEG + 1) * (DEG + 1)];
    sh_basis<DEG>(dir, Y);
    // the row in LDS when staged, else in global memory: one block-uniform branch, each side with
    // plain loads from one address space (a select per coefficient slowed the unmasked kernel by 10 %)
    auto shade = [&](const float* row) {
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            float dcv = 0.f;
            if constexpr (HAS_DC) dcv = dc[3 * i + c];
            auto cf = [&](int k) -> float {
                if constexpr (HAS_DC) return k == 0 ? dcv : row[(k - 1) * 3 + c];
                else return row[k * 3 + c];
            };
            out[3 * i + c] = sh_color<DEG>(dir, Y, cf) + 0.5f;
        }
    };
    if (staged) shade(lds + t * S);
    else shade(coeffs + i * dim * 3);
}

// [3, K, N] layout (band stride N): coalesced per thread without staging.
template <int DEG, bool HAS_DC>
__global__ __launch_bounds__(kBlock) void sh_fwd_3kn_kernel(
    int64_t n, int dim, const float* __restrict__ origin, const float* __restrict__ pos,
    const float* __restrict__ coeffs, const float* __restrict__ dc, const uint32_t* __restrict__ mask,
    int zero_masked, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    if (!mask_ok(mask, i)) {
        if (zero_masked) { out[3 * i] = 0.f; out[3 * i + 1] = 0.f; out[3 * i + 2] = 0.f; }
        return;
    }
    const f3 diff = ld3(pos + 3 * i) - ld3(origin);
    const f3 dir = diff * (1.0f / sqrtf(dot(diff, diff)));
    float Y[(DEG + 1) * (DEG + 1)];
    sh_basis<DEG>(dir, Y);
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const float* base = coeffs + (int64_t)c * n * dim + i;
        const float dcv = HAS_DC ? dc[(int64_t)c * n + i] : 0.f;
        auto cf = [&](int k) -> float {
            if constexpr (HAS_DC) return k == 0 ? dcv : base[(int64_t)(k - 1) * n];
            else return base[(int64_t)k * n];
        };
        out[3 * i + c] = sh_color<DEG>(dir, Y, cf) + 0.5f;
    }
}

// spherical_harmonics_fused_bwd_kernel (sh_bwd.cu:250-315), both layouts. Writes all `dim` bands.
template <int DEG, bool HAS_DC, bool L3KN>
__global__ __launch_bounds__(kBlock) void sh_bwd_kernel(
    int64_t n, int dim, const float* __restrict__ origin, const float* __restrict__ pos,
    const float* __restrict__ coeffs, const uint32_t* __restrict__ mask,
    const float* __restrict__ d_out, float* __restrict__ d_coeffs, float* __restrict__ d_dc,
    float* __restrict__ d_pos, float* __restrict__ origin_partial) {
    constexpr int NY = (DEG + 1) * (DEG + 1);
    constexpr int NB = NY - (HAS_DC ? 1 : 0);
    constexpr int RL = NB * 3;
    constexpr int S = odd_stride(RL > 0 ? RL : 1);
    __shared__ float lds[L3KN ? 1 : kBlock * S];
    __shared__ float red[3][kBlock / 64];
    const int64_t g0 = (int64_t)blockIdx.x * kBlock;
    const int rows = (int)min<int64_t>(kBlock, n - g0);
    const int t = threadIdx.x;
    const int64_t i = g0 + t;
    const bool active = t < rows;
    const bool valid = active && mask_ok(mask, i);
    float go[3] = {0.f, 0.f, 0.f};
    if (valid) { go[0] = d_out[3 * i]; go[1] = d_out[3 * i + 1]; go[2] = d_out[3 * i + 2]; }
    // The coefficients enter only the position gradient, through their product with the colour
    // gradient: a Gaussian whose colour gradient is exactly zero (one no tile composited) gets an
    // exactly zero position gradient without reading them (the reference multiplies them by zero;
    // the results differ at most in the sign of a zero, or where a coefficient is not finite). A
    // block whose rows mostly need them stages them all with wide loads; a sparse block reads only
    // the rows that need them.
    const bool need = valid && (go[0] != 0.f || go[1] != 0.f || go[2] != 0.f);
    bool staged = L3KN;
    if constexpr (!L3KN && NB > 0) {
        staged = 4 * __syncthreads_count(need) > rows;  // block-uniform
        if (staged) {
            stage_rows<RL, S>(lds, coeffs + g0 * dim * 3, (int64_t)dim * 3, rows);
            __syncthreads();
        }
    }
    f3 dpos = mk3(0.f, 0.f, 0.f);
    float Y[NY];
    if (valid) {
        const f3 diff = ld3(pos + 3 * i) - ld3(origin);
        const float il = 1.0f / sqrtf(dot(diff, diff));
        const f3 dir = diff * il;
        sh_basis<DEG>(dir, Y);
        if (need) {
            const float* row = coeffs + i * dim * 3;  // [N, K, 3] layout, read directly when not staged
            float g[NY];
#pragma unroll
            for (int k = 0; k < NY; ++k) {
                float s = 0.f;
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    float cv;
                    const int kb = k - (HAS_DC ? 1 : 0);
                    if (HAS_DC && k == 0) cv = 0.f;  // the DC band has no direction dependence
                    else if constexpr (L3KN) cv = coeffs[((int64_t)c * dim + kb) * n + i];
                    else cv = staged ? lds[t * S + kb * 3 + c] : row[kb * 3 + c];
                    s += cv * go[c];
                }
                g[k] = s;
            }
            const f3 ddir = sh_dir_grad<DEG>(dir, g);
            // normalize_bwd: (d - (d . n) n) / |v|
            dpos = ddir * il - diff * (il * il * il * dot(ddir, diff));
        }
    } else {
#pragma unroll
        for (int k = 0; k < NY; ++k) Y[k] = 0.f;
    }
    if (active) st3(d_pos + 3 * i, dpos);
    // d_coeffs: every band of the row, zero above the used degree and for masked Gaussians
    if constexpr (L3KN) {
        if (active) {
            for (int c = 0; c < 3; ++c) {
                for (int k = 0; k < dim; ++k) {
                    const int kk = k + (HAS_DC ? 1 : 0);
                    const float v = (kk < NY) ? Y[kk] * go[c] : 0.f;
                    d_coeffs[((int64_t)c * dim + k) * n + i] = v;
                }
                if (HAS_DC) d_dc[(int64_t)c * n + i] = Y[0] * go[c];
            }
        }
    } else {
        if (active && HAS_DC) {
            for (int c = 0; c < 3; ++c) d_dc[3 * i + c] = Y[0] * go[c];
        }
        // stage the output rows (dim*3 floats) through LDS in chunks of RL columns, then store
        // coalesced; columns beyond RL are zero.
        __syncthreads();
        if (active) {
#pragma unroll
            for (int k = 0; k < NB; ++k)
#pragma unroll
                for (int c = 0; c < 3; ++c) lds[t * S + k * 3 + c] = Y[k + (HAS_DC ? 1 : 0)] * go[c];
        }
        __syncthreads();
        const int row_len = dim * 3;
        float* dst = d_coeffs + g0 * row_len;
        const int total = rows * row_len;
        if ((row_len & 3) == 0 && ((uintptr_t)dst & 15) == 0) {
            // 16-byte stores (a row holds whole vectors), bypassing the caches: written once, read later
            typedef float v4f __attribute__((ext_vector_type(4)));
            v4f* dst4 = reinterpret_cast<v4f*>(dst);
            for (int e4 = t; e4 < total / 4; e4 += kBlock) {
                const int e = 4 * e4;
                const int r = e / row_len, j = e - r * row_len;
                const float* src = lds + r * S + j;
                v4f v;
                v.x = (j < RL) ? src[0] : 0.f;
                v.y = (j + 1 < RL) ? src[1] : 0.f;
                v.z = (j + 2 < RL) ? src[2] : 0.f;
                v.w = (j + 3 < RL) ? src[3] : 0.f;
                __builtin_nontemporal_store(v, dst4 + e4);
            }
        } else {
            for (int e = t; e < total; e += kBlock) {
                const int r = e / row_len, j = e - r * row_len;
                dst[e] = (j < RL) ? lds[r * S + j] : 0.f;
            }
        }
    }
    // d_origin = -sum(d_positions) (sh_bwd.cu:306-314): wave sums, then one partial per block (none
    // when the caller takes no origin gradient)
    if (!origin_partial) return;
    float ox = wave_sum(-dpos.x), oy = wave_sum(-dpos.y), oz = wave_sum(-dpos.z);
    const int w = t >> 6;
    if ((t & 63) == 0) { red[0][w] = ox; red[1][w] = oy; red[2][w] = oz; }
    __syncthreads();
    if (t < 3) {
        float s = 0.f;
        for (int k = 0; k < kBlock / 64; ++k) s += red[t][k];
        origin_partial[(int64_t)blockIdx.x * 3 + t] = s;
    }
}

// One workgroup of kSumThreads sums the per-block d_origin partials in a fixed order.
constexpr int kSumThreads = 1024;
__global__ __launch_bounds__(kSumThreads) void sum_partials_kernel(const float* __restrict__ part, int nb,
                                                                   float* __restrict__ out) {
    __shared__ float red[3][kSumThreads / 64];
    float s[3] = {0.f, 0.f, 0.f};
    for (int b = threadIdx.x; b < nb; b += kSumThreads)
        for (int c = 0; c < 3; ++c) s[c] += part[3 * b + c];
    for (int c = 0; c < 3; ++c) s[c] = wave_sum(s[c]);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) for (int c = 0; c < 3; ++c) red[c][w] = s[c];
    __syncthreads();
    if (threadIdx.x < 3) {
        float r = 0.f;
        for (int k = 0; k < kSumThreads / 64; ++k) r += red[threadIdx.x][k];
        out[threadIdx.x] = r;
    }
}

template <int DEG, bool DC>
void launch_fwd(bool l3kn, dim3 g, hipStream_t s, int64_t n, int dim, const float* o, const float* p,
                const float* c, const float* dc, const uint32_t* m, int zm, float* out) {
    if (l3kn) sh_fwd_3kn_kernel<DEG, DC><<<g, kBlock, 0, s>>>(n, dim, o, p, c, dc, m, zm, out);
    else sh_fwd_nk3_kernel<DEG, DC><<<g, kBlock, 0, s>>>(n, dim, o, p, c, dc, m, zm, out);
}

template <int DEG, bool DC>
void launch_bwd(bool l3kn, dim3 g, hipStream_t s, int64_t n, int dim, const float* o, const float* p,
                const float* c, const uint32_t* m, const float* dout, float* dcf, float* ddc, float* dp,
                float* part) {
    if (l3kn) sh_bwd_kernel<DEG, DC, true><<<g, kBlock, 0, s>>>(n, dim, o, p, c, m, dout, dcf, ddc, dp, part);
    else sh_bwd_kernel<DEG, DC, false><<<g, kBlock, 0, s>>>(n, dim, o, p, c, m, dout, dcf, ddc, dp, part);
}

}  // namespace

extern "C" int xsg_sh_fwd(int degree, const float* origin, int64_t n, int dim, const float* positions,
                          const float* coeffs, const float* coeffs_dc, const uint32_t* mask,
                          int layout_3kn, float* out, xsg_stream_t stream) {
    // masked Gaussians keep the caller's output values (the reference writes into `output` or zeros)
    return xsg_sh_fwd_ex(degree, origin, n, dim, positions, coeffs, coeffs_dc, mask, layout_3kn, 0, out, stream);
}

extern "C" int xsg_sh_fwd_ex(int degree, const float* origin, int64_t n, int dim, const float* positions,
                             const float* coeffs, const float* coeffs_dc, const uint32_t* mask,
                             int layout_3kn, int zero_masked_arg, float* out, xsg_stream_t stream) {
    // sh_fwd.cu:162-245 checks
    static const int ref_dims[5] = {1, 4, 9, 16, 25};
    if (degree < 0 || degree > 4)
        return xsg_fail(XSG_ERR_INVALID, "Unsupported spherical harmonics degree: %d", degree);
    const int required = ref_dims[degree] - (coeffs_dc ? 1 : 0);
    if (dim < required)
        return xsg_fail(XSG_ERR_INVALID,
                        "Number of harmonics band in coeffs tensor must be higher or equal than %d for "
                        "degree_to_use=%d%s", required, degree,
                        coeffs_dc ? " (zero-degree coeffs passed separately)" : "");
    if (n < 0) return xsg_fail(XSG_ERR_INVALID, "xsg_sh_fwd: n < 0");
    if (n == 0) return XSG_OK;
    const int zero_masked = (zero_masked_arg != 0 && mask) ? 1 : 0;
    const dim3 g(xsg_blocks(n, kBlock));
    const hipStream_t s = (hipStream_t)stream;
    const bool l = layout_3kn != 0;
    const bool dc = coeffs_dc != nullptr;
#define XSG_F(D) \
    (dc ? launch_fwd<D, true>(l, g, s, n, dim, origin, positions, coeffs, coeffs_dc, mask, zero_masked, out) \
        : launch_fwd<D, false>(l, g, s, n, dim, origin, positions, coeffs, coeffs_dc, mask, zero_masked, out))
    switch (degree) {
        case 0: XSG_F(0); break;
        case 1: XSG_F(1); break;
        case 2: XSG_F(2); break;
        case 3: XSG_F(3); break;
        case 4: XSG_F(4); break;
    }
#undef XSG_F
    XSG_TRY_LAUNCH("sh_fwd");
    return XSG_OK;
}

extern "C" size_t xsg_sh_bwd_workspace_bytes(int64_t n) {
    return (size_t)(xsg_blocks(n > 0 ? n : 1, kBlock)) * 3 * sizeof(float);
}

namespace {

// d_coeffs, d_coeffs_dc, d_positions and the per-block d_origin partials (`part`, 3 floats per
// kBlock Gaussians), then their fixed-order sum into d_origin. Shared by both backward entry points.
int sh_bwd_run(int degree, const float* origin, int64_t n, int dim, const float* positions,
               const float* coeffs, const uint32_t* mask, int layout_3kn, const float* d_output, int has_dc,
               float* d_coeffs, float* d_coeffs_dc, float* d_positions, float* d_origin, float* part,
               hipStream_t s) {
    static const int ref_dims[5] = {1, 4, 9, 16, 25};
    if (degree < 0 || degree > 4)
        return xsg_fail(XSG_ERR_INVALID, "Unsupported spherical harmonics degree: %d", degree);
    if (dim < ref_dims[degree] - (has_dc ? 1 : 0))
        return xsg_fail(XSG_ERR_INVALID, "coeffs hold %d bands, degree %d needs %d", dim, degree,
                        ref_dims[degree] - (has_dc ? 1 : 0));
    if (!d_origin) part = nullptr;  // no origin gradient: neither partials nor their sum
    if (n == 0) {  // d_origin = 0 without a memset node (callers may capture this in a graph)
        if (d_origin) sum_partials_kernel<<<1, kSumThreads, 0, s>>>(part, 0, d_origin);
        XSG_TRY_LAUNCH("sh_bwd");
        return XSG_OK;
    }
    const unsigned nb = xsg_blocks(n, kBlock);
    const bool l = layout_3kn != 0;
    const dim3 g(nb);
#define XSG_B(D) \
    (has_dc ? launch_bwd<D, true>(l, g, s, n, dim, origin, positions, coeffs, mask, d_output, d_coeffs, d_coeffs_dc, d_positions, part) \
            : launch_bwd<D, false>(l, g, s, n, dim, origin, positions, coeffs, mask, d_output, d_coeffs, d_coeffs_dc, d_positions, part))
    switch (degree) {
        case 0: XSG_B(0); break;
        case 1: XSG_B(1); break;
        case 2: XSG_B(2); break;
        case 3: XSG_B(3); break;
        case 4: XSG_B(4); break;
    }
#undef XSG_B
    if (d_origin) sum_partials_kernel<<<1, kSumThreads, 0, s>>>(part, (int)nb, d_origin);
    XSG_TRY_LAUNCH("sh_bwd");
    return XSG_OK;
}

// Scratch of xsg_sh_bwd_noalloc: the d_origin partials of up to XSG_SH_BWD_NOALLOC_MAX_N Gaussians
// (3 floats per kBlock Gaussians, 1.5 MiB). One copy per GPU, allocated with the code object and held
// until the process ends; every call on a GPU shares it.
constexpr int64_t kNoAllocParts = 3 * ((XSG_SH_BWD_NOALLOC_MAX_N + kBlock - 1) / kBlock);
static __device__ __align__(256) float scratch[kNoAllocParts];

// The device address of `scratch` on each GPU, looked up once per device (on the first call there,
// with that device current). In host code `scratch` names a host-side stand-in, never memory a
// kernel may touch: kernels only ever get these addresses.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices];

int scratch_for_current_device(float** out) {
    int dev = -1;
    const hipError_t e0 = hipGetDevice(&dev);
    if (e0 != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return xsg_fail(XSG_ERR_LAUNCH, "xsg_sh_bwd_noalloc: no usable current device (%s, device %d)",
                        hipGetErrorString(e0), dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return xsg_fail(XSG_ERR_LAUNCH, "xsg_sh_bwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                            dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return XSG_OK;
}

}  // namespace

extern "C" int xsg_sh_bwd(int degree, const float* origin, int64_t n, int dim, const float* positions,
                          const float* coeffs, const uint32_t* mask, int layout_3kn,
                          const float* d_output, int has_dc, float* d_coeffs, float* d_coeffs_dc,
                          float* d_positions, float* d_origin, void* workspace, xsg_stream_t stream) {
    if (n < 0 || !workspace) return xsg_fail(XSG_ERR_INVALID, "xsg_sh_bwd: bad arguments");
    if (const int rc = xsg_check_workspace(workspace, "xsg_sh_bwd")) return rc;
    return sh_bwd_run(degree, origin, n, dim, positions, coeffs, mask, layout_3kn, d_output, has_dc, d_coeffs,
                      d_coeffs_dc, d_positions, d_origin, (float*)workspace, (hipStream_t)stream);
}

extern "C" int xsg_sh_bwd_noalloc(int degree, const float* origin, int64_t n, int dim, const float* positions,
                                  const float* coeffs, const uint32_t* mask, int layout_3kn,
                                  const float* d_output, int has_dc, float* d_coeffs, float* d_coeffs_dc,
                                  float* d_positions, float* d_origin, xsg_stream_t stream) {
    if (n < 0) return xsg_fail(XSG_ERR_INVALID, "xsg_sh_bwd_noalloc: bad arguments");
    if (n > XSG_SH_BWD_NOALLOC_MAX_N)
        return xsg_fail(XSG_ERR_INVALID,
                        "xsg_sh_bwd_noalloc: %lld Gaussians exceed the scratch limit of %lld; use xsg_sh_bwd with a "
                        "workspace", (long long)n, (long long)XSG_SH_BWD_NOALLOC_MAX_N);
    float* part = nullptr;
    if (const int rc = scratch_for_current_device(&part)) return rc;
    return sh_bwd_run(degree, origin, n, dim, positions, coeffs, mask, layout_3kn, d_output, has_dc, d_coeffs,
                      d_coeffs_dc, d_positions, d_origin, part, (hipStream_t)stream);
}
