// Measurement support (no reference counterpart): the VALU issue ceiling bench.py prices the
// compositor kernels against. Four independent FMA chains per thread, four unrolled steps each, so
// that every wavefront always has an instruction ready and the SIMD's own issue rate is what the
// launch measures.
#include "xsg_common.h"
#include "../../include/xsimgs_amd_bench.h"

namespace {

__global__ __launch_bounds__(256) void valu_ceiling_kernel(int iters, float* __restrict__ out,
                                                            uint64_t* __restrict__ stamps) {
    const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    float a[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] = 0.25f + 1e-7f * threadIdx.x + k;
    const float m = 0.999f, c = 1e-3f;
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int k = 0; k < 4; ++k) a[k] = __builtin_fmaf(a[k], m, c);
    }
    out[(size_t)blockIdx.x * 256 + threadIdx.x] = (a[0] + a[1]) + (a[2] + a[3]);
    const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        uint64_t* st = stamps + 4 * (size_t)blockIdx.x;
        st[0] = t0;
        st[1] = t1;
        st[2] = r0;
        st[3] = r1;
    }
}

}  // namespace

extern "C" int xsg_bench_valu_ceiling(int blocks, int iters, float* out, uint64_t* stamps, void* stream) {
    if (blocks <= 0 || iters <= 0 || !out || !stamps)
        return xsg_fail(XSG_ERR_INVALID, "valu ceiling: blocks %d and iters %d must be positive, buffers given",
                        blocks, iters);
    valu_ceiling_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(iters, out, stamps);
    XSG_TRY_LAUNCH("valu ceiling");
    return XSG_OK;
}
