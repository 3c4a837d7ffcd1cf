/*
 * xsimgs_amd measurement support: entry points with no counterpart in the reference, used by
 * bench.py to price its kernels against what this GPU measurably issues.
 *
 * The same conventions as xsimgs_amd.h: device pointers, a HIP stream, XSG_OK or a negative error
 * code with xsg_last_error() holding the message.
 */
#ifndef XSIMGS_AMD_BENCH_H
#define XSIMGS_AMD_BENCH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* VALU issue ceiling. Launches `blocks` workgroups of 256 threads (four wave64s each; 256 * w
 * blocks put w waves on every SIMD of a 256-CU part) that each run `iters` iterations of 16 FP32
 * FMAs in four independent chains (v_fma_f32, no packed FP32): 16 * iters VALU instructions per
 * wavefront, 64 * iters per thread. `out` takes blocks * 256 floats (the chains' sums, so that
 * nothing is optimised away); `stamps` takes 4 * blocks uint64: per workgroup the shader-clock
 * counter (s_memtime) at start and end, then the 100 MHz real-time counter (s_memrealtime) at start
 * and end, from which the host reads the clock the work ran at. */
int xsg_bench_valu_ceiling(int blocks, int iters, float* out, uint64_t* stamps, void* stream);

#ifdef __cplusplus
}
#endif

#endif
