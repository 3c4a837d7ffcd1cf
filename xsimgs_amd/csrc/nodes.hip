// Scene-assembly producers that feed the rasterization path: the packed instance mask read by
// mask_radii_packed / SH, and the rigid per-instance copy of Gaussians into the frame's buffers
// (reference csrc/nodes/gs_masking.cu, csrc/nodes/container.cu). One thread per element / Gaussian.
#include "xsg_common.h"

namespace {

constexpr int kBlock = 256;

// mask_from_instances_kernel (gs_masking.cu:8-26) on wave64: one ballot covers two 32-bit words,
// written by lanes 0 and 32. Ids at or past n_inst count as enabled instead of reading past the mask.
__global__ __launch_bounds__(kBlock) void packed_mask_kernel(int64_t n, const int32_t* __restrict__ ids,
                                                             const uint8_t* __restrict__ inst_mask, int64_t n_inst,
                                                             uint32_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    bool v = false;
    if (i < n) {
        const int32_t id = ids[i];
        v = (id < 0 || (int64_t)id >= n_inst) ? true : inst_mask[id] != 0;
    }
    const uint64_t b = __ballot(v);
    const int lane = __lane_id();
    const int64_t word = i >> 5;
    if ((lane & 31) == 0 && word < ((n + 31) >> 5)) out[word] = lane ? (uint32_t)(b >> 32) : (uint32_t)b;
}

// Visibility of the regular tilings' Gaussians as a packed mask (an extension): bit i % 32 of word
// i / 32 set when some camera's radii of Gaussian i pass the tiling's test (an instance whose radii are
// not both positive, r.x <= 0 || r.y <= 0, gets no tile), so that every Gaussian a tile can hold has its
// bit. Radii [n_cams, n, 2], camera-major.
__global__ __launch_bounds__(kBlock) void packed_visibility_kernel(int64_t n, int n_cams,
                                                                   const float2* __restrict__ radii,
                                                                   uint32_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    bool v = false;
    if (i < n)
        for (int c = 0; c < n_cams; ++c) {
            const float2 r = radii[(int64_t)c * n + i];
            v = v || !(r.x <= 0.0f || r.y <= 0.0f);
        }
    const uint64_t b = __ballot(v);
    const int lane = __lane_id();
    const int64_t word = i >> 5;
    if ((lane & 31) == 0 && word < ((n + 31) >> 5)) out[word] = lane ? (uint32_t)(b >> 32) : (uint32_t)b;
}

struct RigidArgs {
    int64_t n, n_inst, n_out, buffer_offset;
    const float* pos;
    const float4* rot;
    const int32_t* ids;
    const float4* iq;
    const float* it;
    const float* iv;
    const float* iw;
    const uint8_t* imask;
    const int32_t* per_inst_off;
    const int32_t* gs_inst_off;
};

// output row of Gaussian i or -1 when it is skipped: instance out of range or disabled, or a row
// outside the output buffers (the reference writes such rows unchecked)
template <bool OFFSETS>
XSG_DEV int64_t rigid_row(const RigidArgs& a, int64_t i, uint32_t& k) {
    k = (uint32_t)a.ids[i];
    if ((int64_t)k >= a.n_inst || !a.imask[k]) return -1;
    int64_t r = a.buffer_offset;
    if constexpr (OFFSETS) r += (int64_t)(uint32_t)a.per_inst_off[k] + (int64_t)(uint32_t)a.gs_inst_off[i];
    else r += i;
    return (r >= 0 && r < a.n_out) ? r : -1;
}

XSG_DEV f3 q_rot(float4 q, f3 p) { return quat_apply(q.x, mk3(q.y, q.z, q.w), p); }

XSG_DEV float4 q_mul(float4 a, float4 b) {
    const f3 av = mk3(a.y, a.z, a.w), bv = mk3(b.y, b.z, b.w);
    const f3 v = a.x * bv + b.x * av + cross(av, bv);
    return make_float4(a.x * b.x - dot(av, bv), v.x, v.y, v.z);
}

// copy_gs_rigid_transform_fwd_kernel (container.cu:13-75)
template <bool OFFSETS>
__global__ __launch_bounds__(kBlock) void rigid_fwd_kernel(RigidArgs a, float* __restrict__ out_pos,
                                                           float4* __restrict__ out_rot, float* __restrict__ out_vel,
                                                           uint8_t* __restrict__ out_mask) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= a.n) return;
    uint32_t k;
    const int64_t r = rigid_row<OFFSETS>(a, i, k);
    if (r < 0) return;
    const float4 q = a.iq[k];
    const f3 pr = q_rot(q, ld3(a.pos + 3 * i));
    st3(out_pos + 3 * r, pr + ld3(a.it + 3 * k));
    out_rot[r] = q_mul(q, a.rot[i]);
    if (out_vel) st3(out_vel + 3 * r, ld3(a.iv + 3 * k) + cross(ld3(a.iw + 3 * k), pr));
    if (out_mask) out_mask[r] = 1;
}

__global__ __launch_bounds__(kBlock) void zero_kernel(float* __restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i < n) p[i] = 0.f;
}

// Per-instance gradient sums live in 64-byte slots of a workspace, [n_inst][16] floats: q (4), t, v,
// w (3 each), 3 unused. One slot per instance keeps an instance's 13 atomics in one cache segment;
// packing the four sums densely (4 and 3 floats per instance) put many instances on each cache line
// and made the atomics about ten times slower.
constexpr int kSlot = 16;

// copy_gs_rigid_transform_bwd_kernel (container.cu:78-160). Per-Gaussian gradients are written for
// every Gaussian (zeros where skipped). The 13 per-instance values are summed across the wavefront
// per instance (Gaussians are usually stored instance by instance, so a wavefront holds one or two)
// and added by one 13-lane atomic instruction per instance.
template <bool OFFSETS>
__global__ __launch_bounds__(kBlock) void rigid_bwd_kernel(RigidArgs a, const float* __restrict__ v_pos,
                                                           const float4* __restrict__ v_rot,
                                                           const float* __restrict__ v_vel,
                                                           float* __restrict__ g_pos, float4* __restrict__ g_rot,
                                                           float* __restrict__ slots) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    float c[13];
#pragma unroll
    for (int j = 0; j < 13; ++j) c[j] = 0.f;
    uint32_t k = 0;
    int64_t r = -1;
    if (i < a.n) {
        r = rigid_row<OFFSETS>(a, i, k);
        f3 dp = mk3(0.f, 0.f, 0.f);
        float4 dr = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r >= 0) {
            const float4 q = a.iq[k];
            const f3 u = mk3(q.y, q.z, q.w);
            const f3 p = ld3(a.pos + 3 * i);
            const f3 g = ld3(v_pos + 3 * r);
            c[4] = g.x; c[5] = g.y; c[6] = g.z;
            f3 gp = g;
            if (v_vel) {
                const f3 gv = ld3(v_vel + 3 * r);
                const f3 gw = cross(q_rot(q, p), gv);
                c[7] = gv.x; c[8] = gv.y; c[9] = gv.z;
                c[10] = gw.x; c[11] = gw.y; c[12] = gw.z;
                gp = gp + cross(gv, ld3(a.iw + 3 * k));
            }
            // y = p + 2 (w (u x p) + u x (u x p))
            dp = gp - (2.0f * q.x) * cross(u, gp) + 2.0f * cross(u, cross(u, gp));
            const float dw = 2.0f * dot(gp, cross(u, p));
            const f3 du = (2.0f * q.x) * cross(p, gp) + (2.0f * dot(gp, u)) * p + (2.0f * dot(u, p)) * gp -
                          (4.0f * dot(gp, p)) * u;
            // out_rot = q (x) b
            const float4 b = a.rot[i];
            const f3 bv = mk3(b.y, b.z, b.w);
            const float4 vr = v_rot[r];
            const f3 dqv = mk3(vr.y, vr.z, vr.w);
            const float daw = vr.x * b.x + dot(dqv, bv);
            const f3 dav = b.x * dqv - vr.x * bv + cross(bv, dqv);
            const f3 dbv = q.x * dqv - vr.x * u + cross(dqv, u);
            dr = make_float4(vr.x * q.x + dot(dqv, u), dbv.x, dbv.y, dbv.z);
            c[0] = dw + daw; c[1] = du.x + dav.x; c[2] = du.y + dav.y; c[3] = du.z + dav.z;
        }
        st3(g_pos + 3 * i, dp);
        g_rot[i] = dr;
    }
    const int lane = __lane_id();
    const int nv = v_vel ? 13 : 7;  // without velocity gradients v and w stay 0
    uint64_t rem = __ballot(r >= 0);
    // one instance at a time: the lanes of the first remaining lane's instance are summed across the
    // wavefront and added by one 13-lane atomic; after kMaxRuns instances (shuffled Gaussians) the
    // remaining lanes add their own values
    constexpr int kMaxRuns = 4;
    for (int run = 0; run < kMaxRuns && rem != 0; ++run) {
        const uint32_t kk = (uint32_t)__builtin_amdgcn_readlane((int)k, __builtin_ctzll(rem));
        const bool in = ((rem >> lane) & 1) && k == kk;
        rem &= ~__ballot(in);
        float mine = 0.f;
#pragma unroll
        for (int j = 0; j < 13; ++j) {
            const float t = wave_sum(in ? c[j] : 0.f);
            mine = (lane == j) ? t : mine;
        }
        if (lane < nv) atomicAdd(slots + (int64_t)kk * kSlot + lane, mine);
    }
    if ((rem >> lane) & 1) {
        float* s = slots + (int64_t)k * kSlot;
#pragma unroll
        for (int j = 0; j < 13; ++j)
            if (j < nv) atomicAdd(s + j, c[j]);
    }
}

// the slots into the four per-instance outputs
__global__ __launch_bounds__(kBlock) void rigid_slots_out_kernel(const float* __restrict__ slots, int64_t n_inst,
                                                                 float* __restrict__ g_q, float* __restrict__ g_t,
                                                                 float* __restrict__ g_v, float* __restrict__ g_w) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n_inst * 13) return;
    const int64_t k = i / 13;
    const int j = (int)(i - k * 13);
    const float v = slots[k * kSlot + j];
    if (j < 4) g_q[4 * k + j] = v;
    else if (j < 7) g_t[3 * k + (j - 4)] = v;
    else if (j < 10) g_v[3 * k + (j - 7)] = v;
    else g_w[3 * k + (j - 10)] = v;
}

int rigid_args(const xsg_rigid_desc* d, RigidArgs& a, const char* who) {
    if (!d) return xsg_fail(XSG_ERR_INVALID, "%s: null descriptor", who);
    if (d->n < 0 || d->n_instances < 0 || d->n_out < 0 || d->buffer_offset < 0)
        return xsg_fail(XSG_ERR_INVALID, "%s: negative size", who);
    if ((d->per_instance_offsets == nullptr) != (d->gs_inst_offsets == nullptr))
        return xsg_fail(XSG_ERR_INVALID, "%s: per_instance_offsets and gs_inst_offsets go together", who);
    if (d->n > 0 && (!d->positions || !d->rotations || !d->instance_ids || !d->inst_q || !d->inst_mask))
        return xsg_fail(XSG_ERR_INVALID, "%s: null tensor", who);
    if (reinterpret_cast<uintptr_t>(d->rotations) % 16 || reinterpret_cast<uintptr_t>(d->inst_q) % 16)
        return xsg_fail(XSG_ERR_INVALID, "%s: quaternion arrays must be 16-byte aligned", who);
    a = RigidArgs{d->n, d->n_instances, d->n_out, d->buffer_offset, d->positions,
                  reinterpret_cast<const float4*>(d->rotations), d->instance_ids,
                  reinterpret_cast<const float4*>(d->inst_q), d->inst_t, d->inst_v, d->inst_w, d->inst_mask,
                  d->per_instance_offsets, d->gs_inst_offsets};
    return XSG_OK;
}

// The caller's parameter activations in one launch each way: the 3n scales (exp of their logs) and
// the n opacities (sigmoid of the logits) as one range of chunks of four values, the scales' chunks
// first; the backward multiplies each gradient by its activation's derivative, written from the
// outputs as exp(x)' = exp(x) and sigmoid(x)' = sigmoid(x) (1 - sigmoid(x)). The float expressions
// and their order are those of torch's exp, sigmoid, mul and sigmoid_backward kernels, so the results
// are the same bits. VEC: every array 16-byte aligned, whole chunks move as one 16-byte access.
XSG_DEV float act_exp(float a) { return expf(a); }
XSG_DEV float act_sigmoid(float a) { return 1.0f / (1.0f + expf(-a)); }

template <bool VEC, typename F>
XSG_DEV void act_chunk(const float* __restrict__ x, float* __restrict__ y, int64_t i0, int64_t n, F f) {
    if (VEC && i0 + 4 <= n) {
        const float4 a = *reinterpret_cast<const float4*>(x + i0);
        *reinterpret_cast<float4*>(y + i0) = make_float4(f(a.x), f(a.y), f(a.z), f(a.w));
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (i0 + k < n) y[i0 + k] = f(x[i0 + k]);
    }
}

template <bool VEC, typename F>
XSG_DEV void act_grad_chunk(const float* __restrict__ v, const float* __restrict__ y, float* __restrict__ out,
                            int64_t i0, int64_t n, F f) {
    if (VEC && i0 + 4 <= n) {
        const float4 a = *reinterpret_cast<const float4*>(v + i0);
        const float4 b = *reinterpret_cast<const float4*>(y + i0);
        *reinterpret_cast<float4*>(out + i0) = make_float4(f(a.x, b.x), f(a.y, b.y), f(a.z, b.z), f(a.w, b.w));
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (i0 + k < n) out[i0 + k] = f(v[i0 + k], y[i0 + k]);
    }
}

template <bool VEC>
__global__ __launch_bounds__(kBlock) void activate_fwd_kernel(int64_t n3, int64_t n,
                                                              const float* __restrict__ log_scales,
                                                              const float* __restrict__ logits,
                                                              float* __restrict__ scales,
                                                              float* __restrict__ opacities) {
    const int64_t q = (int64_t)blockIdx.x * kBlock + threadIdx.x, q3 = (n3 + 3) >> 2;
    if (q < q3)
        act_chunk<VEC>(log_scales, scales, 4 * q, n3, act_exp);
    else
        act_chunk<VEC>(logits, opacities, 4 * (q - q3), n, act_sigmoid);
}

template <bool VEC>
__global__ __launch_bounds__(kBlock) void activate_bwd_kernel(int64_t n3, int64_t n,
                                                              const float* __restrict__ scales,
                                                              const float* __restrict__ opacities,
                                                              const float* __restrict__ v_scales,
                                                              const float* __restrict__ v_opacities,
                                                              float* __restrict__ v_log_scales,
                                                              float* __restrict__ v_logits) {
    const int64_t q = (int64_t)blockIdx.x * kBlock + threadIdx.x, q3 = (n3 + 3) >> 2;
    if (q < q3) {
        if (v_scales) act_grad_chunk<VEC>(v_scales, scales, v_log_scales, 4 * q, n3, [](float a, float b) { return a * b; });
    } else if (v_opacities) {
        act_grad_chunk<VEC>(v_opacities, opacities, v_logits, 4 * (q - q3), n,
                            [](float a, float b) { return a * (1.0f - b) * b; });
    }
}

}  // namespace

extern "C" int xsg_packed_mask_from_instances(int64_t n, const int32_t* instance_ids, const uint8_t* instance_mask,
                                              int64_t n_instances, uint32_t* out, xsg_stream_t stream) {
    if (n < 0 || n_instances < 0) return xsg_fail(XSG_ERR_INVALID, "packed_mask_from_instances: negative size");
    if (n == 0) return XSG_OK;
    if (!instance_ids || !out || (n_instances > 0 && !instance_mask))
        return xsg_fail(XSG_ERR_INVALID, "packed_mask_from_instances: null tensor");
    packed_mask_kernel<<<xsg_blocks(n, kBlock), kBlock, 0, (hipStream_t)stream>>>(n, instance_ids, instance_mask,
                                                                                  n_instances, out);
    XSG_TRY_LAUNCH("packed_mask_from_instances");
    return XSG_OK;
}

extern "C" int xsg_rigid_transform_fwd(const xsg_rigid_desc* d, float* out_positions, float* out_rotations,
                                       float* out_velocities, uint8_t* out_mask, xsg_stream_t stream) {
    RigidArgs a;
    const int rc = rigid_args(d, a, "copy_gs_rigid_transform_fwd");
    if (rc != XSG_OK) return rc;
    if (a.n == 0) return XSG_OK;
    if (!d->inst_t || !d->inst_v || !d->inst_w || !out_positions || !out_rotations)
        return xsg_fail(XSG_ERR_INVALID, "copy_gs_rigid_transform_fwd: null tensor");
    if (reinterpret_cast<uintptr_t>(out_rotations) % 16)
        return xsg_fail(XSG_ERR_INVALID, "copy_gs_rigid_transform_fwd: out_rotations must be 16-byte aligned");
    const hipStream_t s = (hipStream_t)stream;
    auto orot = reinterpret_cast<float4*>(out_rotations);
    if (a.gs_inst_off)
        rigid_fwd_kernel<true><<<xsg_blocks(a.n, kBlock), kBlock, 0, s>>>(a, out_positions, orot, out_velocities,
                                                                          out_mask);
    else
        rigid_fwd_kernel<false><<<xsg_blocks(a.n, kBlock), kBlock, 0, s>>>(a, out_positions, orot, out_velocities,
                                                                           out_mask);
    XSG_TRY_LAUNCH("copy_gs_rigid_transform_fwd");
    return XSG_OK;
}

extern "C" size_t xsg_rigid_transform_bwd_workspace_bytes(int64_t n_instances) {
    return sizeof(float) * kSlot * (size_t)(n_instances > 0 ? n_instances : 1);
}

extern "C" int xsg_rigid_transform_bwd(const xsg_rigid_desc* d, const float* v_positions, const float* v_rotations,
                                       const float* v_velocities, float* grad_positions, float* grad_rotations,
                                       float* grad_q, float* grad_t, float* grad_v, float* grad_w, void* workspace,
                                       xsg_stream_t stream) {
    RigidArgs a;
    const int rc = rigid_args(d, a, "copy_gs_rigid_transform_bwd");
    if (rc != XSG_OK) return rc;
    if (a.n_inst > 0 && (!grad_q || !grad_t || !grad_v || !grad_w || !workspace))
        return xsg_fail(XSG_ERR_INVALID, "copy_gs_rigid_transform_bwd: null instance gradient or workspace");
    if (const int rc2 = xsg_check_workspace(workspace, "copy_gs_rigid_transform_bwd")) return rc2;
    if (a.n > 0 && (!d->inst_w || !v_positions || !v_rotations || !grad_positions || !grad_rotations))
        return xsg_fail(XSG_ERR_INVALID, "copy_gs_rigid_transform_bwd: null tensor");
    if (reinterpret_cast<uintptr_t>(v_rotations) % 16 || reinterpret_cast<uintptr_t>(grad_rotations) % 16)
        return xsg_fail(XSG_ERR_INVALID, "copy_gs_rigid_transform_bwd: quaternion arrays must be 16-byte aligned");
    const hipStream_t s = (hipStream_t)stream;
    const int64_t ni = a.n_inst;
    float* slots = static_cast<float*>(workspace);
    // the slots start at zero (a fill kernel, so that the call can be graph-captured)
    if (ni > 0) zero_kernel<<<xsg_blocks(kSlot * ni, kBlock), kBlock, 0, s>>>(slots, kSlot * ni);
    if (a.n > 0) {
        auto vr = reinterpret_cast<const float4*>(v_rotations);
        auto gr = reinterpret_cast<float4*>(grad_rotations);
        if (a.gs_inst_off)
            rigid_bwd_kernel<true><<<xsg_blocks(a.n, kBlock), kBlock, 0, s>>>(a, v_positions, vr, v_velocities,
                                                                             grad_positions, gr, slots);
        else
            rigid_bwd_kernel<false><<<xsg_blocks(a.n, kBlock), kBlock, 0, s>>>(a, v_positions, vr, v_velocities,
                                                                              grad_positions, gr, slots);
    }
    if (ni > 0)
        rigid_slots_out_kernel<<<xsg_blocks(13 * ni, kBlock), kBlock, 0, s>>>(slots, ni, grad_q, grad_t, grad_v,
                                                                             grad_w);
    XSG_TRY_LAUNCH("copy_gs_rigid_transform_bwd");
    return XSG_OK;
}

static bool aligned16(std::initializer_list<const void*> ps) {  // NULL counts as aligned
    for (const void* p : ps)
        if (reinterpret_cast<uintptr_t>(p) % 16) return false;
    return true;
}

extern "C" int xsg_packed_visibility_from_radii(int64_t n, int n_cams, const float* radii, uint32_t* out,
                                                xsg_stream_t stream) {
    if (n < 0 || n_cams < 1) return xsg_fail(XSG_ERR_INVALID, "packed_visibility_from_radii: bad sizes");
    if (n == 0) return XSG_OK;
    if (!radii || !out) return xsg_fail(XSG_ERR_INVALID, "packed_visibility_from_radii: null tensor");
    packed_visibility_kernel<<<xsg_blocks(n, kBlock), kBlock, 0, (hipStream_t)stream>>>(
        n, n_cams, reinterpret_cast<const float2*>(radii), out);
    XSG_TRY_LAUNCH("packed_visibility_from_radii");
    return XSG_OK;
}

extern "C" int xsg_activate_fwd(int64_t n, const float* log_scales, const float* opacity_logits, float* scales,
                                float* opacities, xsg_stream_t stream) {
    if (n < 0) return xsg_fail(XSG_ERR_INVALID, "activate_fwd: negative size");
    if (n == 0) return XSG_OK;
    if (!log_scales || !opacity_logits || !scales || !opacities)
        return xsg_fail(XSG_ERR_INVALID, "activate_fwd: null tensor");
    const unsigned grid = xsg_blocks((3 * n + 3) / 4 + (n + 3) / 4, kBlock);
    const hipStream_t s = (hipStream_t)stream;
    if (aligned16({log_scales, opacity_logits, scales, opacities}))
        activate_fwd_kernel<true><<<grid, kBlock, 0, s>>>(3 * n, n, log_scales, opacity_logits, scales, opacities);
    else
        activate_fwd_kernel<false><<<grid, kBlock, 0, s>>>(3 * n, n, log_scales, opacity_logits, scales, opacities);
    XSG_TRY_LAUNCH("activate_fwd");
    return XSG_OK;
}

extern "C" int xsg_activate_bwd(int64_t n, const float* scales, const float* opacities, const float* v_scales,
                                const float* v_opacities, float* v_log_scales, float* v_opacity_logits,
                                xsg_stream_t stream) {
    if (n < 0) return xsg_fail(XSG_ERR_INVALID, "activate_bwd: negative size");
    if (n == 0 || (!v_scales && !v_opacities)) return XSG_OK;
    if ((v_scales && (!scales || !v_log_scales)) || (v_opacities && (!opacities || !v_opacity_logits)))
        return xsg_fail(XSG_ERR_INVALID, "activate_bwd: null tensor");
    const unsigned grid = xsg_blocks((3 * n + 3) / 4 + (n + 3) / 4, kBlock);
    const hipStream_t s = (hipStream_t)stream;
    if (aligned16({scales, opacities, v_scales, v_opacities, v_log_scales, v_opacity_logits}))
        activate_bwd_kernel<true><<<grid, kBlock, 0, s>>>(3 * n, n, scales, opacities, v_scales, v_opacities,
                                                          v_log_scales, v_opacity_logits);
    else
        activate_bwd_kernel<false><<<grid, kBlock, 0, s>>>(3 * n, n, scales, opacities, v_scales, v_opacities,
                                                           v_log_scales, v_opacity_logits);
    XSG_TRY_LAUNCH("activate_bwd");
    return XSG_OK;
}
