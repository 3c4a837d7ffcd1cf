// xsimgs_amd._C: the reference's pybind surface (xsimgs._C, csrc/ext.cpp:12-20) re-exported over the
// xsimgs_amd C-ABI. This file validates and allocates exactly as the reference ops do, then calls
// the HIP kernels through include/xsimgs_amd.h on the current stream of the input's device.
#include <torch/extension.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <optional>
#include <string>
#include <vector>

#include "../../include/xsimgs_amd.h"
#include "../../include/xsimgs_amd_bench.h"

namespace {

using at::Tensor;
using OptT = std::optional<Tensor>;

void check_rc(int rc) {
    if (rc != XSG_OK) throw std::runtime_error(xsg_last_error());
}

xsg_stream_t stream_of(const Tensor& t) {
    TORCH_CHECK(t.is_cuda(), "xsimgs_amd ops take GPU tensors (got a tensor on ", t.device(), ")");
    return reinterpret_cast<xsg_stream_t>(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream());
}

const float* fptr(const Tensor& t) { return t.data_ptr<float>(); }
const float* fptr(const OptT& t) { return t.has_value() ? t->data_ptr<float>() : nullptr; }

void check_f32(const Tensor& t, const char* name) {
    TORCH_CHECK(t.scalar_type() == at::kFloat, name, " must be a float32 tensor");
}

void check_same_device(const std::vector<Tensor>& ts) {  // toast check_same_device
    for (size_t i = 1; i < ts.size(); ++i)
        TORCH_CHECK(ts[i].device() == ts[0].device(), "All tensors must be on the same device");
}

void all_contiguous(const std::vector<Tensor>& ts) {  // toast all_contiguous
    for (const auto& t : ts) TORCH_CHECK(t.is_contiguous(), "All tensors must be contiguous");
}

Tensor workspace(const Tensor& like, size_t bytes) {
    return at::empty({(int64_t)std::max<size_t>(bytes, 1)}, like.options().dtype(at::kByte));
}

// ------------------------------------------------------------------ compositing
std::vector<int> eval3d_supported_ndims() {
    int dims[64];
    const int n = xsg_eval3d_supported_ndims(dims, 64);
    return std::vector<int>(dims, dims + n);
}

// Camera batch of a compositor call: the reference composites one camera per call; the batched ops
// (an extension of this build) take C cameras over one scene with rays [C, H, W, 3], tile offsets
// [C, th, tw] and flatten ids cam * N + gaussian (isect_regular_tiles_batched), and colours either
// per camera [C, N, ch] or shared by every camera [N, ch].
struct CamBatch {
    int64_t n_cams = 1;
    bool batched = false, colors_shared = false;
};

CamBatch cam_batch(bool batched, const Tensor& means, const OptT& colors, const Tensor& ray_o,
                   const Tensor& ray_d, const Tensor& offsets, const OptT& ray_time_delta) {
    CamBatch b;
    if (!batched) return b;
    b.batched = true;
    TORCH_CHECK(ray_o.dim() == 4 && ray_o.size(3) == 3 && ray_d.sizes() == ray_o.sizes(),
                "batched compositing takes rays [C, H, W, 3]");
    b.n_cams = ray_o.size(0);
    TORCH_CHECK(b.n_cams >= 1, "batched compositing needs at least one camera");
    TORCH_CHECK(offsets.dim() == 3 && offsets.size(0) == b.n_cams, "tile_offsets must be [C, tile_height, tile_width]");
    if (ray_time_delta.has_value())
        TORCH_CHECK(ray_time_delta->numel() == ray_o.numel() / 3, "ray_time_delta must be [C, H, W]");
    const int64_t n = means.numel() / 3;
    if (colors.has_value()) {
        const Tensor& c = *colors;
        if (c.dim() == 2) {
            TORCH_CHECK(c.size(0) == n, "shared colors must be [N, channels]");
            b.colors_shared = true;
        } else {
            TORCH_CHECK(c.dim() == 3 && c.size(0) == b.n_cams && c.size(1) == n,
                        "colors must be [C, N, channels] or [N, channels]");
        }
    }
    return b;
}

xsg_eval3d_args base_args(const Tensor& means, const Tensor& quats, const Tensor& scales, const OptT& colors,
                          const Tensor& opac, int cdim, int width, int height, int tw, int th,
                          const Tensor& ray_o, const Tensor& ray_d, const Tensor& offsets, const Tensor& flat,
                          const CamBatch& cb = CamBatch{}) {
    for (const Tensor* t : {&means, &quats, &scales, &opac, &ray_o, &ray_d}) check_f32(*t, "Gaussian / ray tensors");
    TORCH_CHECK(offsets.scalar_type() == at::kInt && flat.scalar_type() == at::kInt,
                "tile_offsets and flatten_ids must be int32");
    all_contiguous({means, quats, scales, opac, ray_o, ray_d, offsets, flat});
    if (colors.has_value()) { check_f32(*colors, "colors"); all_contiguous({*colors}); }
    xsg_eval3d_args a{};
    a.cdim = cdim;
    a.n = means.numel() / 3;
    a.n_cams = (int)cb.n_cams;
    a.colors_shared = cb.colors_shared ? 1 : 0;
    a.means = fptr(means); a.quats = fptr(quats); a.scales = fptr(scales);
    a.colors = fptr(colors); a.opacities = fptr(opac);
    a.ray_o = fptr(ray_o); a.ray_d = fptr(ray_d);
    a.width = width; a.height = height; a.tile_w = tw; a.tile_h = th;
    a.n_tiles_w = (int)offsets.size(-1);
    a.n_tiles_h = (int)offsets.size(-2);
    a.tile_offsets = offsets.data_ptr<int32_t>();
    a.flatten_ids = flat.data_ptr<int32_t>();
    a.n_isects = flat.numel();
    return a;
}

// optional int32 device tensor of one value per (camera, tile): the backward's work estimates, written
// by the forward and read by the backward (an extension of this build)
int32_t* tile_work_ptr(const OptT& tile_work, const Tensor& offsets) {
    if (!tile_work.has_value()) return nullptr;
    TORCH_CHECK(tile_work->scalar_type() == at::kInt && tile_work->is_contiguous() &&
                    tile_work->numel() == offsets.numel() && tile_work->device() == offsets.device(),
                "tile_work must be a contiguous int32 tensor of one value per (camera, tile) on the offsets' device");
    return tile_work->data_ptr<int32_t>();
}

// optional int64[2] device tensor of evaluated / composited pair counts (an extension of this build)
uint64_t* counts_ptr(const OptT& pair_counts, const Tensor& like) {
    if (!pair_counts.has_value()) return nullptr;
    TORCH_CHECK(pair_counts->scalar_type() == at::kLong && pair_counts->numel() >= 2 && pair_counts->is_contiguous() &&
                    pair_counts->device() == like.device(),
                "pair_counts must be a contiguous int64 tensor of 2 elements on the Gaussians' device");
    return reinterpret_cast<uint64_t*>(pair_counts->data_ptr<int64_t>());
}

// rasterize_eval3d_fwd (eval3d_fwd.cu:248-316) and its dynamic twin (eval3d_dynamic_fwd.cu:249-332)
std::tuple<Tensor, Tensor, Tensor, Tensor> eval3d_fwd_impl(
    const Tensor& means, const OptT& velocity, const Tensor& quats, const Tensor& scales, const OptT& colors,
    const Tensor& opacities, int64_t image_width, int64_t image_height, int64_t tsw, int64_t tsh,
    const Tensor& ray_origs, const Tensor& ray_dirs, const OptT& ray_time_delta, const Tensor& tile_offsets,
    const Tensor& flatten_ids, const OptT& pair_counts, const OptT& tile_work, bool batched = false) {
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(means.device());
    auto opt = means.options();
    const int64_t channels = colors.has_value() ? colors->size(-1) : 0;
    const CamBatch cb = cam_batch(batched, means, colors, ray_origs, ray_dirs, tile_offsets, ray_time_delta);
    if (batched)
        TORCH_CHECK(ray_origs.size(1) == image_height && ray_origs.size(2) == image_width,
                    "rays must be [C, image_height, image_width, 3]");
    std::vector<int64_t> hw{image_height, image_width};
    if (batched) hw.insert(hw.begin(), cb.n_cams);
    std::vector<int64_t> hwc = hw;
    hwc.push_back(channels);
    Tensor renders = at::empty(hwc, opt);
    Tensor depths = at::empty(hw, opt);
    Tensor alphas = at::empty(hw, opt);
    Tensor last_ids = at::empty(hw, opt.dtype(at::kInt));
    xsg_eval3d_args a = base_args(means, quats, scales, colors, opacities, (int)channels, (int)image_width,
                                  (int)image_height, (int)tsw, (int)tsh, ray_origs, ray_dirs, tile_offsets,
                                  flatten_ids, cb);
    if (velocity.has_value()) { check_f32(*velocity, "velocity"); all_contiguous({*velocity}); }
    if (ray_time_delta.has_value()) { check_f32(*ray_time_delta, "ray_time_delta"); all_contiguous({*ray_time_delta}); }
    a.velocity = fptr(velocity);
    a.ray_time_delta = fptr(ray_time_delta);
    a.out_rgb = renders.data_ptr<float>(); a.out_depth = depths.data_ptr<float>();
    a.out_alpha = alphas.data_ptr<float>(); a.out_last_ids = last_ids.data_ptr<int32_t>();
    a.pair_counts = counts_ptr(pair_counts, means);
    a.tile_work = tile_work_ptr(tile_work, tile_offsets);
    check_rc(xsg_eval3d_fwd(&a, stream_of(means)));
    return {renders, depths, alphas, last_ids};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> rasterize_eval3d_fwd(
    const Tensor& means, const Tensor& quats, const Tensor& scales, const OptT& colors, const Tensor& opacities,
    int64_t image_width, int64_t image_height, int64_t tile_size_width, int64_t tile_size_height,
    const Tensor& ray_origs, const Tensor& ray_dirs, const Tensor& tile_offsets, const Tensor& flatten_ids,
    const OptT& pair_counts, const OptT& tile_work) {
    return eval3d_fwd_impl(means, std::nullopt, quats, scales, colors, opacities, image_width, image_height,
                           tile_size_width, tile_size_height, ray_origs, ray_dirs, std::nullopt, tile_offsets,
                           flatten_ids, pair_counts, tile_work);
}

// batched cameras (extension): outputs [C, H, W, ch], [C, H, W] x2, last ids [C, H, W]
std::tuple<Tensor, Tensor, Tensor, Tensor> rasterize_eval3d_fwd_batched(
    const Tensor& means, const Tensor& quats, const Tensor& scales, const OptT& colors, const Tensor& opacities,
    int64_t image_width, int64_t image_height, int64_t tile_size_width, int64_t tile_size_height,
    const Tensor& ray_origs, const Tensor& ray_dirs, const Tensor& tile_offsets, const Tensor& flatten_ids,
    const OptT& velocity, const OptT& ray_time_delta, const OptT& pair_counts, const OptT& tile_work) {
    TORCH_CHECK(velocity.has_value() == ray_time_delta.has_value(),
                "dynamic compositing needs both velocity and ray_time_delta");
    return eval3d_fwd_impl(means, velocity, quats, scales, colors, opacities, image_width, image_height,
                           tile_size_width, tile_size_height, ray_origs, ray_dirs, ray_time_delta, tile_offsets,
                           flatten_ids, pair_counts, tile_work, true);
}

std::tuple<Tensor, Tensor, Tensor, Tensor> rasterize_eval3d_dynamic_fwd(
    const Tensor& means, const OptT& velocity, const Tensor& quats, const Tensor& scales, const OptT& colors,
    const Tensor& opacities, int64_t image_width, int64_t image_height, int64_t tile_size_width,
    int64_t tile_size_height, const Tensor& ray_origs, const Tensor& ray_dirs, const OptT& ray_time_delta,
    const Tensor& tile_offsets, const Tensor& flatten_ids, const OptT& pair_counts, const OptT& tile_work) {
    return eval3d_fwd_impl(means, velocity, quats, scales, colors, opacities, image_width, image_height,
                           tile_size_width, tile_size_height, ray_origs, ray_dirs, ray_time_delta, tile_offsets,
                           flatten_ids, pair_counts, tile_work);
}

struct BwdOut {
    Tensor v_points, v_velocity, v_quat, v_scale, v_opacity;
    std::optional<Tensor> v_colors;
    std::optional<Tensor> v_ray_o, v_ray_d;
    Tensor v_time_delta;
};

// rasterize_eval3d_bwd (eval3d_bwd.cu:297-403) / rasterize_eval3d_dynamic_bwd (eval3d_dynamic_bwd.cu:312-427)
BwdOut eval3d_bwd_impl(const Tensor& points, const OptT& velocity, const Tensor& scale, const Tensor& quat,
                       const Tensor& opacity, const OptT& colors, const Tensor& ray_origins,
                       const Tensor& ray_directions, const OptT& ray_time_delta, int64_t tile_size_x,
                       int64_t tile_size_y, const Tensor& tile_offsets, const Tensor& flatten_ids,
                       const Tensor& render_alpha, const Tensor& last_ids, const OptT& v_render_colors,
                       const Tensor& v_render_depth, const Tensor& v_render_alpha, bool ray_grads,
                       const OptT& pair_counts, int64_t pixels_per_lane, const OptT& tile_work,
                       bool batched = false) {
    if (v_render_colors.has_value() && !v_render_colors->is_contiguous())
        throw std::runtime_error("v_render_colors must be contiguous");
    all_contiguous({v_render_depth, v_render_alpha, render_alpha, last_ids});
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(points.device());
    const CamBatch cb = cam_batch(batched, points, colors, ray_origins, ray_directions, tile_offsets,
                                  ray_time_delta);
    const int64_t width = ray_origins.size(batched ? 2 : 1), height = ray_origins.size(batched ? 1 : 0);
    const int64_t n_pix = cb.n_cams * width * height;
    TORCH_CHECK(render_alpha.numel() == n_pix && last_ids.numel() == n_pix && v_render_depth.numel() == n_pix &&
                    v_render_alpha.numel() == n_pix,
                "render_alpha, last_ids and the depth / alpha gradients must hold one value per ray");
    BwdOut o;
    // every gradient buffer is zero-filled (or fully written) by xsg_eval3d_bwd itself
    o.v_points = at::empty_like(points);
    o.v_scale = at::empty_like(scale);
    o.v_quat = at::empty_like(quat);
    o.v_opacity = at::empty_like(opacity);
    int cdim = 0;
    if (colors.has_value()) {
        o.v_colors = at::empty_like(*colors);
        cdim = (int)colors->size(-1);
        if (v_render_colors.has_value())
            TORCH_CHECK(v_render_colors->numel() == n_pix * cdim, "v_render_colors must be [.., H, W, channels]");
    }
    // ray gradients are skipped when the caller does not need them (only kernels with CDIM <= 16
    // have that variant; larger CDIMs always produce them)
    if (ray_grads || cdim > 16) {
        o.v_ray_o = at::empty_like(ray_origins);
        o.v_ray_d = at::empty_like(ray_directions);
    }
    xsg_eval3d_args a = base_args(points, quat, scale, colors, opacity, cdim, (int)width, (int)height,
                                  (int)tile_size_x, (int)tile_size_y, ray_origins, ray_directions, tile_offsets,
                                  flatten_ids, cb);
    if (velocity.has_value()) {
        check_f32(*velocity, "velocity");
        all_contiguous({*velocity, *ray_time_delta});
        o.v_velocity = at::empty_like(*velocity);
        o.v_time_delta = at::empty_like(*ray_time_delta);
        a.velocity = fptr(velocity);
        a.ray_time_delta = fptr(ray_time_delta);
        a.v_velocity = o.v_velocity.data_ptr<float>();
        a.v_time_delta = o.v_time_delta.data_ptr<float>();
    }
    a.render_alpha = fptr(render_alpha);
    a.last_ids = last_ids.data_ptr<int32_t>();
    a.v_rgb = fptr(v_render_colors);
    a.v_depth = fptr(v_render_depth);
    a.v_alpha = fptr(v_render_alpha);
    a.v_means = o.v_points.data_ptr<float>();
    a.v_quats = o.v_quat.data_ptr<float>();
    a.v_scales = o.v_scale.data_ptr<float>();
    a.v_opacities = o.v_opacity.data_ptr<float>();
    a.v_colors = o.v_colors.has_value() ? o.v_colors->data_ptr<float>() : nullptr;
    a.v_ray_o = o.v_ray_o.has_value() ? o.v_ray_o->data_ptr<float>() : nullptr;
    a.v_ray_d = o.v_ray_d.has_value() ? o.v_ray_d->data_ptr<float>() : nullptr;
    a.pair_counts = counts_ptr(pair_counts, points);
    a.bwd_pixels_per_lane = (int)pixels_per_lane;
    a.tile_work = tile_work_ptr(tile_work, tile_offsets);
    Tensor ws = workspace(points, xsg_eval3d_bwd_workspace_bytes(&a));
    check_rc(xsg_eval3d_bwd(&a, ws.data_ptr(), stream_of(points)));
    return o;
}

std::tuple<Tensor, Tensor, Tensor, Tensor, OptT, OptT, OptT> rasterize_eval3d_bwd(
    const Tensor& points, const Tensor& scale, const Tensor& quat, const Tensor& opacity, const OptT& colors,
    const Tensor& ray_origins, const Tensor& ray_directions, int64_t tile_size_x, int64_t tile_size_y,
    const Tensor& tile_offsets, const Tensor& flatten_ids, const Tensor& render_alpha, const Tensor& last_ids,
    const OptT& v_render_colors, const Tensor& v_render_depth, const Tensor& v_render_alpha, bool ray_grads,
    const OptT& pair_counts, int64_t pixels_per_lane, const OptT& tile_work) {
    BwdOut o = eval3d_bwd_impl(points, std::nullopt, scale, quat, opacity, colors, ray_origins, ray_directions,
                               std::nullopt, tile_size_x, tile_size_y, tile_offsets, flatten_ids, render_alpha,
                               last_ids, v_render_colors, v_render_depth, v_render_alpha, ray_grads, pair_counts,
                               pixels_per_lane, tile_work);
    return {o.v_points, o.v_quat, o.v_scale, o.v_opacity, o.v_colors, o.v_ray_o, o.v_ray_d};
}

// batched cameras (extension): (v_points, v_quat, v_scale, v_opacity, v_colors, v_ray_o, v_ray_d,
// v_velocity, v_time_delta); v_colors has the colours' shape ([N, ch] shared: summed over cameras)
std::tuple<Tensor, Tensor, Tensor, Tensor, OptT, OptT, OptT, OptT, OptT> rasterize_eval3d_bwd_batched(
    const Tensor& points, const Tensor& scale, const Tensor& quat, const Tensor& opacity, const OptT& colors,
    const Tensor& ray_origins, const Tensor& ray_directions, int64_t tile_size_x, int64_t tile_size_y,
    const Tensor& tile_offsets, const Tensor& flatten_ids, const Tensor& render_alpha, const Tensor& last_ids,
    const OptT& v_render_colors, const Tensor& v_render_depth, const Tensor& v_render_alpha,
    const OptT& velocity, const OptT& ray_time_delta, bool ray_grads, const OptT& pair_counts,
    int64_t pixels_per_lane, const OptT& tile_work) {
    TORCH_CHECK(velocity.has_value() == ray_time_delta.has_value(),
                "dynamic compositing needs both velocity and ray_time_delta");
    BwdOut o = eval3d_bwd_impl(points, velocity, scale, quat, opacity, colors, ray_origins, ray_directions,
                               ray_time_delta, tile_size_x, tile_size_y, tile_offsets, flatten_ids, render_alpha,
                               last_ids, v_render_colors, v_render_depth, v_render_alpha, ray_grads, pair_counts,
                               pixels_per_lane, tile_work, true);
    const bool dyn = velocity.has_value();
    return {o.v_points, o.v_quat, o.v_scale, o.v_opacity, o.v_colors, o.v_ray_o, o.v_ray_d,
            dyn ? OptT(o.v_velocity) : std::nullopt, dyn ? OptT(o.v_time_delta) : std::nullopt};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, OptT, OptT, OptT, Tensor> rasterize_eval3d_dynamic_bwd(
    const Tensor& points, const Tensor& velocity, const Tensor& scale, const Tensor& quat, const Tensor& opacity,
    const OptT& colors, const Tensor& ray_origins, const Tensor& ray_directions, const Tensor& ray_time_delta,
    int64_t tile_size_x, int64_t tile_size_y, const Tensor& tile_offsets, const Tensor& flatten_ids,
    const Tensor& render_alpha, const Tensor& last_ids, const OptT& v_render_colors, const Tensor& v_render_depth,
    const Tensor& v_render_alpha, bool ray_grads, const OptT& pair_counts, int64_t pixels_per_lane,
    const OptT& tile_work) {
    BwdOut o = eval3d_bwd_impl(points, velocity, scale, quat, opacity, colors, ray_origins, ray_directions,
                               ray_time_delta, tile_size_x, tile_size_y, tile_offsets, flatten_ids, render_alpha,
                               last_ids, v_render_colors, v_render_depth, v_render_alpha, ray_grads, pair_counts,
                               pixels_per_lane, tile_work);
    return {o.v_points, o.v_velocity, o.v_quat, o.v_scale, o.v_opacity, o.v_colors, o.v_ray_o, o.v_ray_d,
            o.v_time_delta};
}

// ------------------------------------------------------------------ spherical harmonics
void sh_checks(int64_t degree, const Tensor& origin, const Tensor& positions, const Tensor& coeffs, const OptT& mask,
               bool layout_3kn, const OptT& coeffs_dc, int64_t& N, int64_t& dim) {
    std::vector<Tensor> ts{origin, positions, coeffs};
    if (coeffs_dc.has_value()) ts.push_back(*coeffs_dc);
    if (mask.has_value()) ts.push_back(*mask);
    check_same_device(ts);
    all_contiguous(ts);
    N = layout_3kn ? coeffs.size(2) : coeffs.size(0);
    dim = coeffs.size(1);
    TORCH_CHECK(coeffs.size(layout_3kn ? 0 : 2) == 3,
                "coeffs tensor must be [3, K, N] if layout_3kn else [N, K, 3]");
    if (degree < 0 || degree > 4)
        throw std::runtime_error("Unsupported spherical harmonics degree: " + std::to_string(degree));
    static const int64_t ref_dims[5] = {1, 4, 9, 16, 25};
    const bool has_dc = coeffs_dc.has_value();
    const int64_t required = ref_dims[degree] - (has_dc ? 1 : 0);
    TORCH_CHECK(dim >= required, "Number of harmonics band in coeffs tensor must be higher or equal than ",
                required, " for degree_to_use=", degree, has_dc ? " (zero-degree coeffs passed separately)" : "");
    if (has_dc) {
        const auto dc_dim = coeffs_dc->dim();
        TORCH_CHECK(dc_dim == 2 || dc_dim == 3, "coeffs_dc must be 2D or 3D");
        const int64_t ch_axis = layout_3kn ? 0 : dc_dim - 1;
        const int64_t n_axis = layout_3kn ? dc_dim - 1 : 0;
        TORCH_CHECK(coeffs_dc->size(ch_axis) == 3 && coeffs_dc->size(n_axis) == N && coeffs_dc->numel() == 3 * N,
                    "coeffs_dc must hold a single SH band: [N, 3] or [N, 1, 3] if "
                    "!layout_3kn else [3, N] or [3, 1, N]");
    }
}

// spherical_harmonics_fused_fwd (sh_fwd.cu:162-259)
Tensor spherical_harmonics_fused_fwd(int64_t degree_to_use, const Tensor& origin, const Tensor& positions,
                                     const Tensor& coeffs, const OptT& mask, bool layout_3kn, const OptT& coeffs_dc,
                                     const OptT& output) {
    int64_t N, dim;
    sh_checks(degree_to_use, origin, positions, coeffs, mask, layout_3kn, coeffs_dc, N, dim);
    if (output.has_value()) { check_same_device({origin, *output}); all_contiguous({*output}); }
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(positions.device());
    // masked rows keep a given output's values; a fresh output gets zeros there from the kernel itself
    Tensor out = output.has_value() ? *output : at::empty({N, 3}, positions.options());
    check_rc(xsg_sh_fwd_ex((int)degree_to_use, fptr(origin), N, (int)dim, fptr(positions), fptr(coeffs),
                           fptr(coeffs_dc), mask.has_value() ? (const uint32_t*)mask->data_ptr() : nullptr,
                           layout_3kn ? 1 : 0, output.has_value() ? 0 : 1, out.data_ptr<float>(),
                           stream_of(positions)));
    return out;
}

// spherical_harmonics_fused_bwd (sh_bwd.cu:317-390). origin_grad = false (extension): the origin
// gradient, a sum over every Gaussian, is not computed and comes back as None.
std::tuple<Tensor, Tensor, Tensor, OptT> spherical_harmonics_fused_bwd(int64_t degree_to_use, const Tensor& origin,
                                                                     const Tensor& positions, const Tensor& coeffs,
                                                                     const OptT& mask, bool layout_3kn,
                                                                     const Tensor& d_output, const OptT& coeffs_dc,
                                                                     bool origin_grad) {
    all_contiguous({d_output});
    int64_t N, dim;
    sh_checks(degree_to_use, origin, positions, coeffs, mask, layout_3kn, coeffs_dc, N, dim);
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(positions.device());
    const bool has_dc = coeffs_dc.has_value();
    Tensor d_coeffs = at::empty_like(coeffs);
    Tensor d_dc = has_dc ? at::empty_like(*coeffs_dc) : at::empty({0}, coeffs.options());
    Tensor d_pos = at::empty_like(positions);
    Tensor d_origin = origin_grad ? at::empty({3}, origin.options()) : Tensor();
    Tensor ws = workspace(positions, xsg_sh_bwd_workspace_bytes(N));
    check_rc(xsg_sh_bwd((int)degree_to_use, fptr(origin), N, (int)dim, fptr(positions), fptr(coeffs),
                        mask.has_value() ? (const uint32_t*)mask->data_ptr() : nullptr, layout_3kn ? 1 : 0,
                        fptr(d_output), has_dc ? 1 : 0, d_coeffs.data_ptr<float>(),
                        has_dc ? d_dc.data_ptr<float>() : nullptr, d_pos.data_ptr<float>(),
                        origin_grad ? d_origin.data_ptr<float>() : nullptr, ws.data_ptr(), stream_of(positions)));
    return {d_coeffs, d_dc, d_pos, origin_grad ? OptT(d_origin) : std::nullopt};
}

// ------------------------------------------------------------------ binning
// tile_offsets (extension): an int32 tensor that a sorted fill writes the tile offsets into, the values
// isect_offset_encode would compute from the sorted keys. keys = false (extension, with tile_offsets):
// the keys are not written and isect_ids comes back empty.
std::tuple<Tensor, Tensor, Tensor> isect_run(xsg_isect_desc& d, const Tensor& like, bool sort,
                                             const OptT& tile_offsets, bool keys) {
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(like.device());
    int32_t* offs = nullptr;
    if (tile_offsets.has_value()) {
        TORCH_CHECK(sort, "tile_offsets come with a sorted fill");
        TORCH_CHECK(tile_offsets->scalar_type() == at::kInt && tile_offsets->is_contiguous(),
                    "tile_offsets must be a contiguous int32 tensor");
        check_same_device({like, *tile_offsets});
        offs = tile_offsets->data_ptr<int32_t>();
    }
    TORCH_CHECK(keys || offs, "keys=False needs tile_offsets (a sorted fill that writes the offsets)");
    d.sort = sort ? 1 : 0;
    const xsg_stream_t s = stream_of(like);
    Tensor tiles_per_gauss = at::empty({d.n * d.n_cams}, like.options().dtype(at::kInt));
    Tensor cws = workspace(like, xsg_isect_count_workspace_bytes(&d));
    int64_t n_isects = 0, n_visible = 0, n_runs = 0;
    check_rc(xsg_isect_count(&d, tiles_per_gauss.data_ptr<int32_t>(), cws.data_ptr(), &n_isects, &n_visible,
                             &n_runs, s));
    Tensor isect_ids = at::empty({keys ? n_isects : 0}, like.options().dtype(at::kLong));
    Tensor flatten_ids = at::empty({n_isects}, like.options().dtype(at::kInt));
    if (n_isects > 0 || offs) {
        Tensor fws = workspace(like, sort && n_isects > 0 ? xsg_isect_fill_workspace_bytes(&d, n_isects, n_visible,
                                                                                           n_runs)
                                                          : 1);
        check_rc(xsg_isect_fill(&d, n_isects, n_visible, n_runs, sort ? 1 : 0, cws.data_ptr(), fws.data_ptr(),
                                keys ? isect_ids.data_ptr<int64_t>() : nullptr, flatten_ids.data_ptr<int32_t>(), offs,
                                offs ? tile_offsets->numel() : 0, s));
    }
    return {tiles_per_gauss, isect_ids, flatten_ids};
}

// isect_regular_tiles (regular_tiling.cu:72-146)
std::tuple<Tensor, Tensor, Tensor> isect_regular_tiles(const Tensor& means2d, const Tensor& radii, const Tensor& depths,
                                                       int64_t img_width, int64_t img_height, int64_t tile_size_x,
                                                       int64_t tile_size_y, bool sort, bool double_buffer,
                                                       const OptT& tile_offsets, bool keys) {
    (void)double_buffer;  // memory strategy only; results are identical
    check_same_device({means2d, radii, depths});
    all_contiguous({means2d, radii, depths});
    xsg_isect_desc d{};
    d.kind = XSG_TILING_REGULAR;
    d.n_cams = 1;
    d.n = means2d.numel() / 2;
    d.means2d = fptr(means2d); d.radii = fptr(radii); d.depths = fptr(depths);
    d.img_width = (float)img_width; d.img_height = (float)img_height;
    d.tile_w = (int)tile_size_x; d.tile_h = (int)tile_size_y;
    auto r = isect_run(d, depths, sort, tile_offsets, keys);
    std::get<0>(r) = std::get<0>(r).view(depths.sizes());
    return r;
}

// isect_regular_tiles over [C, N] projections of C cameras sharing one scene: keys carry the camera id
// above the tile bits and flatten ids are cam * N + gaussian (extension for batched camera rigs).
std::tuple<Tensor, Tensor, Tensor> isect_regular_tiles_batched(const Tensor& means2d, const Tensor& radii,
                                                               const Tensor& depths, int64_t img_width,
                                                               int64_t img_height, int64_t tile_size_x,
                                                               int64_t tile_size_y, bool sort, const OptT& tile_offsets,
                                                               bool keys) {
    check_same_device({means2d, radii, depths});
    all_contiguous({means2d, radii, depths});
    TORCH_CHECK(depths.dim() == 2, "batched tiling takes [C, N] depths");
    xsg_isect_desc d{};
    d.kind = XSG_TILING_REGULAR;
    d.n_cams = (int)depths.size(0);
    d.n = depths.size(1);
    d.means2d = fptr(means2d); d.radii = fptr(radii); d.depths = fptr(depths);
    d.img_width = (float)img_width; d.img_height = (float)img_height;
    d.tile_w = (int)tile_size_x; d.tile_h = (int)tile_size_y;
    auto r = isect_run(d, depths, sort, tile_offsets, keys);
    std::get<0>(r) = std::get<0>(r).view(depths.sizes());
    return r;
}

std::tuple<Tensor, Tensor, Tensor> isect_seam_tiles(int kind, const Tensor& camera_pack, const Tensor& points,
                                                    const OptT& points_velocity, const Tensor& scale, const Tensor& quat,
                                                    const OptT& opacity, const Tensor& flag, const Tensor& means2d,
                                                    const Tensor& radii, const Tensor& depths, const OptT& elev,
                                                    int64_t tile_size_x, int64_t tile_size_y, double img_width,
                                                    double img_height, double ut_alpha, double ut_beta,
                                                    double ut_kappa, bool sort, const OptT& tile_offsets, bool keys) {
    TORCH_CHECK(camera_pack.is_cuda(), "camera_pack must be CUDA tensor")
    std::vector<Tensor> ts{camera_pack, points, points_velocity.value_or(points), scale, quat, flag, means2d,
                           radii, depths};
    if (elev.has_value()) ts.push_back(*elev);
    check_same_device(ts);
    all_contiguous(ts);
    xsg_isect_desc d{};
    d.kind = kind;
    d.n_cams = 1;
    d.n = means2d.numel() / 2;
    d.means2d = fptr(means2d); d.radii = fptr(radii); d.depths = fptr(depths);
    d.flags = flag.data_ptr<uint8_t>();
    d.camera_pack = fptr(camera_pack);
    d.points = fptr(points); d.velocity = fptr(points_velocity); d.scales = fptr(scale);
    d.quats = fptr(quat); d.opacity = fptr(opacity);
    d.elev_boundaries = elev.has_value() ? fptr(*elev) : nullptr;
    d.n_elev = elev.has_value() ? (int)elev->size(0) : 0;
    d.img_width = (float)img_width; d.img_height = (float)img_height;
    d.tile_w = (int)tile_size_x; d.tile_h = (int)tile_size_y;
    d.ut_alpha = (float)ut_alpha; d.ut_beta = (float)ut_beta; d.ut_kappa = (float)ut_kappa;
    auto r = isect_run(d, depths, sort, tile_offsets, keys);
    std::get<0>(r) = std::get<0>(r).view(depths.sizes());
    return r;
}

// isect_lidar_tiles (phm_lidar_tiling.cu:239-375)
std::tuple<Tensor, Tensor, Tensor> isect_lidar_tiles(const Tensor& camera_pack, const Tensor& points,
                                                     const OptT& points_velocity, const Tensor& scale,
                                                     const Tensor& quat, const OptT& opacity, const Tensor& flag,
                                                     const Tensor& means2d, const Tensor& radii, const Tensor& depths,
                                                     const Tensor& elev_boundaries, int64_t tile_size_x,
                                                     double img_width, double img_height, double ut_alpha,
                                                     double ut_beta, double ut_kappa, bool sort, bool double_buffer,
                                                     const OptT& tile_offsets, bool keys) {
    (void)double_buffer;
    return isect_seam_tiles(XSG_TILING_LIDAR, camera_pack, points, points_velocity, scale, quat, opacity, flag,
                            means2d, radii, depths, elev_boundaries, tile_size_x, 1, img_width, img_height, ut_alpha,
                            ut_beta, ut_kappa, sort, tile_offsets, keys);
}

// isect_spherical_tiles (phm_spherical_tiling.cu:179-314)
std::tuple<Tensor, Tensor, Tensor> isect_spherical_tiles(const Tensor& camera_pack, const Tensor& points,
                                                         const OptT& points_velocity, const Tensor& scale,
                                                         const Tensor& quat, const OptT& opacity, const Tensor& flag,
                                                         const Tensor& means2d, const Tensor& radii,
                                                         const Tensor& depths, int64_t tile_size_x,
                                                         int64_t tile_size_y, double img_width, double img_height,
                                                         double ut_alpha, double ut_beta, double ut_kappa, bool sort,
                                                         bool double_buffer, const OptT& tile_offsets, bool keys) {
    (void)double_buffer;
    return isect_seam_tiles(XSG_TILING_SPHERICAL, camera_pack, points, points_velocity, scale, quat, opacity, flag,
                            means2d, radii, depths, std::nullopt, tile_size_x, tile_size_y, img_width, img_height,
                            ut_alpha, ut_beta, ut_kappa, sort, tile_offsets, keys);
}

// isect_offset_encode (tiling_common.cu:73-99); n_cams > 1 gives [n_cams, th, tw] (batched rigs)
Tensor isect_offset_encode(const Tensor& isect_ids, int64_t tile_width, int64_t tile_height, int64_t n_cams) {
    TORCH_CHECK(isect_ids.is_cuda() && isect_ids.is_contiguous(), "isect_ids must be contiguous cuda tensor")
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(isect_ids.device());
    const int64_t n = isect_ids.size(0);
    std::vector<int64_t> shape = {tile_height, tile_width};
    if (n_cams > 1) shape.insert(shape.begin(), n_cams);
    Tensor offsets = at::empty(shape, isect_ids.options().dtype(at::kInt));
    check_rc(xsg_isect_offset_encode(isect_ids.data_ptr<int64_t>(), n, (int)tile_width, (int)tile_height, (int)n_cams,
                                     offsets.data_ptr<int32_t>(), stream_of(isect_ids)));
    return offsets;
}

// mask_radii / mask_radii_packed (mask_radii.cu:60-88), in place
void mask_radii(const Tensor& mask, const Tensor& radii) {
    if (radii.size(-1) != 2) throw std::runtime_error("radii must be [..., 2] tensor");
    TORCH_CHECK(mask.dtype() == at::kBool, "Mask must be torch.bool tensor");
    const int64_t N = radii.numel() / 2;
    TORCH_CHECK(mask.numel() == N, "Mask size mismatch with radii");
    check_same_device({mask, radii});
    all_contiguous({mask, radii});
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(radii.device());
    check_rc(xsg_mask_radii(N, (const uint8_t*)mask.data_ptr(), radii.data_ptr<float>(), stream_of(radii)));
}

void mask_radii_packed(const Tensor& packed_mask, const Tensor& radii) {
    if (radii.size(-1) != 2) throw std::runtime_error("radii must be [..., 2] tensor");
    TORCH_CHECK(packed_mask.dtype() == at::kUInt32, "Packed mask must be UInt32 tensor");
    const int64_t N = radii.numel() / 2;
    TORCH_CHECK(packed_mask.numel() * 32 >= N, "Packed mask size mismatch with radii");
    check_same_device({packed_mask, radii});
    all_contiguous({packed_mask, radii});
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(radii.device());
    check_rc(xsg_mask_radii_packed(N, (const uint32_t*)packed_mask.data_ptr(), radii.data_ptr<float>(),
                                   stream_of(radii)));
}

// generic stable radix sort (sort_intersections' cub::DeviceRadixSort::SortPairs)
std::tuple<Tensor, Tensor> radix_sort_pairs(const Tensor& keys, const Tensor& values, int64_t begin_bit,
                                            int64_t end_bit) {
    TORCH_CHECK(keys.scalar_type() == at::kLong && values.scalar_type() == at::kInt, "keys int64, values int32");
    all_contiguous({keys, values});
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(keys.device());
    const int64_t n = keys.numel();
    Tensor k0 = keys.clone(), v0 = values.clone();
    Tensor k1 = at::empty_like(keys), v1 = at::empty_like(values);
    Tensor ws = workspace(keys, xsg_radix_sort_workspace_bytes(n));
    int sel = 0;
    check_rc(xsg_radix_sort_pairs_u64_i32(k0.data_ptr<int64_t>(), v0.data_ptr<int32_t>(), k1.data_ptr<int64_t>(),
                                          v1.data_ptr<int32_t>(), n, (int)begin_bit, (int)end_bit, ws.data_ptr(),
                                          &sel, stream_of(keys)));
    return sel ? std::make_tuple(k1, v1) : std::make_tuple(k0, v0);
}

// ------------------------------------------------------------------ scene-assembly producers
// mask_from_instances (csrc/nodes/gs_masking.cu:29-44)
// Extension: the packed mask of the Gaussians some tile of a regular tiling can hold, from the UT
// projection's radii [N, 2] or [C, N, 2] (any camera)
Tensor packed_visibility_mask(const Tensor& radii) {
    check_f32(radii, "radii");
    all_contiguous({radii});
    TORCH_CHECK((radii.dim() == 2 || radii.dim() == 3) && radii.size(-1) == 2, "radii must be [N, 2] or [C, N, 2]");
    const int64_t n = radii.size(-2);
    const int n_cams = radii.dim() == 3 ? (int)radii.size(0) : 1;
    TORCH_CHECK(n_cams >= 1, "radii must hold at least one camera");
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(radii.device());
    Tensor out = at::empty({(n + 31) / 32}, radii.options().dtype(at::kUInt32));
    check_rc(xsg_packed_visibility_from_radii(n, n_cams, fptr(radii), (uint32_t*)out.data_ptr(), stream_of(radii)));
    return out;
}

// Extension: the caller's parameter activations, scales = exp(log_scales) and opacities =
// sigmoid(opacity_logits), in one launch; and their gradients in one launch (either may be None).
std::tuple<Tensor, Tensor> activate_fwd(const Tensor& log_scales, const Tensor& opacity_logits) {
    check_same_device({log_scales, opacity_logits});
    all_contiguous({log_scales, opacity_logits});
    check_f32(log_scales, "log_scales");
    check_f32(opacity_logits, "opacity_logits");
    const int64_t n = opacity_logits.numel();
    TORCH_CHECK(log_scales.numel() == 3 * n, "log_scales must hold three values per opacity logit");
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(log_scales.device());
    Tensor scales = at::empty_like(log_scales), opacities = at::empty_like(opacity_logits);
    check_rc(xsg_activate_fwd(n, fptr(log_scales), fptr(opacity_logits), scales.data_ptr<float>(),
                              opacities.data_ptr<float>(), stream_of(log_scales)));
    return {scales, opacities};
}

std::tuple<Tensor, Tensor> activate_bwd(const Tensor& scales, const Tensor& opacities, const OptT& v_scales,
                                        const OptT& v_opacities) {
    std::vector<Tensor> ts{scales, opacities};
    for (const OptT* o : {&v_scales, &v_opacities})
        if (o->has_value()) ts.push_back(**o);
    check_same_device(ts);
    all_contiguous(ts);
    for (const auto& t : ts) check_f32(t, "activation tensors");
    const int64_t n = opacities.numel();
    TORCH_CHECK(scales.numel() == 3 * n, "scales must hold three values per opacity");
    TORCH_CHECK(!v_scales.has_value() || v_scales->numel() == 3 * n, "v_scales must match scales");
    TORCH_CHECK(!v_opacities.has_value() || v_opacities->numel() == n, "v_opacities must match opacities");
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(scales.device());
    Tensor v_log_scales, v_logits;
    if (v_scales.has_value()) v_log_scales = at::empty_like(scales);
    if (v_opacities.has_value()) v_logits = at::empty_like(opacities);
    check_rc(xsg_activate_bwd(n, fptr(scales), fptr(opacities), fptr(v_scales), fptr(v_opacities),
                              v_scales.has_value() ? v_log_scales.data_ptr<float>() : nullptr,
                              v_opacities.has_value() ? v_logits.data_ptr<float>() : nullptr, stream_of(scales)));
    return {v_log_scales, v_logits};
}

Tensor packed_mask_from_instances(const Tensor& instance_ids, const Tensor& instance_mask) {
    check_same_device({instance_ids, instance_mask});
    all_contiguous({instance_ids, instance_mask});
    TORCH_CHECK(instance_ids.scalar_type() == at::kInt, "instance_ids must be int32");
    TORCH_CHECK(instance_mask.element_size() == 1, "instance_mask must be a bool / uint8 tensor");
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(instance_ids.device());
    const int64_t n = instance_ids.numel();
    Tensor out = at::empty({(n + 31) / 32}, instance_ids.options().dtype(at::kUInt32));
    check_rc(xsg_packed_mask_from_instances(n, instance_ids.data_ptr<int32_t>(),
                                            (const uint8_t*)instance_mask.data_ptr(), instance_mask.numel(),
                                            (uint32_t*)out.data_ptr(), stream_of(instance_ids)));
    return out;
}

xsg_rigid_desc rigid_desc(const Tensor& positions, const Tensor& rotations, const Tensor& instance_id,
                          const Tensor& inst_q, const OptT& inst_t, const OptT& inst_v, const Tensor& inst_w,
                          const Tensor& inst_mask, int64_t n_out, int64_t buffer_offset, const OptT& per_inst_off,
                          const OptT& gs_inst_off) {
    std::vector<Tensor> ts{positions, rotations, instance_id, inst_q, inst_w, inst_mask};
    for (const OptT* o : {&inst_t, &inst_v, &per_inst_off, &gs_inst_off})
        if (o->has_value()) ts.push_back(**o);
    check_same_device(ts);
    all_contiguous(ts);
    for (const Tensor* t : {&positions, &rotations, &inst_q, &inst_w}) check_f32(*t, "positions / quaternions");
    TORCH_CHECK(instance_id.scalar_type() == at::kInt, "instance_id must be int32");
    TORCH_CHECK(inst_mask.element_size() == 1, "inst_mask must be a bool / uint8 tensor");
    TORCH_CHECK(per_inst_off.has_value() == gs_inst_off.has_value(),
                "per_instance_offsets and gs_inst_offsets go together");
    if (gs_inst_off.has_value())
        TORCH_CHECK(per_inst_off->scalar_type() == at::kInt && gs_inst_off->scalar_type() == at::kInt,
                    "instance offsets must be int32");
    const int64_t n = positions.size(0), k = inst_q.size(0);
    TORCH_CHECK(positions.numel() == 3 * n && rotations.numel() == 4 * n && instance_id.numel() == n,
                "positions [N, 3], rotations [N, 4], instance_id [N]");
    TORCH_CHECK(inst_q.numel() == 4 * k && inst_w.numel() == 3 * k && inst_mask.numel() == k,
                "inst_q [K, 4], inst_w [K, 3], inst_mask [K]");
    if (gs_inst_off.has_value())
        TORCH_CHECK(per_inst_off->numel() == k && gs_inst_off->numel() == n,
                    "per_instance_offsets [K], gs_inst_offsets [N]");
    xsg_rigid_desc d{};
    d.n = n; d.n_instances = k; d.n_out = n_out; d.buffer_offset = buffer_offset;
    d.positions = fptr(positions); d.rotations = fptr(rotations); d.instance_ids = instance_id.data_ptr<int32_t>();
    d.inst_q = fptr(inst_q); d.inst_t = fptr(inst_t); d.inst_v = fptr(inst_v); d.inst_w = fptr(inst_w);
    d.inst_mask = (const uint8_t*)inst_mask.data_ptr();
    d.per_instance_offsets = per_inst_off.has_value() ? per_inst_off->data_ptr<int32_t>() : nullptr;
    d.gs_inst_offsets = gs_inst_off.has_value() ? gs_inst_off->data_ptr<int32_t>() : nullptr;
    return d;
}

// copy_gs_rigid_transform_fwd (csrc/nodes/container.cu:171-215): writes the output buffers in place
void copy_gs_rigid_transform_fwd(const Tensor& positions, const Tensor& rotations, const Tensor& instance_id,
                                 const Tensor& inst_q, const Tensor& inst_t, const Tensor& inst_v,
                                 const Tensor& inst_w, const Tensor& inst_mask, const Tensor& out_positions,
                                 const Tensor& out_rotations, const OptT& out_velocities, const OptT& out_mask,
                                 int64_t buffer_offset, const OptT& per_instance_offsets,
                                 const OptT& gs_inst_offsets) {
    TORCH_CHECK(buffer_offset >= 0, "buffer_offset must be non-negative");
    const int64_t k = inst_q.size(0);
    TORCH_CHECK(inst_t.numel() == 3 * k && inst_v.numel() == 3 * k, "inst_t, inst_v [K, 3]");
    check_f32(inst_t, "inst_t");
    check_f32(inst_v, "inst_v");
    xsg_rigid_desc d = rigid_desc(positions, rotations, instance_id, inst_q, inst_t, inst_v, inst_w, inst_mask,
                                  out_positions.size(0), buffer_offset, per_instance_offsets, gs_inst_offsets);
    std::vector<Tensor> outs{out_positions, out_rotations};
    if (out_velocities.has_value()) outs.push_back(*out_velocities);
    if (out_mask.has_value()) outs.push_back(*out_mask);
    outs.push_back(positions);
    check_same_device(outs);
    all_contiguous(outs);
    const int64_t b = out_positions.size(0);
    check_f32(out_positions, "out_positions");
    check_f32(out_rotations, "out_rotations");
    TORCH_CHECK(out_positions.numel() == 3 * b && out_rotations.numel() == 4 * b, "out buffers [B, 3], [B, 4]");
    if (out_velocities.has_value()) {
        check_f32(*out_velocities, "out_velocities");
        TORCH_CHECK(out_velocities->numel() == 3 * b, "out_velocities [B, 3]");
    }
    if (out_mask.has_value())
        TORCH_CHECK(out_mask->element_size() == 1 && out_mask->numel() == b, "out_mask: bool [B]");
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(positions.device());
    check_rc(xsg_rigid_transform_fwd(&d, out_positions.data_ptr<float>(), out_rotations.data_ptr<float>(),
                                     out_velocities.has_value() ? out_velocities->data_ptr<float>() : nullptr,
                                     out_mask.has_value() ? (uint8_t*)out_mask->data_ptr() : nullptr,
                                     stream_of(positions)));
}

// copy_gs_rigid_transform_bwd (csrc/nodes/container.cu:218-266)
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> copy_gs_rigid_transform_bwd(
    const Tensor& positions, const Tensor& rotations, const Tensor& instance_id, const Tensor& inst_q,
    const Tensor& inst_w, const Tensor& inst_mask, int64_t buffer_offset, const OptT& per_instance_offsets,
    const OptT& gs_inst_offsets, const Tensor& v_positions, const Tensor& v_rotations, const OptT& v_velocities) {
    TORCH_CHECK(buffer_offset >= 0, "buffer_offset must be non-negative");
    xsg_rigid_desc d = rigid_desc(positions, rotations, instance_id, inst_q, std::nullopt, std::nullopt, inst_w,
                                  inst_mask, v_positions.size(0), buffer_offset, per_instance_offsets,
                                  gs_inst_offsets);
    const int64_t b = v_positions.size(0);
    Tensor vp = v_positions.contiguous(), vr = v_rotations.contiguous();
    OptT vv = v_velocities.has_value() ? OptT(v_velocities->contiguous()) : std::nullopt;
    check_f32(vp, "v_positions");
    check_f32(vr, "v_rotations");
    TORCH_CHECK(vp.numel() == 3 * b && vr.numel() == 4 * b, "v_positions [B, 3], v_rotations [B, 4]");
    if (vv.has_value()) {
        check_f32(*vv, "v_velocities");
        TORCH_CHECK(vv->numel() == 3 * b, "v_velocities [B, 3]");
    }
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(positions.device());
    Tensor g_pos = at::empty_like(positions), g_rot = at::empty_like(rotations);
    Tensor g_q = at::empty_like(inst_q), g_t = at::empty_like(inst_w), g_v = at::empty_like(inst_w),
           g_w = at::empty_like(inst_w);
    Tensor ws = workspace(positions, xsg_rigid_transform_bwd_workspace_bytes(d.n_instances));
    check_rc(xsg_rigid_transform_bwd(&d, vp.data_ptr<float>(), vr.data_ptr<float>(), fptr(vv),
                                     g_pos.data_ptr<float>(), g_rot.data_ptr<float>(), g_q.data_ptr<float>(),
                                     g_t.data_ptr<float>(), g_v.data_ptr<float>(), g_w.data_ptr<float>(),
                                     ws.data_ptr(), stream_of(positions)));
    return {g_pos, g_rot, g_q, g_t, g_v, g_w};
}

// ------------------------------------------------------------------ cameras
struct CamSpec {
    int kind;
    std::vector<int> impl_dims;
};

// pack_camera (include/cameras/pack_kernels.h:11-47): validated, then concatenated into the flat
// layout the kernels read. torch.cat keeps the pack differentiable w.r.t. the camera tensors.
Tensor camera_pack(const CamSpec& spec, const std::vector<Tensor>& tensors) {
    static const int base_dims[7] = {4, 3, 3, 3, 2, 1, 1};
    const size_t expected = 7 + spec.impl_dims.size();
    if (tensors.size() != expected)
        throw std::runtime_error("Tensor list size mismatch. Expected " + std::to_string(expected) +
                                 ", but found: " + std::to_string(tensors.size()));
    check_same_device(tensors);
    std::vector<Tensor> flat;
    for (size_t i = 0; i < tensors.size(); ++i) {
        TORCH_CHECK(tensors[i].scalar_type() == at::kFloat, "Camera tensors must be float32");
        const int want = i < 7 ? base_dims[i] : spec.impl_dims[i - 7];
        TORCH_CHECK(tensors[i].numel() == want, "Only single camera is currently supported (tensor ", i,
                    " has ", tensors[i].numel(), " elements, expected ", want, ")");
        flat.push_back(tensors[i].reshape({1, want}));
    }
    return at::cat(flat, 1).contiguous();
}

void validate_pack(const CamSpec& spec, const Tensor& pack) {  // camera.h:56-62
    TORCH_CHECK(pack.numel() == xsg_camera_pack_elements(spec.kind), "Only single camera is currently supported");
    TORCH_CHECK(pack.dtype() == at::kFloat, "Camera type must be float32");
    TORCH_CHECK(pack.is_contiguous(), "Camera pack must be contiguous tensor");
    TORCH_CHECK(pack.is_cuda(), "Camera pack must be on the GPU");
}

// CameraRaysFunction (include/cameras/ray_kernels.h:164-226): forward launch_camera_ray_fwd,
// backward camera_ray_backward into the pack's gradient. Outputs: [ray_o if return_origins], ray_d,
// [valid, non-differentiable].
struct CameraRaysFn : public torch::autograd::Function<CameraRaysFn> {
    static torch::autograd::variable_list forward(torch::autograd::AutogradContext* ctx, const Tensor& pack,
                                                  int64_t kind, int64_t width, int64_t height, bool world_space,
                                                  bool normalized, bool return_origins, bool return_valid) {
        const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(pack.device());
        auto opt = pack.options();
        Tensor ray_o = return_origins ? at::empty({height, width, 3}, opt) : Tensor();
        Tensor ray_d = at::empty({height, width, 3}, opt);
        Tensor valid = return_valid ? at::empty({height, width}, opt.dtype(at::kBool)) : Tensor();
        check_rc(xsg_camera_rays((int)kind, fptr(pack), (int)width, (int)height, world_space ? 1 : 0,
                                 normalized ? 1 : 0, return_origins ? ray_o.data_ptr<float>() : nullptr,
                                 ray_d.data_ptr<float>(), return_valid ? (uint8_t*)valid.data_ptr() : nullptr,
                                 stream_of(pack)));
        ctx->save_for_backward({pack});
        ctx->saved_data["kind"] = kind;
        ctx->saved_data["world_space"] = world_space;
        ctx->saved_data["normalized"] = normalized;
        ctx->saved_data["return_origins"] = return_origins;
        torch::autograd::variable_list out;
        if (return_origins) out.push_back(ray_o);
        out.push_back(ray_d);
        if (return_valid) {
            ctx->mark_non_differentiable({valid});
            out.push_back(valid);
        }
        return out;
    }

    static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                   torch::autograd::variable_list grads) {
        const Tensor pack = ctx->get_saved_variables()[0];
        const bool ro = ctx->saved_data["return_origins"].toBool();
        const Tensor d_ray_d = grads[ro ? 1 : 0].contiguous();
        const Tensor d_ray_o = ro ? grads[0].contiguous() : Tensor();
        const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(pack.device());
        const int height = (int)d_ray_d.size(0), width = (int)d_ray_d.size(1);
        Tensor grad_pack = at::empty_like(pack);
        Tensor ws = workspace(pack, xsg_camera_rays_bwd_workspace_bytes(width, height));
        check_rc(xsg_camera_rays_bwd((int)ctx->saved_data["kind"].toInt(), fptr(pack), width, height,
                                     ctx->saved_data["world_space"].toBool() ? 1 : 0,
                                     ctx->saved_data["normalized"].toBool() ? 1 : 0,
                                     d_ray_o.defined() ? fptr(d_ray_o) : nullptr, fptr(d_ray_d),
                                     grad_pack.data_ptr<float>(), ws.data_ptr(), stream_of(pack)));
        return {grad_pack, Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

// the autograd function only when the pack needs a gradient (its bookkeeping costs host time)
bool needs_grad(const Tensor& t) { return t.requires_grad() && at::GradMode::is_enabled(); }

// out (extension): preallocated contiguous float32 (ray_o, ray_d) of [height, width, 3] each (ray_o
// ignored without return_origins), e.g. one camera's slices of a rig's [C, H, W, 3] buffers; not with
// a pack that needs a gradient
py::object camera_rays(const CamSpec& spec, const Tensor& pack, int64_t width, int64_t height, bool world_space,
                       bool normalized, bool return_origins, bool return_valid,
                       const std::optional<std::tuple<Tensor, Tensor>>& out_rays) {
    validate_pack(spec, pack);
    torch::autograd::variable_list res;
    if (out_rays.has_value()) {
        TORCH_CHECK(!needs_grad(pack), "camera_rays: out= takes a pack that needs no gradient");
        TORCH_CHECK(!return_valid, "camera_rays: out= comes without return_valid");
        const auto& [ro, rd] = *out_rays;
        std::vector<Tensor> ts{pack, rd};
        if (return_origins) ts.push_back(ro);
        check_same_device(ts);
        for (size_t i = 1; i < ts.size(); ++i)
            TORCH_CHECK(ts[i].scalar_type() == at::kFloat && ts[i].is_contiguous() &&
                            ts[i].numel() == height * width * 3,
                        "camera_rays: out tensors must be contiguous float32 of height x width x 3");
        const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(pack.device());
        check_rc(xsg_camera_rays(spec.kind, fptr(pack), (int)width, (int)height, world_space ? 1 : 0,
                                 normalized ? 1 : 0, return_origins ? ro.data_ptr<float>() : nullptr,
                                 rd.data_ptr<float>(), nullptr, stream_of(pack)));
        py::list o;
        o.append(return_origins ? py::cast(ro) : py::none());
        o.append(py::cast(rd));
        return std::move(o);
    }
    if (needs_grad(pack)) {
        res = CameraRaysFn::apply(pack, (int64_t)spec.kind, width, height, world_space, normalized, return_origins,
                                  return_valid);
    } else {
        torch::autograd::AutogradContext ctx;
        res = CameraRaysFn::forward(&ctx, pack, (int64_t)spec.kind, width, height, world_space, normalized,
                                    return_origins, return_valid);
    }
    py::list out;
    size_t i = 0;
    out.append(return_origins ? py::cast(res[i++]) : py::none());
    out.append(py::cast(res[i++]));
    if (return_valid) out.append(py::cast(res[i]));
    return out;
}

// CameraPixelTime[Delta]Function (include/cameras/time_kernels.h:364-458): the gradient w.r.t. the
// pack is sum(g u), sum(g v), sum(g) on rolling_time and trigger_time (-sum(g) on pose_time for the
// delta variant).
struct PixelTimeFn : public torch::autograd::Function<PixelTimeFn> {
    static Tensor forward(torch::autograd::AutogradContext* ctx, const Tensor& pack, int64_t kind, int64_t width,
                          int64_t height, bool delta) {
        const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(pack.device());
        Tensor out = at::empty({height, width}, pack.options());
        check_rc(xsg_pixel_time((int)kind, fptr(pack), (int)width, (int)height, nullptr, 0, delta ? 1 : 0,
                                out.data_ptr<float>(), stream_of(pack)));
        ctx->save_for_backward({pack});
        ctx->saved_data["kind"] = kind;
        ctx->saved_data["delta"] = delta;
        return out;
    }

    static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                   torch::autograd::variable_list grads) {
        const Tensor pack = ctx->get_saved_variables()[0];
        const Tensor g = grads[0].contiguous();
        const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(pack.device());
        const int height = (int)g.size(0), width = (int)g.size(1);
        Tensor grad_pack = at::empty_like(pack);
        Tensor ws = workspace(pack, xsg_pixel_time_bwd_workspace_bytes(width, height, 0));
        check_rc(xsg_pixel_time_bwd((int)ctx->saved_data["kind"].toInt(), fptr(pack), width, height, nullptr, 0,
                                    ctx->saved_data["delta"].toBool() ? 1 : 0, fptr(g), grad_pack.data_ptr<float>(),
                                    nullptr, ws.data_ptr(), stream_of(pack)));
        return {grad_pack, Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

// CameraPixelTime[Delta]FromUVFunction (include/cameras/time_kernels.h:398-489): gradients w.r.t. the
// pack and the uv coordinates (d_uv = g rolling_time).
struct PixelTimeUvFn : public torch::autograd::Function<PixelTimeUvFn> {
    static Tensor forward(torch::autograd::AutogradContext* ctx, const Tensor& pack, const Tensor& uv, int64_t kind,
                          bool delta) {
        const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(pack.device());
        auto sizes = uv.sizes().vec();
        sizes.pop_back();
        Tensor out = at::empty(sizes, uv.options());
        Tensor uvc = uv.contiguous();
        check_rc(xsg_pixel_time((int)kind, fptr(pack), 0, 0, fptr(uvc), uv.numel() / 2, delta ? 1 : 0,
                                out.data_ptr<float>(), stream_of(pack)));
        ctx->save_for_backward({pack, uvc});
        ctx->saved_data["kind"] = kind;
        ctx->saved_data["delta"] = delta;
        return out;
    }

    static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                   torch::autograd::variable_list grads) {
        const auto saved = ctx->get_saved_variables();
        const Tensor pack = saved[0], uvc = saved[1];
        const Tensor g = grads[0].contiguous();
        const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(pack.device());
        const int64_t n = uvc.numel() / 2;
        Tensor grad_pack = at::empty_like(pack);
        Tensor d_uv = ctx->needs_input_grad(1) ? at::empty_like(uvc) : Tensor();
        Tensor ws = workspace(pack, xsg_pixel_time_bwd_workspace_bytes(0, 0, n));
        check_rc(xsg_pixel_time_bwd((int)ctx->saved_data["kind"].toInt(), fptr(pack), 0, 0, fptr(uvc), n,
                                    ctx->saved_data["delta"].toBool() ? 1 : 0, fptr(g), grad_pack.data_ptr<float>(),
                                    d_uv.defined() ? d_uv.data_ptr<float>() : nullptr, ws.data_ptr(),
                                    stream_of(pack)));
        return {grad_pack, d_uv, Tensor(), Tensor()};
    }
};

Tensor pixel_time(const CamSpec& spec, const Tensor& pack, int64_t width, int64_t height, bool delta) {
    validate_pack(spec, pack);
    if (needs_grad(pack)) return PixelTimeFn::apply(pack, (int64_t)spec.kind, width, height, delta);
    torch::autograd::AutogradContext ctx;
    return PixelTimeFn::forward(&ctx, pack, (int64_t)spec.kind, width, height, delta);
}

Tensor pixel_time_uv(const CamSpec& spec, const Tensor& pack, const Tensor& uv, bool delta) {
    validate_pack(spec, pack);
    TORCH_CHECK(uv.size(-1) == 2, "UV coordinates last dimension must be 2")
    TORCH_CHECK(uv.device() == pack.device(), "Camera and UV-s must be on the same device")
    TORCH_CHECK(uv.dtype() == at::kFloat, "UV coordinates must be float32 tensor")
    if (needs_grad(pack) || needs_grad(uv)) return PixelTimeUvFn::apply(pack, uv, (int64_t)spec.kind, delta);
    torch::autograd::AutogradContext ctx;
    return PixelTimeUvFn::forward(&ctx, pack, uv, (int64_t)spec.kind, delta);
}

// undistort_map (include/cameras/distortion.h:33-56)
Tensor undistort_map(const CamSpec& spec, const Tensor& pack, int64_t width, int64_t height, bool normalized_range) {
    validate_pack(spec, pack);
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(pack.device());
    Tensor out = at::empty({height, width, 2}, pack.options());
    check_rc(xsg_undistort_map(spec.kind, fptr(pack), (int)width, (int)height, normalized_range ? 1 : 0,
                               out.data_ptr<float>(), stream_of(pack)));
    return out;
}

std::tuple<Tensor, Tensor> projection(const CamSpec& spec, bool no_jac, const Tensor& pack, const Tensor& points,
                                      const OptT& points_velocity, double thr, double max_res, double margin,
                                      int mode) {
    validate_pack(spec, pack);
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(pack.device());
    const int64_t N = points.size(0);
    Tensor mask = at::empty({N}, pack.options().dtype(at::kBool));
    Tensor uvdt = at::empty({N, 4}, pack.options());
    Tensor pts = points.contiguous();
    OptT vel = points_velocity.has_value() ? OptT(points_velocity->contiguous()) : std::nullopt;
    check_rc(xsg_project_points(spec.kind, fptr(pack), N, fptr(pts), fptr(vel), (float)thr, (float)max_res,
                                (float)margin, mode, no_jac ? 1 : 0, uvdt.data_ptr<float>(),
                                (uint8_t*)mask.data_ptr(), stream_of(pack)));
    return {uvdt, mask};
}

// launch_unscented_transform[_phm] (ut_kernels.h:249-305, ut_phm_kernels.h:125-173)
// out (extension): four preallocated contiguous tensors (flags u8 [N], radii [N, 2], means2d [N, 2],
// depths [N], float32) that receive the results, e.g. one camera's slices of a rig's [C, N, ...]
// buffers, which then need no stacking
using UtOut = std::optional<std::tuple<Tensor, Tensor, Tensor, Tensor>>;

std::tuple<Tensor, Tensor, Tensor, Tensor> projection_utgs(const CamSpec& spec, bool phm, const Tensor& pack,
                                                           const Tensor& points, const OptT& points_velocity,
                                                           const Tensor& scales, const Tensor& quats,
                                                           const OptT& opacity, double width, double height,
                                                           double ut_alpha, double ut_beta, double ut_kappa,
                                                           double thr, double max_res, double margin,
                                                           const UtOut& out) {
    validate_pack(spec, pack);
    check_same_device({pack, points, scales, quats});
    std::vector<Tensor> ts{points, scales, quats};
    if (points_velocity.has_value()) ts.push_back(*points_velocity);
    if (opacity.has_value()) ts.push_back(*opacity);
    all_contiguous(ts);
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(points.device());
    const int64_t N = points.size(0);
    Tensor flags, radii, mean2d, depths;
    if (out.has_value()) {
        std::tie(flags, radii, mean2d, depths) = *out;
        check_same_device({points, flags, radii, mean2d, depths});
        TORCH_CHECK(flags.scalar_type() == at::kByte && radii.scalar_type() == at::kFloat &&
                        mean2d.scalar_type() == at::kFloat && depths.scalar_type() == at::kFloat,
                    "out: flags must be uint8, radii / means2d / depths float32");
        TORCH_CHECK(flags.numel() == N && radii.numel() == 2 * N && mean2d.numel() == 2 * N && depths.numel() == N,
                    "out: tensors for ", N, " points expected");
        all_contiguous({flags, radii, mean2d, depths});
    } else {
        flags = at::empty({N}, points.options().dtype(at::kByte));
        radii = at::empty({N, 2}, points.options());
        mean2d = at::empty({N, 2}, points.options());
        depths = at::empty({N}, points.options());
    }
    check_rc(xsg_ut_project(spec.kind, phm ? 1 : 0, fptr(pack), N, fptr(points), fptr(points_velocity),
                            fptr(scales), fptr(quats), fptr(opacity), (float)width, (float)height, (float)ut_alpha,
                            (float)ut_beta, (float)ut_kappa, (float)thr, (float)max_res, (float)margin,
                            flags.data_ptr<uint8_t>(), radii.data_ptr<float>(), mean2d.data_ptr<float>(),
                            depths.data_ptr<float>(), stream_of(points)));
    return {flags, radii, mean2d, depths};
}

// projection_utgs over a rig (extension): packs [C, pack elements] of C cameras of this kind, one
// launch; returns flags [C, N], radii [C, N, 2], means2d [C, N, 2], depths [C, N]
std::tuple<Tensor, Tensor, Tensor, Tensor> projection_utgs_rig(const CamSpec& spec, const Tensor& packs,
                                                               const Tensor& points, const OptT& points_velocity,
                                                               const Tensor& scales, const Tensor& quats,
                                                               const OptT& opacity, double width, double height,
                                                               double ut_alpha, double ut_beta, double ut_kappa,
                                                               double thr, double max_res, double margin) {
    TORCH_CHECK(packs.is_cuda() && packs.dtype() == at::kFloat && packs.is_contiguous() && packs.dim() == 2 &&
                    packs.size(1) == xsg_camera_pack_elements(spec.kind),
                "packs must be a contiguous float32 CUDA tensor of [cameras, ", xsg_camera_pack_elements(spec.kind),
                "]");
    check_same_device({packs, points, scales, quats});
    std::vector<Tensor> ts{points, scales, quats};
    if (points_velocity.has_value()) ts.push_back(*points_velocity);
    if (opacity.has_value()) ts.push_back(*opacity);
    all_contiguous(ts);
    const c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(points.device());
    const int64_t C = packs.size(0), N = points.size(0);
    Tensor flags = at::empty({C, N}, points.options().dtype(at::kByte));
    Tensor radii = at::empty({C, N, 2}, points.options());
    Tensor mean2d = at::empty({C, N, 2}, points.options());
    Tensor depths = at::empty({C, N}, points.options());
    check_rc(xsg_ut_project_rig(spec.kind, (int)C, fptr(packs), packs.size(1), N, fptr(points),
                                fptr(points_velocity), fptr(scales), fptr(quats), fptr(opacity), (float)width,
                                (float)height, (float)ut_alpha, (float)ut_beta, (float)ut_kappa, (float)thr,
                                (float)max_res, (float)margin, flags.data_ptr<uint8_t>(), radii.data_ptr<float>(),
                                mean2d.data_ptr<float>(), depths.data_ptr<float>(), stream_of(points)));
    return {flags, radii, mean2d, depths};
}

template <int I>
struct CameraTag {};

// pybind_camera (include/cameras/bind.h:20-126): the same static methods, projection_utgs_phm for
// the phase-modelled (spherical, lidar) cameras and undistort_map for the models with distort_uv.
template <int I>
void bind_camera(py::module& m, const char* name, CamSpec spec, bool phm) {
    auto cls = py::class_<CameraTag<I>>(m, name);
    cls.def_static("pack", [spec](const std::vector<Tensor>& tensors) { return camera_pack(spec, tensors); },
                   py::arg("tensors"));
    cls.def_static("camera_rays",
                   [spec](const Tensor& pack, int64_t width, int64_t height, bool world_space, bool normalized,
                          bool return_origins, bool return_valid,
                          const std::optional<std::tuple<Tensor, Tensor>>& out) {
                       return camera_rays(spec, pack, width, height, world_space, normalized, return_origins,
                                          return_valid, out);
                   },
                   py::arg("pack"), py::arg("width"), py::arg("height"), py::arg("world_space") = true,
                   py::arg("normalized") = true, py::arg("return_origins") = true, py::arg("return_valid") = false,
                   py::arg("out") = py::none());
    cls.def_static("pixel_time",
                   [spec](const Tensor& pack, int64_t w, int64_t h) { return pixel_time(spec, pack, w, h, false); },
                   py::arg("pack"), py::arg("width"), py::arg("height"));
    cls.def_static("pixel_time_delta",
                   [spec](const Tensor& pack, int64_t w, int64_t h) { return pixel_time(spec, pack, w, h, true); },
                   py::arg("pack"), py::arg("width"), py::arg("height"));
    cls.def_static("pixel_time_from_uv",
                   [spec](const Tensor& pack, const Tensor& uvs) { return pixel_time_uv(spec, pack, uvs, false); },
                   py::arg("pack"), py::arg("uvs"));
    cls.def_static("pixel_time_delta_from_uv",
                   [spec](const Tensor& pack, const Tensor& uvs) { return pixel_time_uv(spec, pack, uvs, true); },
                   py::arg("pack"), py::arg("uvs"));
    for (int nojac = 0; nojac < 2; ++nojac) {
        cls.def_static(nojac ? "projection_nojac" : "projection",
                       [spec, nojac](const Tensor& pack, const Tensor& points, const OptT& vel, double thr,
                                     double max_res, double margin, int mode) {
                           return projection(spec, nojac != 0, pack, points, vel, thr, max_res, margin, mode);
                       },
                       py::arg("pack"), py::arg("points"), py::arg("points_velocity") = py::none(),
                       py::arg("residual_thr_early_stop") = 1e-4f, py::arg("max_residual") = 0.002f,
                       py::arg("max_margin") = 1.0f, py::arg("projection_mode") = XSG_MODE_CENTRAL);
    }
    for (int with_phm = 0; with_phm < (phm ? 2 : 1); ++with_phm) {
        cls.def_static(with_phm ? "projection_utgs_phm" : "projection_utgs",
                       [spec, with_phm](const Tensor& pack, const Tensor& points, const OptT& vel, const Tensor& scales,
                                        const Tensor& quats, const OptT& opacity, double width, double height,
                                        double a, double b, double k, double thr, double max_res, double margin,
                                        const UtOut& out) {
                           return projection_utgs(spec, with_phm != 0, pack, points, vel, scales, quats, opacity,
                                                  width, height, a, b, k, thr, max_res, margin, out);
                       },
                       py::arg("pack"), py::arg("points"), py::arg("points_velocity"), py::arg("scales"),
                       py::arg("quats"), py::arg("opacity"), py::arg("width"), py::arg("height"),
                       py::arg("ut_alpha") = 0.1f, py::arg("ut_beta") = 2.0f, py::arg("ut_kappa") = 0.0f,
                       py::arg("residual_thr_early_stop") = 1e-4f, py::arg("max_residual") = 0.002f,
                       py::arg("max_margin") = 1.0f, py::arg("out") = py::none());
    }
    if (!phm)
        cls.def_static("projection_utgs_rig",
                       [spec](const Tensor& packs, const Tensor& points, const OptT& vel, const Tensor& scales,
                              const Tensor& quats, const OptT& opacity, double width, double height, double a,
                              double b, double k, double thr, double max_res, double margin) {
                           return projection_utgs_rig(spec, packs, points, vel, scales, quats, opacity, width,
                                                      height, a, b, k, thr, max_res, margin);
                       },
                       py::arg("packs"), py::arg("points"), py::arg("points_velocity"), py::arg("scales"),
                       py::arg("quats"), py::arg("opacity"), py::arg("width"), py::arg("height"),
                       py::arg("ut_alpha") = 0.1f, py::arg("ut_beta") = 2.0f, py::arg("ut_kappa") = 0.0f,
                       py::arg("residual_thr_early_stop") = 1e-4f, py::arg("max_residual") = 0.002f,
                       py::arg("max_margin") = 1.0f);
    if (spec.kind == XSG_CAM_DISTORTED || spec.kind == XSG_CAM_FISHEYE) {
        cls.def_static("undistort_map",
                       [spec](const Tensor& pack, int64_t width, int64_t height, bool normalized_range) {
                           return undistort_map(spec, pack, width, height, normalized_range);
                       },
                       py::arg("pack"), py::arg("width"), py::arg("height"), py::arg("normalized_range") = false);
    }
}

// measurement support for bench.py: the VALU issue ceiling launch, on the current stream
void bench_valu_ceiling(int64_t blocks, int64_t iters, const Tensor& out, const Tensor& stamps) {
    TORCH_CHECK(blocks > 0 && blocks <= (1 << 20) && iters > 0 && iters <= (1 << 24), "valu ceiling: blocks ",
                blocks, " / iters ", iters, " out of range");
    check_f32(out, "out");
    TORCH_CHECK(stamps.scalar_type() == at::kLong, "stamps must be an int64 tensor");
    TORCH_CHECK(out.is_contiguous() && stamps.is_contiguous(), "out and stamps must be contiguous");
    TORCH_CHECK(out.numel() >= blocks * 256 && stamps.numel() >= 4 * blocks,
                "out needs blocks * 256 floats and stamps 4 * blocks entries");
    check_same_device({out, stamps});
    check_rc(xsg_bench_valu_ceiling((int)blocks, (int)iters, out.data_ptr<float>(),
                                    reinterpret_cast<uint64_t*>(stamps.data_ptr()), stream_of(out)));
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "xsimgs_amd: MI355X (gfx950) kernels for the xsimgs Gaussian-splatting hot path";
    m.def("abi_version", &xsg_abi_version);
    m.def("bench_valu_ceiling", &bench_valu_ceiling, py::arg("blocks"), py::arg("iters"), py::arg("out"),
          py::arg("stamps"));

    // rasterization (csrc/rasterization/*_bind)
    m.def("rasterize_eval3d_fwd", &rasterize_eval3d_fwd, py::arg("means"), py::arg("quats"), py::arg("scales"),
          py::arg("colors"), py::arg("opacities"), py::arg("image_width"), py::arg("image_height"),
          py::arg("tile_size_width"), py::arg("tile_size_height"), py::arg("ray_origs"), py::arg("ray_dirs"),
          py::arg("tile_offsets"), py::arg("flatten_ids"), py::arg("pair_counts") = py::none(),
          py::arg("tile_work") = py::none());
    // positional like the reference (eval3d_bwd.cu:406-408); `ray_grads` (extension, default True)
    // lets autograd skip the per-pixel ray gradients when the rays do not require grad
    m.def("rasterize_eval3d_bwd", &rasterize_eval3d_bwd, py::arg("points"), py::arg("scale"), py::arg("quat"),
          py::arg("opacity"), py::arg("colors"), py::arg("ray_origins"), py::arg("ray_directions"),
          py::arg("tile_size_x"), py::arg("tile_size_y"), py::arg("tile_offsets"), py::arg("flatten_ids"),
          py::arg("render_alpha"), py::arg("last_ids"), py::arg("v_render_colors"), py::arg("v_render_depth"),
          py::arg("v_render_alpha"), py::arg("ray_grads") = true, py::arg("pair_counts") = py::none(),
          py::arg("pixels_per_lane") = 0, py::arg("tile_work") = py::none());
    m.def("rasterize_eval3d_dynamic_fwd", &rasterize_eval3d_dynamic_fwd, py::arg("means"), py::arg("velocity"),
          py::arg("quats"), py::arg("scales"), py::arg("colors"), py::arg("opacities"), py::arg("image_width"),
          py::arg("image_height"), py::arg("tile_size_width"), py::arg("tile_size_height"), py::arg("ray_origs"),
          py::arg("ray_dirs"), py::arg("ray_time_delta"), py::arg("tile_offsets"), py::arg("flatten_ids"),
          py::arg("pair_counts") = py::none(), py::arg("tile_work") = py::none());
    m.def("rasterize_eval3d_dynamic_bwd", &rasterize_eval3d_dynamic_bwd, py::arg("points"), py::arg("velocity"),
          py::arg("scale"), py::arg("quat"), py::arg("opacity"), py::arg("colors"), py::arg("ray_origins"),
          py::arg("ray_directions"), py::arg("ray_time_delta"), py::arg("tile_size_x"), py::arg("tile_size_y"),
          py::arg("tile_offsets"), py::arg("flatten_ids"), py::arg("render_alpha"), py::arg("last_ids"),
          py::arg("v_render_colors"), py::arg("v_render_depth"), py::arg("v_render_alpha"),
          py::arg("ray_grads") = true, py::arg("pair_counts") = py::none(),
          py::arg("pixels_per_lane") = 0, py::arg("tile_work") = py::none());
    // batched cameras (extension): C cameras over one scene in one launch per pass
    m.def("rasterize_eval3d_fwd_batched", &rasterize_eval3d_fwd_batched, py::arg("means"), py::arg("quats"),
          py::arg("scales"), py::arg("colors"), py::arg("opacities"), py::arg("image_width"), py::arg("image_height"),
          py::arg("tile_size_width"), py::arg("tile_size_height"), py::arg("ray_origs"), py::arg("ray_dirs"),
          py::arg("tile_offsets"), py::arg("flatten_ids"), py::arg("velocity") = py::none(),
          py::arg("ray_time_delta") = py::none(), py::arg("pair_counts") = py::none(),
          py::arg("tile_work") = py::none());
    m.def("rasterize_eval3d_bwd_batched", &rasterize_eval3d_bwd_batched, py::arg("points"), py::arg("scale"),
          py::arg("quat"), py::arg("opacity"), py::arg("colors"), py::arg("ray_origins"), py::arg("ray_directions"),
          py::arg("tile_size_x"), py::arg("tile_size_y"), py::arg("tile_offsets"), py::arg("flatten_ids"),
          py::arg("render_alpha"), py::arg("last_ids"), py::arg("v_render_colors"), py::arg("v_render_depth"),
          py::arg("v_render_alpha"), py::arg("velocity") = py::none(), py::arg("ray_time_delta") = py::none(),
          py::arg("ray_grads") = true, py::arg("pair_counts") = py::none(),
          py::arg("pixels_per_lane") = 0, py::arg("tile_work") = py::none());
    m.def("eval3d_supported_ndims", &eval3d_supported_ndims);

    // color (csrc/color/sh_bind.cpp)
    m.def("spherical_harmonics_fused_fwd", &spherical_harmonics_fused_fwd, py::arg("degree_to_use"),
          py::arg("origin"), py::arg("positions"), py::arg("coeffs"), py::arg("mask"), py::arg("layout_3kn"),
          py::arg("coeffs_dc") = py::none(), py::arg("output") = py::none());
    m.def("spherical_harmonics_fused_bwd", &spherical_harmonics_fused_bwd, py::arg("degree_to_use"),
          py::arg("origin"), py::arg("positions"), py::arg("coeffs"), py::arg("mask"), py::arg("layout_3kn"),
          py::arg("d_output"), py::arg("coeffs_dc") = py::none(), py::arg("origin_grad") = true);

    // tiling (csrc/tiling/bind_tiling.cpp)
    m.def("isect_offset_encode", &isect_offset_encode, py::arg("isect_ids"), py::arg("tile_width"),
          py::arg("tile_height"), py::arg("n_cams") = 1);
    m.def("isect_regular_tiles", &isect_regular_tiles, py::arg("means2d"), py::arg("radii"), py::arg("depth"),
          py::arg("img_width"), py::arg("img_height"), py::arg("tile_size_x"), py::arg("tile_size_y"),
          py::arg("sort") = true, py::arg("double_buffer") = true, py::arg("tile_offsets") = py::none(),
          py::arg("keys") = true);
    m.def("isect_regular_tiles_batched", &isect_regular_tiles_batched, py::arg("means2d"), py::arg("radii"),
          py::arg("depth"), py::arg("img_width"), py::arg("img_height"), py::arg("tile_size_x"),
          py::arg("tile_size_y"), py::arg("sort") = true, py::arg("tile_offsets") = py::none(),
          py::arg("keys") = true);
    m.def("isect_lidar_tiles", &isect_lidar_tiles, py::arg("camera_pack"), py::arg("points"),
          py::arg("points_velocity"), py::arg("scale"), py::arg("quat"), py::arg("opacity"), py::arg("flag"),
          py::arg("means2d"), py::arg("radii"), py::arg("depths"), py::arg("elev_boundaries"),
          py::arg("tile_size_x"), py::arg("img_width"), py::arg("img_height"), py::arg("ut_alpha") = 0.1f,
          py::arg("ut_beta") = 2.0f, py::arg("ut_kappa") = 0.0f, py::arg("sort") = true,
          py::arg("double_buffer") = true, py::arg("tile_offsets") = py::none(), py::arg("keys") = true);
    m.def("isect_spherical_tiles", &isect_spherical_tiles, py::arg("camera_pack"), py::arg("points"),
          py::arg("points_velocity"), py::arg("scale"), py::arg("quat"), py::arg("opacity"), py::arg("flag"),
          py::arg("means2d"), py::arg("radii"), py::arg("depths"), py::arg("tile_size_x"), py::arg("tile_size_y"),
          py::arg("img_width"), py::arg("img_height"), py::arg("ut_alpha") = 0.1f, py::arg("ut_beta") = 2.0f,
          py::arg("ut_kappa") = 0.0f, py::arg("sort") = true, py::arg("double_buffer") = true,
          py::arg("tile_offsets") = py::none(), py::arg("keys") = true);
    m.def("mask_radii_packed", &mask_radii_packed, py::arg("packed_mask"), py::arg("radii"));
    // scene-assembly producers (csrc/nodes/gs_masking.cu:44-47, container.cu:269-303)
    m.def("packed_mask_from_instances", &packed_mask_from_instances, py::arg("instance_ids"),
          py::arg("instance_mask"));
    // extension: the visibility mask of the regular tilings' Gaussians (an SH mask)
    m.def("packed_visibility_mask", &packed_visibility_mask, py::arg("radii"));
    // extension: the caller's parameter activations and their gradients
    m.def("activate_fwd", &activate_fwd, py::arg("log_scales"), py::arg("opacity_logits"));
    m.def("activate_bwd", &activate_bwd, py::arg("scales"), py::arg("opacities"), py::arg("v_scales"),
          py::arg("v_opacities"));
    m.def("copy_gs_rigid_transform_fwd", &copy_gs_rigid_transform_fwd, py::arg("positions"), py::arg("rotations"),
          py::arg("instance_id"), py::arg("inst_q"), py::arg("inst_t"), py::arg("inst_v"), py::arg("inst_w"),
          py::arg("inst_mask"), py::arg("out_positions"), py::arg("out_rotations"), py::arg("out_velocities"),
          py::arg("out_mask"), py::arg("buffer_offset"), py::arg("per_instance_offsets") = py::none(),
          py::arg("gs_inst_offsets") = py::none());
    m.def("copy_gs_rigid_transform_bwd", &copy_gs_rigid_transform_bwd, py::arg("positions"), py::arg("rotations"),
          py::arg("instance_id"), py::arg("inst_q"), py::arg("inst_w"), py::arg("inst_mask"), py::arg("buffer_offset"),
          py::arg("per_instance_offsets"), py::arg("gs_inst_offsets"), py::arg("v_positions"),
          py::arg("v_rotations"), py::arg("v_velocities"));
    m.def("mask_radii", &mask_radii, py::arg("mask"), py::arg("radii"));
    m.def("radix_sort_pairs", &radix_sort_pairs, py::arg("keys"), py::arg("values"), py::arg("begin_bit"),
          py::arg("end_bit"));

    // cameras (csrc/cameras/cameras_bind.h)
    py::module_ enum_mod = py::module_::import("enum");
    m.attr("ProjectionMode") = enum_mod.attr("IntEnum")(
        "ProjectionMode", py::dict(py::arg("Central") = (int)XSG_MODE_CENTRAL,
                                   py::arg("NegativeDelta") = (int)XSG_MODE_NEGATIVE,
                                   py::arg("PositiveDelta") = (int)XSG_MODE_POSITIVE));
    bind_camera<0>(m, "PerspectiveCamera", CamSpec{XSG_CAM_PINHOLE, {4}}, false);
    bind_camera<1>(m, "SphericalCamera", CamSpec{XSG_CAM_SPHERICAL, {4}}, true);
    bind_camera<2>(m, "LidarCamera", CamSpec{XSG_CAM_LIDAR, {4, 2}}, true);
    bind_camera<3>(m, "DistortedPerspectiveCamera", CamSpec{XSG_CAM_DISTORTED, {4, 8, 1}}, false);
    bind_camera<4>(m, "OpenCVFisheyeCamera", CamSpec{XSG_CAM_FISHEYE, {4, 4}}, false);
}
