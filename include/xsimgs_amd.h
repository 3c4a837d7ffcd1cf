/*
 * xsimgs_amd C-ABI: the Gaussian-splatting rasterization hot path of xsimgs on MI355X (gfx950).
 *
 * Every entry point takes device pointers, explicit sizes and a HIP stream, never allocates
 * device memory (scratch comes in through a `workspace` argument sized by the matching
 * *_workspace_bytes query and aligned to 256 bytes, as hipMalloc returns it; a misaligned one is
 * rejected with XSG_ERR_INVALID), and returns XSG_OK or a negative error code; xsg_last_error()
 * then holds a message (thread-local). Work is enqueued on `stream`; the only blocking call is
 * xsg_isect_count, which copies the intersection total to the host (as the reference's
 * `.item()` does); the pinned host buffer it reads that through is the C-ABI's one host allocation
 * (per host thread and device, freed by xsg_release_thread_resources).
 *
 * Reference interfaces replaced (whesense/xsimgs, pybind module xsimgs._C):
 *   xsg_ut_project            <Camera>.projection_utgs[_phm]   include/cameras/bind.h:82-114,
 *                             ut_kernels.h:249-305, ut_phm_kernels.h:125-173
 *   xsg_project_points        <Camera>.projection[_nojac]       bind.h:66-81, projection_kernels.h:259-309
 *   xsg_camera_rays           <Camera>.camera_rays (forward)    bind.h:47-53, ray_kernels.h:7-59
 *   xsg_pixel_time*           <Camera>.pixel_time*              bind.h:54-65, time_kernels.h:5-241
 *   xsg_undistort_map         <Camera>.undistort_map            distortion.h:33-56
 *   xsg_camera_rays_bwd       camera_ray_backward               ray_kernels.h:61-161
 *   xsg_pixel_time_bwd        pixel_time*_backward              time_kernels.h:123-330
 *   xsg_sh_fwd / xsg_sh_bwd   spherical_harmonics_fused_{fwd,bwd} csrc/color/sh_fwd.cu:248-259,
 *                             sh_bwd.cu:379-390
 *   xsg_mask_radii[_packed]   mask_radii / mask_radii_packed    csrc/tiling/mask_radii.cu:82-88
 *   xsg_packed_mask_from_instances
 *                             packed_mask_from_instances        csrc/nodes/gs_masking.cu:8-47
 *   xsg_rigid_transform_fwd / _bwd
 *                             copy_gs_rigid_transform_{fwd,bwd} csrc/nodes/container.cu:13-266
 *   xsg_isect_count + xsg_isect_fill
 *                             isect_regular_tiles / isect_lidar_tiles / isect_spherical_tiles
 *                             regular_tiling.cu:138-146, phm_lidar_tiling.cu:354-375,
 *                             phm_spherical_tiling.cu:294-314
 *   xsg_radix_sort_pairs_u64_i32
 *                             sort_intersections (cub SortPairs) tiling_common.cu:102-162
 *   xsg_isect_offset_encode   isect_offset_encode               tiling_common.cu:165-168
 *   xsg_eval3d_fwd / xsg_eval3d_bwd (static and dynamic)
 *                             rasterize_eval3d_[dynamic_]{fwd,bwd} eval3d_fwd.cu:310-316,
 *                             eval3d_bwd.cu:406-408, eval3d_dynamic_fwd.cu:325-332,
 *                             eval3d_dynamic_bwd.cu:322-432
 *   xsg_eval3d_supported_ndims eval3d_supported_ndims           eval3d_bind.cpp:12-15
 */
#ifndef XSIMGS_AMD_H
#define XSIMGS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XSG_ABI_VERSION 3

/* return codes */
#define XSG_OK 0
#define XSG_ERR_INVALID (-1)     /* bad argument (shape, dtype-implied size, degree, CDIM ...) */
#define XSG_ERR_LDS (-2)         /* tile too large for the local data share */
#define XSG_ERR_LAUNCH (-3)      /* HIP launch / runtime failure */
#define XSG_ERR_UNSUPPORTED (-4) /* feature not provided by this build */

/* camera kinds and projection modes (enum class ProjectionMode, include/cameras/camera.h:15-19) */
#define XSG_CAM_PINHOLE 0
#define XSG_CAM_SPHERICAL 1
#define XSG_CAM_LIDAR 2
#define XSG_CAM_DISTORTED 3
#define XSG_CAM_FISHEYE 4
#define XSG_MODE_CENTRAL 0
#define XSG_MODE_NEGATIVE 1
#define XSG_MODE_POSITIVE 2

/* tiling kinds */
#define XSG_TILING_REGULAR 0    /* isect_regular_tiles: exclusive rectangle, flags ignored */
#define XSG_TILING_LIDAR 1      /* isect_lidar_tiles: irregular elevation grid, inclusive */
#define XSG_TILING_SPHERICAL 2  /* isect_spherical_tiles: regular angular grid, exclusive */

typedef struct ihipStream_t* xsg_stream_t; /* == hipStream_t */

const char* xsg_last_error(void);
int xsg_abi_version(void);

/* Number of float32 elements of a camera pack of `kind` (pinhole/spherical 21, lidar 23,
 * distorted perspective 30, OpenCV fisheye 25).
 * Replaces Camera<Impl>::pack_elements (camera.h:141-143); the layout is documented in
 * xsimgs_amd/csrc/xsg_common.h. */
int xsg_camera_pack_elements(int kind);

/* ---------------------------------------------------------------- cameras */
int xsg_ut_project(int kind, int phm, const float* pack, int64_t n, const float* means,
                   const float* velocity, const float* scales, const float* quats,
                   const float* opacity, float width, float height, float ut_alpha, float ut_beta,
                   float ut_kappa, float residual_thr, float max_residual, float max_margin,
                   uint8_t* flags, float* radii, float* means2d, float* depths, xsg_stream_t stream);

/* Extension, no reference counterpart (the reference projects one camera per call,
 * ut_kernels.h:249-305): the UT projection of one scene by n_cams cameras of one kind (pinhole,
 * distorted or fisheye), packs [n_cams] at a stride of pack_stride floats; each Gaussian is read once
 * and projected with every camera as xsg_ut_project does. Outputs are [n_cams, n] camera-major. */
int xsg_ut_project_rig(int kind, int n_cams, const float* packs, int64_t pack_stride, int64_t n,
                       const float* means, const float* velocity, const float* scales, const float* quats,
                       const float* opacity, float width, float height, float ut_alpha, float ut_beta,
                       float ut_kappa, float residual_thr, float max_residual, float max_margin,
                       uint8_t* flags, float* radii, float* means2d, float* depths, xsg_stream_t stream);

int xsg_project_points(int kind, const float* pack, int64_t n, const float* points,
                       const float* velocity, float residual_thr, float max_residual,
                       float max_margin, int mode, int no_jacobian, float* uvdt, uint8_t* mask,
                       xsg_stream_t stream);

int xsg_camera_rays(int kind, const float* pack, int width, int height, int world_space,
                    int normalized, float* ray_o, float* ray_d, uint8_t* valid,
                    xsg_stream_t stream);

/* <Camera>.undistort_map (distortion.h:33-56) of the distorted perspective and fisheye models: per
 * pixel (float2, row-major [height, width]) the distorted image position of the pixel's undistorted
 * uv, in [0, 1] with normalized_range, else in [-1, 1] */
int xsg_undistort_map(int kind, const float* pack, int width, int height, int normalized_range, float* out,
                      xsg_stream_t stream);

/* per-pixel (uv == NULL) or per-uv capture time; `delta` subtracts the pose time */
int xsg_pixel_time(int kind, const float* pack, int width, int height, const float* uv, int64_t n_uv,
                   int delta, float* out, xsg_stream_t stream);

/* Gradient of sum(d_ray_o * ray_o + d_ray_d * ray_d) w.r.t. the camera pack (camera_ray_backward,
 * ray_kernels.h:61-161). grad_pack gets all xsg_camera_pack_elements(kind) values in pack order
 * (q0, t0, v, w, rolling_time, trigger_time, pose_time, the model's tensors; 0 for the lidar beam
 * address and the distorted model's max_radius^2);
 * it needs no zero-initialisation. d_ray_o may be NULL (no origin gradient). The sum over pixels
 * is deterministic: per-block partials in `workspace`, then one fixed-order reduction. */
size_t xsg_camera_rays_bwd_workspace_bytes(int width, int height);
int xsg_camera_rays_bwd(int kind, const float* pack, int width, int height, int world_space,
                        int normalized, const float* d_ray_o, const float* d_ray_d, float* grad_pack,
                        void* workspace, xsg_stream_t stream);

/* Gradient of sum(grad * time) for xsg_pixel_time's output w.r.t. the pack (rolling_time,
 * trigger_time and, with `delta`, pose_time; every other element 0) and, when uv is given and
 * d_uv is not NULL, w.r.t. uv (d_uv[i] = grad[i] * rolling_time). time_kernels.h:123-330. */
size_t xsg_pixel_time_bwd_workspace_bytes(int width, int height, int64_t n_uv);
int xsg_pixel_time_bwd(int kind, const float* pack, int width, int height, const float* uv,
                       int64_t n_uv, int delta, const float* grad, float* grad_pack, float* d_uv,
                       void* workspace, xsg_stream_t stream);

/* ------------------------------------------------------- spherical harmonics */
int xsg_sh_fwd(int degree, const float* origin, int64_t n, int dim, const float* positions,
               const float* coeffs, const float* coeffs_dc, const uint32_t* mask, int layout_3kn,
               float* out, xsg_stream_t stream);
/* Extension (no counterpart in the reference): xsg_sh_fwd that, with zero_masked != 0, writes zeros
 * to the rows the mask excludes instead of leaving them as the caller had them, so a caller with a
 * fresh output buffer needs no separate fill. zero_masked = 0 is xsg_sh_fwd. */
int xsg_sh_fwd_ex(int degree, const float* origin, int64_t n, int dim, const float* positions,
                  const float* coeffs, const float* coeffs_dc, const uint32_t* mask, int layout_3kn,
                  int zero_masked, float* out, xsg_stream_t stream);

size_t xsg_sh_bwd_workspace_bytes(int64_t n);
/* d_coeffs (every band written), d_coeffs_dc (if has_dc), d_positions and d_origin[3] are outputs;
 * none needs zero-initialisation. d_origin may be NULL (an extension): the origin gradient, a sum over
 * every Gaussian, is then not computed. */
int xsg_sh_bwd(int degree, const float* origin, int64_t n, int dim, const float* positions,
               const float* coeffs, const uint32_t* mask, int layout_3kn, const float* d_output,
               int has_dc, float* d_coeffs, float* d_coeffs_dc, float* d_positions,
               float* d_origin, void* workspace, xsg_stream_t stream);

/* xsg_sh_bwd without a workspace. No counterpart in the reference: for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). The
 * per-block d_origin partials live in a file-scope device array of this library instead, one per GPU
 * (1.5 MiB, held until the process ends), sized for n <= XSG_SH_BWD_NOALLOC_MAX_N Gaussians; a larger
 * n is rejected with XSG_ERR_INVALID before anything runs. It calls no allocator. Every call on one GPU
 * shares that array: calls that overlap on a GPU (several streams or host threads) race and must be
 * serialised by the caller. Outputs as xsg_sh_bwd; the stream must belong to the current device. */
#define XSG_SH_BWD_NOALLOC_MAX_N (1LL << 25)
int xsg_sh_bwd_noalloc(int degree, const float* origin, int64_t n, int dim, const float* positions,
                       const float* coeffs, const uint32_t* mask, int layout_3kn, const float* d_output,
                       int has_dc, float* d_coeffs, float* d_coeffs_dc, float* d_positions,
                       float* d_origin, xsg_stream_t stream);

/* ------------------------------------------------- scene-assembly producers */
/* packed_mask_from_instances (gs_masking.cu:8-47): out[(n + 31) / 32], bit i % 32 of word i / 32 set
 * when instance_ids[i] < 0 or instance_mask[instance_ids[i]] != 0. Ids at or past n_instances count
 * as enabled (the reference reads past the mask there). */
int xsg_packed_mask_from_instances(int64_t n, const int32_t* instance_ids, const uint8_t* instance_mask,
                                   int64_t n_instances, uint32_t* out, xsg_stream_t stream);

/* Gaussians and instances of copy_gs_rigid_transform_{fwd,bwd} (container.cu:13-266). Gaussian i of
 * instance k = instance_ids[i] goes to row buffer_offset + i, or buffer_offset +
 * per_instance_offsets[k] + gs_inst_offsets[i] when both offset arrays are given; Gaussians of a
 * disabled instance (inst_mask[k] == 0), with k outside [0, n_instances) or with a row outside
 * [0, n_out) are skipped. Quaternions are (w, x, y, z), float4-aligned. */
typedef struct {
    int64_t n;              /* Gaussians */
    int64_t n_instances;
    int64_t n_out;          /* rows of the output buffers */
    int64_t buffer_offset;
    const float* positions;       /* [n, 3] */
    const float* rotations;       /* [n, 4] */
    const int32_t* instance_ids;  /* [n] */
    const float* inst_q;          /* [n_instances, 4] */
    const float* inst_t;          /* [n_instances, 3] (forward only) */
    const float* inst_v;          /* [n_instances, 3] (forward only) */
    const float* inst_w;          /* [n_instances, 3] */
    const uint8_t* inst_mask;     /* [n_instances] */
    const int32_t* per_instance_offsets;  /* [n_instances] or NULL */
    const int32_t* gs_inst_offsets;       /* [n] or NULL */
} xsg_rigid_desc;

/* out_pos = q_k p + t_k, out_rot = q_k (x) q, out_vel = v_k + w_k x (q_k p), out_mask = 1, written
 * in place at each Gaussian's row; other rows are left untouched. out_velocities and out_mask may be
 * NULL. */
int xsg_rigid_transform_fwd(const xsg_rigid_desc* d, float* out_positions, float* out_rotations,
                            float* out_velocities, uint8_t* out_mask, xsg_stream_t stream);

/* Gradients of the forward: grad_positions [n, 3] and grad_rotations [n, 4] (zeros for skipped
 * Gaussians) and the per-instance sums grad_q [n_instances, 4], grad_t, grad_v, grad_w
 * [n_instances, 3]; every output is written (no zero-fill needed). v_velocities may be NULL (then
 * grad_v and grad_w are 0). The instance sums are accumulated with float atomics in `workspace`
 * (xsg_rigid_transform_bwd_workspace_bytes(n_instances) bytes): their summation order varies. */
size_t xsg_rigid_transform_bwd_workspace_bytes(int64_t n_instances);
int xsg_rigid_transform_bwd(const xsg_rigid_desc* d, const float* v_positions, const float* v_rotations,
                            const float* v_velocities, float* grad_positions, float* grad_rotations,
                            float* grad_q, float* grad_t, float* grad_v, float* grad_w, void* workspace,
                            xsg_stream_t stream);

/* Extension, no reference counterpart: the Gaussians some tile of a regular tiling can hold, as a packed
 * mask in packed_mask_from_instances's format (out[(n + 31) / 32], bit i % 32 of word i / 32): set when
 * some camera's radii of Gaussian i (radii [n_cams, n, 2], camera-major, as the UT projection writes
 * them) pass the tiling's test, i.e. are not (r.x <= 0 or r.y <= 0). A caller that evaluates SH colours
 * after the projection passes it as the SH mask, so that the colours of Gaussians no tile holds, which
 * the compositor never reads, are not evaluated. */
int xsg_packed_visibility_from_radii(int64_t n, int n_cams, const float* radii, uint32_t* out,
                                     xsg_stream_t stream);

/* Extension, no reference counterpart: the parameter activations a training caller applies before
 * the path (torch.exp of the log-scales, torch.sigmoid of the opacity logits; the reference takes
 * activated scales and opacities, render.py:85-96) in one launch, and their gradients in one
 * launch: scales [n, 3] = exp(log_scales), opacities [n] = sigmoid(opacity_logits);
 * v_log_scales = v_scales * scales, v_opacity_logits = v_opacities * (1 - opacities) * opacities,
 * bit-identical to torch's kernels. In the backward either gradient pair may be NULL (that output
 * is then not written). */
int xsg_activate_fwd(int64_t n, const float* log_scales, const float* opacity_logits, float* scales,
                     float* opacities, xsg_stream_t stream);
int xsg_activate_bwd(int64_t n, const float* scales, const float* opacities, const float* v_scales,
                     const float* v_opacities, float* v_log_scales, float* v_opacity_logits,
                     xsg_stream_t stream);

/* ------------------------------------------------------------------ binning */
int xsg_mask_radii(int64_t n, const uint8_t* mask, float* radii, xsg_stream_t stream);
int xsg_mask_radii_packed(int64_t n, const uint32_t* packed_mask, float* radii, xsg_stream_t stream);

typedef struct {
    int kind;                 /* XSG_TILING_* */
    int n_cams;               /* >= 1; inputs are [n_cams, n] camera-major, keys carry the camera id */
    int64_t n;                /* Gaussians per camera */
    const float* means2d;     /* [n_cams, n, 2] pixels */
    const float* radii;       /* [n_cams, n, 2] */
    const float* depths;      /* [n_cams, n] */
    const uint8_t* flags;     /* [n_cams, n]; lidar / spherical only */
    /* lidar / spherical seam re-projection (flag == 2); NULL for regular tiling */
    const float* camera_pack;
    const float* points;      /* [n, 3] */
    const float* velocity;    /* [n, 3] or NULL */
    const float* scales;      /* [n, 3] */
    const float* quats;       /* [n, 4] */
    const float* opacity;     /* [n] or NULL */
    const float* elev_boundaries; /* lidar: [n_elev] */
    int n_elev;
    float img_width, img_height;  /* image size (float, as the reference lidar/spherical ops take it) */
    int tile_w, tile_h;
    float ut_alpha, ut_beta, ut_kappa;
    int sort;                 /* 1 when xsg_isect_fill will sort: xsg_isect_count then also orders the
                                 spans by depth before its readback; xsg_isect_fill must get the same */
} xsg_isect_desc;

/* geometry derived from a descriptor: tiles along u / v, tile count, key bits above 32 */
int xsg_isect_geometry(const xsg_isect_desc* d, int* n_tiles_w, int* n_tiles_h, int* tile_n_bits,
                       int* key_bits_above_32);

size_t xsg_isect_count_workspace_bytes(const xsg_isect_desc* d);
/* Pass 1: tiles per Gaussian into tiles_per_gauss [n_cams*n]; on the host, *n_isects receives the
 * total, *n_visible the number of non-empty spans and *n_runs the number of (span, tile row) runs,
 * which xsg_isect_fill takes back. Blocks on `stream` for that one device->host copy.
 * `workspace` carries state into xsg_isect_fill.
 * Host resources: the totals arrive in a 64-byte mapped pinned host buffer (hipHostMalloc) with one
 * event, created on a host thread's first call on a device and reused by that thread's later calls
 * on it; they stay allocated until that thread calls xsg_release_thread_resources. */
int xsg_isect_count(const xsg_isect_desc* d, int32_t* tiles_per_gauss, void* workspace,
                    int64_t* n_isects, int64_t* n_visible, int64_t* n_runs, xsg_stream_t stream);

/* Frees the calling host thread's xsg_isect_count readback buffers and events (every device it used;
 * a later count allocates them again). A caller whose binding threads end, or that wants the pinned
 * memory back, calls it from each such thread once its counts have returned. No reference
 * counterpart: the reference reads its totals with `.item()` through torch's allocator
 * (regular_tiling.cu:112, phm_lidar_tiling.cu:316). */
int xsg_release_thread_resources(void);

size_t xsg_isect_fill_workspace_bytes(const xsg_isect_desc* d, int64_t n_isects, int64_t n_visible,
                                      int64_t n_runs);
/* Pass 2: intersection keys ((cam | tile) << 32 | depth bits) and flattened Gaussian ids
 * (cam * n + gaussian); sorted by key bits [0, 32 + key_bits_above_32) with ties in fill order
 * when `sort`, else in the reference's fill order. Consumes (overwrites) count_workspace.
 * tile_offsets (optional, sorted fills only; NULL skips it): the n_tile_offsets =
 * n_cams * n_tiles_h * n_tiles_w offsets that xsg_isect_offset_encode would compute from the
 * sorted keys, produced by the fill itself (extension: it saves the search that
 * isect_offset_encode, tiling_common.cu:25-71, runs over the keys).
 * isect_ids may be NULL in a sorted fill that writes tile_offsets (extension): the keys are then not
 * written, as a renderer that takes the offsets never reads them (rendering/render.py:45-81 uses
 * them only to encode the offsets). */
int xsg_isect_fill(const xsg_isect_desc* d, int64_t n_isects, int64_t n_visible, int64_t n_runs,
                   int sort, void* count_workspace, void* fill_workspace, int64_t* isect_ids,
                   int32_t* flatten_ids, int32_t* tile_offsets, int64_t n_tile_offsets, xsg_stream_t stream);

/* offsets [n_cams, n_tiles_h, n_tiles_w]: first sorted index of every (camera, tile). Keys of a
 * negative depth (sign-extended bits, all ones above bit 31) sort after every tile; the offsets are
 * those of the other keys (the reference's encoder races on them, tiling_common.cu:41-60). The
 * compositor's last tile runs to n_isects (utils.h:52-57), so it composites those entries after its
 * own, as the reference's compositor does. */
int xsg_isect_offset_encode(const int64_t* isect_ids, int64_t n_isects, int n_tiles_w, int n_tiles_h,
                            int n_cams, int32_t* offsets, xsg_stream_t stream);

/* Stable LSD radix sort of (key, value) pairs by key bits [begin_bit, end_bit).
 * The sorted data ends in (keys, vals) when *selector == 0, else in (keys_alt, vals_alt). */
size_t xsg_radix_sort_workspace_bytes(int64_t n);
int xsg_radix_sort_pairs_u64_i32(int64_t* keys, int32_t* vals, int64_t* keys_alt, int32_t* vals_alt,
                                 int64_t n, int begin_bit, int end_bit, void* workspace,
                                 int* selector, xsg_stream_t stream);

/* ------------------------------------------------------------ compositing */
/* Writes the supported colour dimensions (common.h:5-25) into out[0..cap) and returns their count. */
int xsg_eval3d_supported_ndims(int* out, int cap);

typedef struct {
    int cdim;                      /* colour channels; 0 = no colours */
    int64_t n;                     /* Gaussians */
    int n_cams;                    /* >= 1; cameras batched camera-major */
    const float* means;            /* [n, 3] */
    const float* quats;            /* [n, 4] (w, x, y, z), normalised inside */
    const float* scales;           /* [n, 3] activated */
    const float* colors;           /* [n_cams, n, cdim] ([n, cdim] if colors_shared) or NULL */
    const float* opacities;        /* [n] activated */
    const float* velocity;         /* dynamic scenes: [n, 3], else NULL */
    const float* ray_time_delta;   /* dynamic scenes: [n_cams, H, W], else NULL */
    const float* ray_o;            /* [n_cams, H, W, 3] */
    const float* ray_d;            /* [n_cams, H, W, 3] */
    int width, height, tile_w, tile_h, n_tiles_w, n_tiles_h;
    const int32_t* tile_offsets;   /* [n_cams, n_tiles_h, n_tiles_w] */
    const int32_t* flatten_ids;    /* [n_isects], values cam * n + gaussian */
    int64_t n_isects;
    /* forward outputs */
    float* out_rgb;                /* [n_cams, H, W, cdim] */
    float* out_depth;              /* [n_cams, H, W] */
    float* out_alpha;              /* [n_cams, H, W] */
    int32_t* out_last_ids;         /* [n_cams, H, W] */
    /* backward inputs */
    const float* render_alpha;
    const int32_t* last_ids;
    const float* v_rgb;            /* [n_cams, H, W, cdim] or NULL */
    const float* v_depth;
    const float* v_alpha;
    /* backward outputs: accumulated with atomics, zero-initialised by xsg_eval3d_bwd itself */
    float* v_means;
    float* v_quats;
    float* v_scales;
    float* v_opacities;
    float* v_colors;               /* NULL when cdim == 0 */
    float* v_ray_o;                /* both NULL: per-pixel ray gradients are not computed */
    float* v_ray_d;
    float* v_velocity;             /* dynamic only */
    float* v_time_delta;           /* dynamic only */
    /* optional (NULL: not counted): pair_counts[0] += (pixel, Gaussian) pairs whose alpha was
     * evaluated (backward: pairs at or before the pixel's last id), pair_counts[1] += pairs that were
     * composited; the caller initialises them. Pairs that no pixel of a wavefront can take are
     * skipped unevaluated and not counted. */
    uint64_t* pair_counts;
    /* 0: colors are [n_cams, n, cdim] and v_colors likewise; 1: colors [n, cdim] are shared by every
     * camera (a rig whose cameras share one origin sees one set of view-dependent colours) and
     * v_colors [n, cdim] receives the sum over cameras. An extension of this build. */
    int colors_shared;
    /* backward only, tiles of 129 to 256 pixels without per-pixel ray gradients: pixels per lane, 4 (a
     * wavefront per 16x16 tile) or 2 (two), or 0 to choose: 4 when the grid fills the GPU's wave slots
     * (3 x 1024 wavefronts), else 2. The gradients agree to float32 rounding either way. An extension. */
    int bwd_pixels_per_lane;
    /* optional, [n_cams * n_tiles_h * n_tiles_w]: per (camera, tile) the backward's work estimate, the
     * number of the tile's intersections up to its pixels' largest last id. xsg_eval3d_fwd writes it
     * when non-NULL; xsg_eval3d_bwd reads it when non-NULL instead of deriving it from last_ids (a
     * pass over every pixel). It only orders the backward's tiles: any values give the same
     * gradients up to float32 rounding of the atomic sums. An extension. */
    int32_t* tile_work;
} xsg_eval3d_args;

int xsg_eval3d_fwd(const xsg_eval3d_args* a, xsg_stream_t stream);
/* Workspace of xsg_eval3d_bwd for these arguments (sizes only are read): the per-Gaussian
 * accumulators of the symmetric M gradient (6 floats per Gaussian) and, per (camera, tile), its work
 * estimate and the order in which the tiles are launched (two int32). */
size_t xsg_eval3d_bwd_workspace_bytes(const xsg_eval3d_args* a);
int xsg_eval3d_bwd(const xsg_eval3d_args* a, void* workspace, xsg_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
