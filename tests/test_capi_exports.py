"""The C-ABI library loads and exports every entry point that include/*.h declares.

CPU only: the library is loaded with ctypes and only its host-side queries are called (version,
pack sizes, workspace sizes, argument validation that fails before any launch).
"""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]
LIB = os.path.join(ROOT, "xsimgs_amd", "libxsimgs_hip.so")


def declared_symbols():
    text = "\n".join(open(h).read() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(xsg_\w+)\s*\(", text, flags=re.M)))


class Eval3dArgs(C.Structure):  # xsg_eval3d_args, field for field
    _fields_ = [("cdim", C.c_int), ("n", C.c_int64), ("n_cams", C.c_int)] + \
        [(k, C.c_void_p) for k in ("means", "quats", "scales", "colors", "opacities", "velocity",
                                   "ray_time_delta", "ray_o", "ray_d")] + \
        [(k, C.c_int) for k in ("width", "height", "tile_w", "tile_h", "n_tiles_w", "n_tiles_h")] + \
        [("tile_offsets", C.c_void_p), ("flatten_ids", C.c_void_p), ("n_isects", C.c_int64)] + \
        [(k, C.c_void_p) for k in ("out_rgb", "out_depth", "out_alpha", "out_last_ids", "render_alpha",
                                   "last_ids", "v_rgb", "v_depth", "v_alpha", "v_means", "v_quats",
                                   "v_scales", "v_opacities", "v_colors", "v_ray_o", "v_ray_d",
                                   "v_velocity", "v_time_delta", "pair_counts")] + \
        [("colors_shared", C.c_int), ("bwd_pixels_per_lane", C.c_int)]


class IsectDesc(C.Structure):  # xsg_isect_desc, field for field
    _fields_ = [("kind", C.c_int), ("n_cams", C.c_int), ("n", C.c_int64)] + \
        [(k, C.c_void_p) for k in ("means2d", "radii", "depths", "flags", "camera_pack", "points", "velocity",
                                   "scales", "quats", "opacity", "elev_boundaries")] + \
        [("n_elev", C.c_int), ("img_width", C.c_float), ("img_height", C.c_float), ("tile_w", C.c_int),
         ("tile_h", C.c_int), ("ut_alpha", C.c_float), ("ut_beta", C.c_float), ("ut_kappa", C.c_float),
         ("sort", C.c_int)]


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built: run __graft_entry__.build()")
    import torch  # noqa: F401  (loads torch's HIP runtime first, as the package does)
    return C.CDLL(LIB)


def test_header_declares_the_hot_path():
    syms = declared_symbols()
    for s in ("xsg_ut_project", "xsg_sh_fwd", "xsg_sh_bwd", "xsg_isect_count", "xsg_isect_fill",
              "xsg_isect_offset_encode", "xsg_radix_sort_pairs_u64_i32", "xsg_eval3d_fwd", "xsg_eval3d_bwd"):
        assert s in syms
    assert len(syms) >= 20


def test_every_declared_symbol_is_exported(lib):
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_host_queries(lib):
    lib.xsg_abi_version.restype = C.c_int
    assert lib.xsg_abi_version() == 3
    assert lib.xsg_camera_pack_elements(0) == 21
    assert lib.xsg_camera_pack_elements(1) == 21
    assert lib.xsg_camera_pack_elements(2) == 23
    assert lib.xsg_camera_pack_elements(7) < 0
    buf = (C.c_int * 64)()
    n = lib.xsg_eval3d_supported_ndims(buf, 64)
    assert list(buf[:n]) == [0, 1, 2, 3, 4, 5, 8, 9, 16, 17, 32, 33, 64, 65, 128, 129, 256, 257, 512, 513]
    lib.xsg_sh_bwd_workspace_bytes.restype = C.c_size_t
    lib.xsg_eval3d_bwd_workspace_bytes.restype = C.c_size_t
    lib.xsg_radix_sort_workspace_bytes.restype = C.c_size_t
    # the backward's workspace: 6 floats per Gaussian, then two int32 per (camera, tile)
    a = Eval3dArgs(cdim=3, n=1000, n_cams=2, n_tiles_w=120, n_tiles_h=68)
    assert lib.xsg_eval3d_bwd_workspace_bytes(C.byref(a)) >= 1000 * 6 * 4 + 2 * 2 * 120 * 68 * 4
    assert lib.xsg_eval3d_bwd_workspace_bytes(None) == 0
    assert lib.xsg_radix_sort_workspace_bytes(C.c_int64(1 << 20)) > 0
    # the measurement launch rejects an empty grid on the host
    assert lib.xsg_bench_valu_ceiling(0, 1, None, None, None) < 0
    # the allocation-free SH backward rejects sizes over its scratch limit on the host, before any
    # pointer is used or any HIP call is made
    vp = C.c_void_p
    lib.xsg_sh_bwd_noalloc.argtypes = [C.c_int, vp, C.c_int64, C.c_int, vp, vp, vp, C.c_int, vp, C.c_int, vp, vp,
                                       vp, vp, vp]
    lib.xsg_last_error.restype = C.c_char_p
    assert lib.xsg_sh_bwd_noalloc(3, None, (1 << 25) + 1, 16, None, None, None, 0, None, 0, None, None, None, None,
                                  None) == -1
    assert b"scratch limit" in lib.xsg_last_error()


def test_invalid_arguments_fail_before_launch(lib):
    lib.xsg_last_error.restype = C.c_char_p
    # SH degree outside 0..4 is rejected on the host
    rc = lib.xsg_sh_fwd(7, None, C.c_int64(1), 64, None, None, None, None, 0, None, None)
    assert rc == -1
    assert b"degree" in lib.xsg_last_error().lower()


def test_fill_without_keys_needs_tile_offsets(lib):
    """A sorted fill may leave the keys out (isect_ids NULL) only when it writes the tile offsets; an
    unsorted one, or one without offsets, fails on the host before any launch."""
    lib.xsg_last_error.restype = C.c_char_p
    d = IsectDesc(kind=0, n_cams=1, n=100, img_width=64.0, img_height=32.0, tile_w=16, tile_h=16, sort=1)
    nw, nh, tb, kb = C.c_int(), C.c_int(), C.c_int(), C.c_int()
    assert lib.xsg_isect_geometry(C.byref(d), C.byref(nw), C.byref(nh), C.byref(tb), C.byref(kb)) == 0
    assert (nw.value, nh.value) == (4, 2)
    fake = C.c_void_p(1 << 20)
    i64 = C.c_int64
    for sort, offs in ((1, None), (0, None)):
        rc = lib.xsg_isect_fill(C.byref(d), i64(10), i64(5), i64(5), sort, fake, fake, None, fake, offs,
                                i64(0), None)
        assert rc == -1
        assert b"keys may be left out" in lib.xsg_last_error()


def test_rig_projection_rejects_before_launch(lib):
    """xsg_ut_project_rig: phase-modelled kinds and a pack stride below the kind's pack size fail on
    the host; placeholder pointers are never dereferenced."""
    lib.xsg_last_error.restype = C.c_char_p
    fake = C.c_void_p(1 << 20)
    f = C.c_float
    args = lambda kind, stride: (kind, 2, fake, C.c_int64(stride), C.c_int64(10), fake, None, fake, fake, None,
                                 f(64), f(32), f(0.1), f(2.0), f(0.0), f(1e-4), f(2e-3), f(1.0), fake, fake, fake,
                                 fake, None)
    assert lib.xsg_ut_project_rig(*args(2, 23)) < 0
    assert b"pinhole, distorted or fisheye" in lib.xsg_last_error()
    assert lib.xsg_ut_project_rig(*args(0, 20)) == -1
    assert b"pack stride" in lib.xsg_last_error()


def test_misaligned_workspace_is_rejected_before_launch(lib):
    """Workspaces must be 256-byte aligned; the pointers here are placeholders that no call reaches."""
    lib.xsg_last_error.restype = C.c_char_p
    fake = C.c_void_p(1 << 20)
    sel = C.c_int(0)
    rc = lib.xsg_radix_sort_pairs_u64_i32(fake, fake, fake, fake, C.c_int64(1000), 0, 32,
                                          C.c_void_p((1 << 20) + 16), C.byref(sel), None)
    assert rc < 0
    assert b"aligned" in lib.xsg_last_error()
    rc = lib.xsg_sh_bwd(3, fake, C.c_int64(10), 16, fake, fake, None, 0, fake, 0, fake, None, fake, fake,
                        C.c_void_p((1 << 20) + 4), None)
    assert rc < 0
    assert b"aligned" in lib.xsg_last_error()
