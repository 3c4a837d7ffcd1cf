"""GPU parity of every hot-path stage against the CPU oracle, on identical seeded inputs.

Each stage is fed the same inputs on both sides (the GPU's own upstream results), so a stage is
judged on its own: binning, sort and tile ranges must be bit-exact; renders within 1e-4 absolute;
gradients within 1e-3 relative with a 1e-5 absolute floor.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from xsimgs_amd import _C, frame, synthetic
from tests import _judge as J
from tests._util import GRAD_ATOL, GRAD_RTOL, RENDER_ATOL, frac_close, np_, report

pytestmark = pytest.mark.gpu


def _cam_pack(spec, dev):
    return frame.make_camera(spec, dev).pack


@pytest.fixture(scope="module")
def cfg0(dev):
    sc = synthetic.make_cfg0()
    st = frame.prepare(sc, dev, requires_grad=False)
    return sc, st


# ------------------------------------------------------------------ SH
@pytest.mark.parametrize("degree,layout_3kn,with_dc,with_mask,sparse", [
    (0, False, False, False, False), (3, False, False, False, False), (3, True, False, False, False),
    (3, False, True, True, False), (4, True, True, False, False), (2, False, False, True, False),
    (1, True, False, True, False), (3, False, False, False, True), (3, True, False, False, True),
    (4, False, True, True, True), (3, False, False, True, True), (2, False, True, True, True)])
def test_sh_fwd_bwd(dev, degree, layout_3kn, with_dc, with_mask, sparse):
    """sparse: the colour gradient is zero for most Gaussians (those no tile composited), as in a
    frame; the backward then reads coefficients only for the rows that need them, except in blocks
    of 256 Gaussians where most do (here: the first block dense, the second at about a third). With a
    mask, sparse also thins the mask (most bits clear past the first block, as a frame's visibility
    mask is), so that the forward reads the rows of sparse blocks one by one."""
    g = torch.Generator().manual_seed(7 + degree)
    n = 3001
    K = (degree + 1) ** 2 + 2            # extra unused bands must come back zero in d_coeffs
    pos = torch.randn(n, 3, generator=g) * 5
    origin = torch.tensor([0.3, -0.2, 0.1])
    kb = K - (1 if with_dc else 0)
    coeffs = torch.randn(3, kb, n, generator=g) if layout_3kn else torch.randn(n, kb, 3, generator=g)
    dc = (torch.randn(3, n, generator=g) if layout_3kn else torch.randn(n, 3, generator=g)) if with_dc else None
    mask = torch.randint(-2**31, 2**31 - 1, ((n + 31) // 32,), generator=g, dtype=torch.int32) if with_mask else None
    if with_mask and sparse:
        bits = torch.rand(n, generator=g) < 0.08
        bits[:256] = torch.rand(256, generator=g) < 0.6
        words = np.packbits(np.pad(bits.numpy(), (0, 32 * ((n + 31) // 32) - n)), bitorder="little")
        mask = torch.from_numpy(words.view(np.int32).copy())
    d_out = torch.randn(n, 3, generator=g)
    if sparse:
        keep = torch.rand(n, generator=g) < 0.12
        keep[:256] = True
        keep[256:512] = torch.rand(256, generator=g) < 0.35
        d_out[~keep] = 0.0
        d_out[keep.nonzero()[::7, 0], 1:] = 0.0   # a gradient zero in some channels only still needs them
    D = lambda t: None if t is None else t.to(dev)
    out = _C.spherical_harmonics_fused_fwd(degree, D(origin), D(pos), D(coeffs), D(mask), layout_3kn, D(dc))
    m_np = None if mask is None else mask.numpy().view(np.uint32)
    ref = O.sh_fwd(degree, origin, pos, coeffs, dc=dc, mask=m_np, layout_3kn=layout_3kn)
    print(report("sh_fwd", np_(out), ref))
    assert frac_close(np_(out), ref, RENDER_ATOL) == 1.0
    dco, ddc, dpos, dori = _C.spherical_harmonics_fused_bwd(degree, D(origin), D(pos), D(coeffs), D(mask),
                                                            layout_3kn, D(d_out), D(dc))
    rdco, rddc, rdpos, rdori = O.sh_bwd(degree, origin, pos, coeffs, d_out, dc=dc, mask=m_np, layout_3kn=layout_3kn)
    for name, a, b in (("d_coeffs", dco, rdco), ("d_dc", ddc, rddc), ("d_pos", dpos, rdpos), ("d_origin", dori, rdori)):
        print(report(name, np_(a), b))
        assert np_(a).shape == b.shape, name
        assert frac_close(np_(a), b, GRAD_ATOL, GRAD_RTOL) == 1.0, name
    # origin_grad=False (extension): no origin gradient, the same bits for everything else
    nco, ndc, npos, nori = _C.spherical_harmonics_fused_bwd(degree, D(origin), D(pos), D(coeffs), D(mask),
                                                            layout_3kn, D(d_out), D(dc), origin_grad=False)
    assert nori is None
    for a, b in ((nco, dco), (ndc, ddc), (npos, dpos)):
        assert torch.equal(a, b)


# ------------------------------------------------------------------ projection, rays
def test_ut_projection_pinhole(dev, cfg0):
    """Flags equal to the oracle's except where float32 does not decide them; value errors no worse
    than the float32 oracle's (tests/_judge.py); culled Gaussians all zeros."""
    sc, st = cfg0
    spec = sc.cameras[0]
    pack = _cam_pack(spec, dev)
    got = _C.PerspectiveCamera.projection_utgs(
        pack, st.means, None, torch.exp(st.log_scales), st.quats, torch.sigmoid(st.opacity_logits),
        spec.width, spec.height)
    J.judge_ut(got, spec, sc.means.numpy(), sc.scales.numpy(), sc.quats.numpy(), sc.opacity.numpy(), spec.width,
               spec.height, label="cfg0")


@pytest.mark.parametrize("cfg", ["cfg0", "cfg3"])
def test_camera_rays(dev, cfg):
    sc = synthetic.make_cfg0() if cfg == "cfg0" else synthetic.make_cfg3(n=1000)
    spec = sc.cameras[0]
    cam = frame.make_camera(spec, dev)
    ro, rd = cam.camera_rays(spec.width, spec.height)
    rro, rrd = O.camera_rays(spec, spec.width, spec.height)
    print(report("ray_d", np_(rd), rrd))
    assert np.abs(np_(ro) - rro).max() <= 1e-6
    assert np.abs(np_(rd) - rrd).max() <= 2e-6


# ------------------------------------------------------------------ binning
def _ut(st, spec, dev, phm=False):
    cam = frame.make_camera(spec, dev)
    fn = cam.ext_cls.projection_utgs_phm if phm else cam.ext_cls.projection_utgs
    return cam, fn(cam.pack, st.means, None, torch.exp(st.log_scales), st.quats,
                   torch.sigmoid(st.opacity_logits), spec.width, spec.height)


@pytest.mark.parametrize("sort", [True, False])
def test_isect_regular_bitexact(dev, cfg0, sort):
    sc, st = cfg0
    spec = sc.cameras[0]
    _, (flags, radii, m2, dep) = _ut(st, spec, dev)
    tpg, ids, fl = _C.isect_regular_tiles(m2, radii, dep, spec.width, spec.height, 16, 16, sort=sort)
    rtpg, rids, rfl = O.isect_regular(np_(m2), np_(radii), np_(dep), spec.width, spec.height, 16, 16, sort=sort)
    assert np.array_equal(np_(tpg), rtpg)
    assert np.array_equal(np_(ids), rids)
    assert np.array_equal(np_(fl), rfl)
    if sort:  # tile ranges are defined for sorted keys only (the reference's encoder races otherwise)
        off = _C.isect_offset_encode(ids, 16, 16)
        assert np.array_equal(np_(off), O.offset_encode(rids, 16, 16))


@pytest.mark.parametrize("layout_3kn", [False, True])
def test_sh_fwd_ex_zero_masked(dev, layout_3kn):
    """xsg_sh_fwd_ex (an extension) through the C-ABI: with zero_masked the rows the mask excludes
    become zeros, without it they keep what the buffer held, as xsg_sh_fwd leaves them; the other rows
    are the oracle's either way."""
    import ctypes
    from xsimgs_amd import _build
    lib = ctypes.CDLL(_build.lib_path())
    n, degree, dim = 1000, 3, 16
    g = np.random.default_rng(5)
    pos = g.normal(size=(n, 3)).astype(np.float32)
    origin = np.array([0.1, -0.2, 0.3], np.float32)
    coeffs = g.normal(size=(3, dim, n) if layout_3kn else (n, dim, 3)).astype(np.float32)
    keep = g.random(n) < 0.3
    words = np.packbits(np.pad(keep, (0, 32 * ((n + 31) // 32) - n)), bitorder="little").view(np.uint32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    tp, to, tc, tm = T(pos), T(origin), T(coeffs), T(words.view(np.int32))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    outs = []
    for fn, extra in ((lib.xsg_sh_fwd, ()), (lib.xsg_sh_fwd_ex, (0,)), (lib.xsg_sh_fwd_ex, (1,))):
        out = torch.full((n, 3), 7.0, device=dev)
        assert fn(degree, P(to), ctypes.c_int64(n), dim, P(tp), P(tc), None, P(tm), int(layout_3kn), *extra,
                  P(out), stream) == 0
        outs.append(np_(out))
    ref = O.sh_fwd(degree, origin, pos, coeffs, mask=words, layout_3kn=layout_3kn)
    assert np.array_equal(outs[0], outs[1])
    assert (outs[0][~keep] == 7.0).all() and (outs[2][~keep] == 0.0).all()
    assert np.array_equal(outs[2][keep], outs[0][keep])
    assert frac_close(outs[2][keep], ref[keep], RENDER_ATOL) == 1.0

def test_release_thread_resources(dev, cfg0):
    """xsg_isect_count's per-thread readback buffer and event: released through the C-ABI on the thread
    that used them (the test's own and a worker thread), re-created by the next count, which bins as
    before; a second release with nothing held is a no-op."""
    import ctypes
    import threading
    from xsimgs_amd import _build
    lib = ctypes.CDLL(_build.lib_path())
    sc, st = cfg0
    spec = sc.cameras[0]
    _, (flags, radii, m2, dep) = _ut(st, spec, dev)

    def bin_once():
        tpg, ids, fl = _C.isect_regular_tiles(m2, radii, dep, spec.width, spec.height, 16, 16)
        return np_(tpg), np_(ids), np_(fl)
    want = bin_once()
    assert lib.xsg_release_thread_resources() == 0
    assert lib.xsg_release_thread_resources() == 0
    for a, b in zip(bin_once(), want):
        assert np.array_equal(a, b)
    out = {}

    def worker():
        out["bins"] = bin_once()
        out["rc"] = lib.xsg_release_thread_resources()
        out["again"] = bin_once()
        out["rc2"] = lib.xsg_release_thread_resources()
    t = threading.Thread(target=worker)
    t.start()
    t.join()
    assert out["rc"] == 0 and out["rc2"] == 0
    for k in ("bins", "again"):
        for a, b in zip(out[k], want):
            assert np.array_equal(a, b)
    assert lib.xsg_release_thread_resources() == 0


def test_fill_tile_offsets(dev, cfg0):
    """The sorted fill's tile offsets equal isect_offset_encode on its keys: one camera, a batched rig
    of three (camera bits in the keys), and no intersections at all (every offset 0)."""
    sc, st = cfg0
    spec = sc.cameras[0]
    _, (flags, radii, m2, dep) = _ut(st, spec, dev)
    ntx, nty = (spec.width + 15) // 16, (spec.height + 15) // 16
    off = torch.full((nty, ntx), -7, dtype=torch.int32, device=dev)
    _, ids, _ = _C.isect_regular_tiles(m2, radii, dep, spec.width, spec.height, 16, 16, tile_offsets=off)
    assert np.array_equal(np_(off), np_(_C.isect_offset_encode(ids, ntx, nty)))
    # three cameras: the second sees nothing, the third a shifted copy
    m2b = torch.stack([m2, m2 + 1e6, m2 + 3.5]).contiguous()
    rb = torch.stack([radii, radii, radii]).contiguous()
    db = torch.stack([dep, dep, dep * 1.5]).contiguous()
    offb = torch.full((3, nty, ntx), -7, dtype=torch.int32, device=dev)
    _, idsb, _ = _C.isect_regular_tiles_batched(m2b, rb, db, spec.width, spec.height, 16, 16, tile_offsets=offb)
    assert np.array_equal(np_(offb), np_(_C.isect_offset_encode(idsb, ntx, nty, 3)))
    off0 = torch.full((nty, ntx), -7, dtype=torch.int32, device=dev)
    _, ids0, _ = _C.isect_regular_tiles(m2 + 1e6, radii, dep, spec.width, spec.height, 16, 16, tile_offsets=off0)
    assert ids0.numel() == 0 and int(off0.abs().max()) == 0
    with pytest.raises(RuntimeError, match="tile offsets"):
        _C.isect_regular_tiles(m2, radii, dep, spec.width, spec.height, 16, 16,
                               tile_offsets=torch.empty(ntx * nty + 1, dtype=torch.int32, device=dev))
    with pytest.raises(RuntimeError, match="sorted fill"):
        _C.isect_regular_tiles(m2, radii, dep, spec.width, spec.height, 16, 16, sort=False, tile_offsets=off)


def test_isect_regular_many_visible(dev):
    """More visible instances than the depth pre-order's capped grid covers in one tile each
    (256 workgroups x 1024 keys), so its workgroups loop over several tiles; bit-exact against the
    oracle, with tile offsets."""
    g = np.random.default_rng(21)
    n, W, H = 700_000, 1920, 1080
    m2 = np.stack([g.uniform(0, W, n), g.uniform(0, H, n)], 1).astype(np.float32)
    r = g.uniform(0.5, 20.0, (n, 2)).astype(np.float32)
    d = g.uniform(0.3, 90.0, n).astype(np.float32)
    d[: n // 50] = d[n // 2]  # ties in depth
    T = lambda a: torch.from_numpy(a).to(dev)
    off = torch.empty(((H + 15) // 16, (W + 15) // 16), dtype=torch.int32, device=dev)
    tpg, ids, fl = _C.isect_regular_tiles(T(m2), T(r), T(d), W, H, 16, 16, tile_offsets=off)
    print("visible", int((tpg > 0).sum()), "isects", ids.numel(), flush=True)
    assert int((tpg > 0).sum()) > 2 * 256 * 1024
    rtpg, rids, rfl = O.isect_regular(m2, r, d, W, H, 16, 16)
    assert np.array_equal(np_(tpg), rtpg)
    assert np.array_equal(np_(ids), rids)
    assert np.array_equal(np_(fl), rfl)
    assert np.array_equal(np_(off), O.offset_encode(rids, (W + 15) // 16, (H + 15) // 16))


def test_isect_presort_tile_sizes(dev):
    """The depth pre-order takes one of two schemes by the call's number of virtual instances: from 3 M
    on, four LSD passes in tiles of 2048 keys; below, a most-significant-digit pass over the keys'
    offsets from the smallest visible key and an LDS sort of each bucket. Both must order the keys as
    the oracle does. A 3.2 M-Gaussian scene (LSD) and its first half (buckets), with ties in depth; a
    call's result does not depend on an earlier call's size (the small scene binned between two
    identical calls)."""
    g = np.random.default_rng(23)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    W, H = 1920, 1080
    n = 3_200_000
    m2 = np.stack([g.uniform(0, W, n), g.uniform(0, H, n)], 1).astype(np.float32)
    r = g.uniform(0.5, 6.0, (n, 2)).astype(np.float32)
    d = g.uniform(0.3, 90.0, n).astype(np.float32)
    d[: n // 50] = d[n // 2]  # ties in depth
    for k in (n, n // 2):
        a = _C.isect_regular_tiles(T(m2[:k]), T(r[:k]), T(d[:k]), W, H, 16, 16)
        _C.isect_regular_tiles(T(m2[:2000]), T(r[:2000]), T(d[:2000]), W, H, 16, 16)
        b = _C.isect_regular_tiles(T(m2[:k]), T(r[:k]), T(d[:k]), W, H, 16, 16)
        print("instances", k, "visible", int((a[0] > 0).sum()), "isects", a[1].numel(), flush=True)
        rtpg, rids, rfl = O.isect_regular(m2[:k], r[:k], d[:k], W, H, 16, 16)
        for got in (a, b):
            assert np.array_equal(np_(got[0]), rtpg)
            assert np.array_equal(np_(got[1]), rids)
            assert np.array_equal(np_(got[2]), rfl)


@pytest.mark.parametrize("C_,n", [(6, 60_000), (16, 20_000)])
def test_isect_regular_batched_cameras(dev, C_, n):
    """Cameras binned in one call (camera bits above the tile bits) equal each camera's oracle binning
    in turn, with the camera id in the keys and ids offset by cam * N, and with the tile offsets of
    the keys. Six cameras: 6 x 68 tile rows plus the negative-depth bucket are 409 row buckets, sorted
    in one 9-bit pass whose digit totals give the row starts inside the segment counter
    (seg_count_rows_kernel, up to 1024 buckets). Sixteen: 1089 row buckets, two 8-bit passes, row
    starts from the sorted runs' boundaries (row_start_kernel) and each segment's row by a search of the
    rows' segment bases in LDS (row_segments_kernel, seg_count_kernel)."""
    g = np.random.default_rng(23 + C_)
    W, H = 1920, 1080
    m2 = np.stack([g.uniform(-40, W + 40, (C_, n)), g.uniform(-40, H + 40, (C_, n))], -1).astype(np.float32)
    r = g.uniform(0.5, 40.0, (C_, n, 2)).astype(np.float32)
    d = g.uniform(0.3, 90.0, (C_, n)).astype(np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    ntx, nty = (W + 15) // 16, (H + 15) // 16
    off = torch.empty((C_, nty, ntx), dtype=torch.int32, device=dev)
    tpg, ids, fl = _C.isect_regular_tiles_batched(T(m2), T(r), T(d), W, H, 16, 16, tile_offsets=off)
    tnb = int(np.floor(np.log2(ntx * nty))) + 1
    want_ids, want_fl, want_tpg = [], [], []
    for c in range(C_):
        rtpg, rids, rfl = O.isect_regular(m2[c], r[c], d[c], W, H, 16, 16)
        want_tpg.append(rtpg)
        want_ids.append(rids + (np.int64(c) << np.int64(tnb + 32)))
        want_fl.append(rfl + np.int32(c * n))
    want_ids, want_fl = np.concatenate(want_ids), np.concatenate(want_fl)
    print("isects", ids.numel(), flush=True)
    assert np.array_equal(np_(tpg), np.stack(want_tpg))
    assert np.array_equal(np_(ids), want_ids)
    assert np.array_equal(np_(fl), want_fl)
    assert np.array_equal(np_(off), O.offset_encode(want_ids, ntx, nty, C_))


def _rig_expected(m2, r, d, W, H, tsx, tsy):
    """Oracle binning of a rig: each camera's sorted keys with the camera id OR-ed in above the tile
    bits (regular_tiling.cu:37-43; a negative depth's sign-extended bits keep the whole upper half at
    ones), merged by a stable sort on the keys as unsigned numbers -- the reference's single stable
    sort of all cameras' keys."""
    C_, n = d.shape
    ntx, nty = (W + tsx - 1) // tsx, (H + tsy - 1) // tsy
    tnb = int(np.floor(np.log2(ntx * nty))) + 1
    tpg, ids, fl = [], [], []
    for c in range(C_):
        rtpg, rids, rfl = O.isect_regular(m2[c], r[c], d[c], W, H, tsx, tsy)
        tpg.append(rtpg)
        ids.append(rids | (np.int64(c) << np.int64(tnb + 32)))
        fl.append(rfl + np.int32(c * n))
    ids, fl = np.concatenate(ids), np.concatenate(fl)
    order = np.argsort(ids.view(np.uint64), kind="stable")
    return np.stack(tpg), ids[order], fl[order]


@pytest.mark.parametrize("C_,n,neg", [(4, 800_000, False), (4, 800_000, True), (3, 1_100_000, False)],
                         ids=["4cam", "4cam-negative-depth", "3cam"])
def test_isect_large_rig(dev, C_, n, neg):
    """Rigs of at least 3 M camera instances, where the depth pre-order takes its four LSD passes: the
    keys, ids and offsets must equal the oracle's stable sort of every camera's keys. Four 1920x1080
    cameras have 4 x 68 + 1 = 273 row buckets, past what is placed directly: the runs are expanded and
    sorted by row bucket (one 9-bit pass); three cameras have 205, and their runs are placed directly
    from the depth order that interleaves the cameras. Ties in depth across and within cameras, and
    in one case a negative depth (its entries after every tile of every camera)."""
    g = np.random.default_rng(31 + C_ + int(neg))
    W, H = 1920, 1080
    m2 = np.stack([g.uniform(-20, W + 20, (C_, n)), g.uniform(-20, H + 20, (C_, n))], -1).astype(np.float32)
    r = g.uniform(0.5, 12.0, (C_, n, 2)).astype(np.float32)
    d = g.uniform(0.3, 90.0, (C_, n)).astype(np.float32)
    d[:, : n // 40] = d[0, n // 2]  # ties in depth, within and across cameras
    if neg:
        d[1, 7] = -2.5
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    ntx, nty = (W + 15) // 16, (H + 15) // 16
    off = torch.empty((C_, nty, ntx), dtype=torch.int32, device=dev)
    tpg, ids, fl = _C.isect_regular_tiles_batched(T(m2), T(r), T(d), W, H, 16, 16, tile_offsets=off)
    w_tpg, w_ids, w_fl = _rig_expected(m2, r, d, W, H, 16, 16)
    print("isects", ids.numel(), flush=True)
    assert np.array_equal(np_(tpg), w_tpg)
    assert np.array_equal(np_(ids), w_ids)
    assert np.array_equal(np_(fl), w_fl)
    assert np.array_equal(np_(off), O.offset_encode(w_ids[w_ids >= 0], ntx, nty, C_))


@pytest.mark.parametrize("n_cams", [1, 3])
def test_isect_negative_depth(dev, n_cams):
    """Instances with a negative depth (-0.0 included) and a footprint -- the projection never yields
    them, a direct caller can -- are binned bit-exactly: their sign-extended depth bits fill the key's
    tile bits, so their entries sort after every tile of every camera. Tile ranges cover the other keys
    only: the offsets (from the fill and from isect_offset_encode) equal the reference encoder's on the
    non-negative keys. On the full key list the reference's encoder maps those keys to tile
    2^tile_bits - 1 - n_tiles, and its last thread writes n_isects over every later tile while other
    threads write their starts (tiling_common.cu:41-60): a race, so nothing to compare against there."""
    g = np.random.default_rng(31 + n_cams)
    n, W, H = 5000, 773, 1117
    m2 = np.stack([g.uniform(-30, W + 30, (n_cams, n)), g.uniform(-30, H + 30, (n_cams, n))], -1).astype(np.float32)
    r = g.uniform(0.0, 30.0, (n_cams, n, 2)).astype(np.float32)
    d = g.uniform(-5.0, 90.0, (n_cams, n)).astype(np.float32)
    d[:, :10] = -0.0
    d[:, 10:60] = d[:, 70:71]  # ties
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    ntx, nty = (W + 15) // 16, (H + 15) // 16
    shape = (nty, ntx) if n_cams == 1 else (n_cams, nty, ntx)
    off = torch.full(shape, -7, dtype=torch.int32, device=dev)
    if n_cams == 1:
        tpg, ids, fl = _C.isect_regular_tiles(T(m2[0]), T(r[0]), T(d[0]), W, H, 16, 16, tile_offsets=off)
        tpg = tpg.view(1, -1)
    else:
        tpg, ids, fl = _C.isect_regular_tiles_batched(T(m2), T(r), T(d), W, H, 16, 16, tile_offsets=off)
    wtpg, wids, wfl = _rig_expected(m2, r, d, W, H, 16, 16)
    print("isects", ids.numel(), "negative-depth entries", int((wids < 0).sum()), flush=True)
    assert int((wids < 0).sum()) > 100
    assert np.array_equal(np_(tpg), wtpg)
    assert np.array_equal(np_(ids), wids)
    assert np.array_equal(np_(fl), wfl)
    want_off = O.offset_encode(wids[wids >= 0], ntx, nty, n_cams)
    assert np.array_equal(np_(off), want_off)
    enc = _C.isect_offset_encode(ids, ntx, nty) if n_cams == 1 else _C.isect_offset_encode(ids, ntx, nty, n_cams)
    assert np.array_equal(np_(enc), want_off)


@pytest.mark.parametrize("n_cams", [1, 2])
@pytest.mark.parametrize("tile", [(8, 8), (16, 8), (12, 10), (32, 32), (10, 6)])
def test_isect_regular_tile_shapes(dev, tile, n_cams):
    """Tiles other than 16x16, on an image that no tile shape divides: keys, ids, counts and offsets
    bit-exact against the oracle, one camera (sorted and unsorted) and a rig of two."""
    tsx, tsy = tile
    g = np.random.default_rng(tsx * 100 + tsy + n_cams)
    n, W, H = 20_000, 1861, 930
    m2 = np.stack([g.uniform(-50, W + 50, (n_cams, n)), g.uniform(-50, H + 50, (n_cams, n))], -1).astype(np.float32)
    r = g.uniform(0.0, 24.0, (n_cams, n, 2)).astype(np.float32)
    d = g.uniform(0.1, 90.0, (n_cams, n)).astype(np.float32)
    d[:, : n // 10] = d[:, n // 2 : n // 2 + 1]  # ties
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    ntx, nty = (W + tsx - 1) // tsx, (H + tsy - 1) // tsy
    shape = (nty, ntx) if n_cams == 1 else (n_cams, nty, ntx)
    off = torch.full(shape, -7, dtype=torch.int32, device=dev)
    if n_cams == 1:
        tpg, ids, fl = _C.isect_regular_tiles(T(m2[0]), T(r[0]), T(d[0]), W, H, tsx, tsy, tile_offsets=off)
        tpg = tpg.view(1, -1)
        _, ids_u, fl_u = _C.isect_regular_tiles(T(m2[0]), T(r[0]), T(d[0]), W, H, tsx, tsy, sort=False)
        _, rids_u, rfl_u = O.isect_regular(m2[0], r[0], d[0], W, H, tsx, tsy, sort=False)
        assert np.array_equal(np_(ids_u), rids_u)
        assert np.array_equal(np_(fl_u), rfl_u)
    else:
        tpg, ids, fl = _C.isect_regular_tiles_batched(T(m2), T(r), T(d), W, H, tsx, tsy, tile_offsets=off)
    wtpg, wids, wfl = _rig_expected(m2, r, d, W, H, tsx, tsy)
    print("tile", tile, "cameras", n_cams, "isects", ids.numel(), flush=True)
    assert np.array_equal(np_(tpg), wtpg)
    assert np.array_equal(np_(ids), wids)
    assert np.array_equal(np_(fl), wfl)
    assert np.array_equal(np_(off), O.offset_encode(wids, ntx, nty, n_cams))


def test_isect_regular_edge_cases(dev):
    # empty input, all-culled input, Gaussians on tile borders and outside the image, negative depth
    W, H = 100, 70
    m2 = torch.tensor([[0.0, 0.0], [16.0, 16.0], [99.9, 69.9], [-30.0, 10.0], [50.0, 35.0], [50.0, 35.0],
                       [200.0, 200.0], [8.0, 8.0]])
    r = torch.tensor([[1.0, 1.0], [16.0, 0.5], [3.0, 3.0], [31.0, 2.0], [0.0, 5.0], [7.5, 7.5],
                      [500.0, 500.0], [2.0, 2.0]])
    d = torch.tensor([1.0, 2.0, 2.0, 3.0, 4.0, 2.0, 9.0, -1.5])
    # the last Gaussian has a negative depth: its sign-extended key (tiling_common.cuh:37) saturates
    # the tile bits, which the sort must reproduce; tile ranges are only defined without it
    for n in (0, m2.shape[0] - 1, m2.shape[0]):
        tpg, ids, fl = _C.isect_regular_tiles(m2[:n].to(dev).contiguous(), r[:n].to(dev).contiguous(),
                                              d[:n].to(dev).contiguous(), W, H, 16, 16)
        rtpg, rids, rfl = O.isect_regular(m2[:n], r[:n], d[:n], W, H, 16, 16)
        assert np.array_equal(np_(tpg), rtpg) and np.array_equal(np_(ids), rids) and np.array_equal(np_(fl), rfl)
        if n < m2.shape[0]:
            off = _C.isect_offset_encode(ids, 7, 5)
            assert np.array_equal(np_(off), O.offset_encode(rids, 7, 5))


def test_radix_sort_pairs(dev):
    g = np.random.default_rng(3)
    for n, bits in ((1, 45), (1000, 45), (300_001, 45), (70_000, 13), (12345, 64)):
        keys = g.integers(0, 2**62, n, dtype=np.int64) & ((1 << min(bits, 63)) - 1)
        keys[: n // 3] = keys[n // 2] if n > 3 else keys[0]       # heavy ties
        vals = np.arange(n, dtype=np.int32)
        k, v = _C.radix_sort_pairs(torch.from_numpy(keys).to(dev), torch.from_numpy(vals).to(dev), 0, bits)
        rk, rv = O.sort_pairs(keys, vals, bits)
        mask = np.uint64((1 << bits) - 1) if bits < 64 else np.uint64(0xFFFFFFFFFFFFFFFF)
        order = np.argsort(keys.view(np.uint64) & mask, kind="stable")
        assert np.array_equal(np_(k), rk) and np.array_equal(np_(v), rv)
        assert np.array_equal(rv, vals[order])


# ------------------------------------------------------------------ compositing
def _binned(st, sc, dev):
    spec = sc.cameras[0]
    cam, (flags, radii, m2, dep) = _ut(st, spec, dev, sc.use_phm)
    tsx, tsy = sc.tile_size
    tpg, ids, fl = cam.isect_gs_tiles(st.means, torch.exp(st.log_scales), st.quats, spec.width, spec.height,
                                      flags, radii, m2, dep, opacity=torch.sigmoid(st.opacity_logits),
                                      tile_size_x=tsx, tile_size_y=tsy)
    off = _C.isect_offset_encode(ids, (spec.width + tsx - 1) // tsx, (spec.height + tsy - 1) // tsy)
    ro, rd = cam.camera_rays(spec.width, spec.height)
    return cam, off, fl, ro, rd


def test_eval3d_fwd_bwd_cfg0(dev, cfg0):
    sc, st = cfg0
    spec = sc.cameras[0]
    cam, off, fl, ro, rd = _binned(st, sc, dev)
    scales = torch.exp(st.log_scales)
    opac = torch.sigmoid(st.opacity_logits)
    colors = _C.spherical_harmonics_fused_fwd(0, cam.pose.t, st.means, st.sh, None, False)
    rgb, depth, alpha, last = _C.rasterize_eval3d_fwd(st.means, st.quats, scales, colors.unsqueeze(0),
                                                      opac.view(1, -1), spec.width, spec.height, 16, 16, ro, rd,
                                                      off, fl)
    hoff, hfl = np_(off), np_(fl)
    inp = dict(means=np_(st.means), quats=np_(st.quats), scales=np_(scales), opac=np_(opac), colors=np_(colors),
               ro=np_(ro), rd=np_(rd))
    ref = O.eval3d_fwd(inp["means"], inp["quats"], inp["scales"], inp["colors"], inp["opac"], inp["ro"], inp["rd"],
                       hoff, hfl, 16, 16)
    got = [np_(rgb), np_(depth), np_(alpha), np_(last)]
    # every pixel outside 1e-4 of the f32 oracle, or with another last id, undetermined in float32 or
    # right against f64
    J.judge_renders(got, ref, inp, hoff, hfl, 16, 16, label="cfg0")
    g = torch.Generator().manual_seed(11)
    vr = (torch.randn(spec.height, spec.width, 3, generator=g) * 1e-3).to(dev)
    vd = (torch.randn(spec.height, spec.width, generator=g) * 1e-3).to(dev)
    va = (torch.randn(spec.height, spec.width, generator=g) * 1e-3).to(dev)
    grads = _C.rasterize_eval3d_bwd(st.means, scales, st.quats, opac, colors, ro, rd, 16, 16, off, fl, alpha, last,
                                    vr, vd, va)
    refs = J.bwd_runs(inp, hoff, hfl, got[2], got[3], np_(vr), np_(vd), np_(va), 16, 16, None)
    names = ["v_means", "v_quats", "v_scales", "v_opacity", "v_colors"]
    J.judge_grads(dict(zip(names, grads[:5])), refs, np.unique(hfl), label="cfg0")
    J.judge_pixel_grads(dict(v_ray_o=grads[5], v_ray_d=grads[6]), refs, np.ones(got[2].shape, bool), label="cfg0")


def test_eval3d_bwd_without_ray_grads(dev, cfg0):
    """ray_grads=False (autograd when rays need no gradient) gives the same Gaussian gradients."""
    sc, st = cfg0
    spec = sc.cameras[0]
    cam, off, fl, ro, rd = _binned(st, sc, dev)
    scales = torch.exp(st.log_scales)
    opac = torch.sigmoid(st.opacity_logits)
    colors = _C.spherical_harmonics_fused_fwd(0, cam.pose.t, st.means, st.sh, None, False)
    _, _, alpha, last = _C.rasterize_eval3d_fwd(st.means, st.quats, scales, colors.unsqueeze(0), opac.view(1, -1),
                                                spec.width, spec.height, 16, 16, ro, rd, off, fl)
    g = torch.Generator().manual_seed(12)
    vr = (torch.randn(spec.height, spec.width, 3, generator=g) * 1e-3).to(dev)
    vd = (torch.randn(spec.height, spec.width, generator=g) * 1e-3).to(dev)
    va = (torch.randn(spec.height, spec.width, generator=g) * 1e-3).to(dev)
    a = _C.rasterize_eval3d_bwd(st.means, scales, st.quats, opac, colors, ro, rd, 16, 16, off, fl, alpha, last,
                                vr, vd, va)
    b = _C.rasterize_eval3d_bwd(st.means, scales, st.quats, opac, colors, ro, rd, 16, 16, off, fl, alpha, last,
                                vr, vd, va, False)
    assert b[5] is None and b[6] is None
    for x, y in zip(a[:5], b[:5]):
        assert frac_close(np_(y), np_(x), GRAD_ATOL, GRAD_RTOL) == 1.0


def _tile_work_np(last, off, fl_n, W, H, tsx, tsy):
    """Per tile: its intersections up to the largest last id of its pixels (the backward's launch-order
    estimate), from the forward's last ids and the tile offsets."""
    ntx, nty = (W + tsx - 1) // tsx, (H + tsy - 1) // tsy
    o = off.reshape(-1).astype(np.int64)
    ends = np.append(o[1:], fl_n)
    work = np.zeros(ntx * nty, np.int64)
    for t in range(ntx * nty):
        ty, tx = divmod(t, ntx)
        m = int(last[ty * tsy:(ty + 1) * tsy, tx * tsx:(tx + 1) * tsx].max())
        work[t] = max(0, min(ends[t] - 1, m) - o[t] + 1)
    return work


def test_eval3d_tile_work_from_forward(dev, cfg0):
    """The forward's per-tile work estimates (tile_work=, an extension) equal the formula on its last ids;
    a backward that reads them, or garbage in their place (they only order the tiles), gives the
    gradients of one that derives them itself."""
    sc, st = cfg0
    spec = sc.cameras[0]
    cam, off, fl, ro, rd = _binned(st, sc, dev)
    scales = torch.exp(st.log_scales)
    opac = torch.sigmoid(st.opacity_logits)
    colors = _C.spherical_harmonics_fused_fwd(0, cam.pose.t, st.means, st.sh, None, False)
    work = torch.full((off.numel(),), -7, dtype=torch.int32, device=dev)
    _, _, alpha, last = _C.rasterize_eval3d_fwd(st.means, st.quats, scales, colors.unsqueeze(0), opac.view(1, -1),
                                                spec.width, spec.height, 16, 16, ro, rd, off, fl, tile_work=work)
    want = _tile_work_np(np_(last), np_(off), fl.numel(), spec.width, spec.height, 16, 16)
    assert want.max() > 0
    np.testing.assert_array_equal(np_(work).astype(np.int64), want)
    g = torch.Generator().manual_seed(13)
    vr = (torch.randn(spec.height, spec.width, 3, generator=g) * 1e-3).to(dev)
    vd = (torch.randn(spec.height, spec.width, generator=g) * 1e-3).to(dev)
    va = (torch.randn(spec.height, spec.width, generator=g) * 1e-3).to(dev)
    args = (st.means, scales, st.quats, opac, colors, ro, rd, 16, 16, off, fl, alpha, last, vr, vd, va)
    a = _C.rasterize_eval3d_bwd(*args)
    b = _C.rasterize_eval3d_bwd(*args, tile_work=work)
    junk = torch.from_numpy(np.random.default_rng(3).integers(-2**31, 2**31 - 1, off.numel(),
                                                              dtype=np.int64).astype(np.int32)).to(dev)
    c = _C.rasterize_eval3d_bwd(*args, tile_work=junk)
    for x, y, z in zip(a, b, c):
        assert frac_close(np_(y), np_(x), GRAD_ATOL, GRAD_RTOL) == 1.0
        assert frac_close(np_(z), np_(x), GRAD_ATOL, GRAD_RTOL) == 1.0


# ------------------------------------------------------------------ scenes built for one rule each
def _pinhole_scene(dev, seed, n=300, W=52, H=38, f=40.0):
    """Random Gaussians in front of a small pinhole camera, projected by the GPU's UT."""
    g = np.random.default_rng(seed)
    z = np.exp(g.uniform(np.log(2.0), np.log(20.0), n))
    xy = g.uniform(-0.8, 0.8, (n, 2)) * z[:, None] * np.array([W / 2 / f, H / 2 / f])
    means = np.concatenate([xy, z[:, None]], 1).astype(np.float32)
    scales = np.exp(g.uniform(np.log(0.02), np.log(0.3), (n, 3))).astype(np.float32)
    quats = g.standard_normal((n, 4)).astype(np.float32)
    opac = g.uniform(0.05, 0.95, n).astype(np.float32)
    colors = g.uniform(0.0, 1.0, (n, 3)).astype(np.float32)
    spec = synthetic.pinhole(W, H, f, f, W / 2, H / 2)
    cam = frame.make_camera(spec, dev)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    flags, radii, m2, dep = cam.ext_cls.projection_utgs(cam.pack, T(means), None, T(scales), T(quats), T(opac), W, H)
    ro, rd = cam.camera_rays(W, H)
    return dict(means=means, scales=scales, quats=quats, opac=opac, colors=colors, W=W, H=H, spec=spec,
                radii=radii, m2=m2, dep=dep, ro=np_(ro), rd=np_(rd))


def _render_and_judge(dev, s, off, fl, tsx, tsy, label, g):
    """GPU forward and backward (with ray gradients) against the oracle on the given binning."""
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    W, H = s["W"], s["H"]
    means, quats, scales, opac, colors = (T(s[k]) for k in ("means", "quats", "scales", "opac", "colors"))
    ro, rd = T(s["ro"]), T(s["rd"])
    rgb, depth, alpha, last = _C.rasterize_eval3d_fwd(means, quats, scales, colors.unsqueeze(0), opac.view(1, -1),
                                                      W, H, tsx, tsy, ro, rd, off, fl)
    got = [np_(rgb), np_(depth), np_(alpha), np_(last)]
    inp = dict(means=s["means"], quats=s["quats"], scales=s["scales"], opac=s["opac"], colors=s["colors"],
               ro=s["ro"], rd=s["rd"])
    hoff, hfl = np_(off), np_(fl)
    ref32 = O.eval3d_fwd(s["means"], s["quats"], s["scales"], s["colors"], s["opac"], s["ro"], s["rd"], hoff, hfl,
                         tsx, tsy)
    J.judge_renders(got, ref32, inp, hoff, hfl, tsx, tsy, label=label)
    vr = (g.standard_normal((H, W, 3)) * 1e-3).astype(np.float32)
    vd = (g.standard_normal((H, W)) * 1e-3).astype(np.float32)
    va = (g.standard_normal((H, W)) * 1e-3).astype(np.float32)
    names = ["v_means", "v_quats", "v_scales", "v_opacity", "v_colors"]
    refs = J.bwd_runs(inp, hoff, hfl, got[2], got[3], vr, vd, va, tsx, tsy, None)
    rows = np.unique(hfl)
    for ray_grads in (True, False):
        out = _C.rasterize_eval3d_bwd(means, scales, quats, opac, colors, ro, rd, tsx, tsy, off, fl, alpha, last,
                                      T(vr), T(vd), T(va), ray_grads)
        J.judge_grads(dict(zip(names, out[:5])), refs, rows, label=f"{label} ray_grads={ray_grads}")
    return got


def test_eval3d_negative_depth_last_tile(dev):
    """Entries keyed with a negative depth sort after every tile (tiling_common.cuh:37); the last tile's
    range runs to n_isects (utils.h:52-57), so the last tile composites them after its own entries, in
    the forward and the backward, exactly as the oracle does with the same offsets."""
    s = _pinhole_scene(dev, 41)
    W, H = s["W"], s["H"]
    # Gaussians in front of the last tile's pixels (bottom right), keyed with a negative depth
    g = np.random.default_rng(42)
    k = 30
    px = np.stack([g.uniform(48, 52, k), g.uniform(32, 38, k)], 1)
    z = g.uniform(3.0, 8.0, k)
    corner = np.stack([(px[:, 0] - W / 2) / 40.0 * z, (px[:, 1] - H / 2) / 40.0 * z, z], 1).astype(np.float32)
    s["means"][:k] = corner
    s["opac"][:k] = 0.6
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    cam = frame.make_camera(s["spec"], dev)
    flags, radii, m2, dep = cam.ext_cls.projection_utgs(cam.pack, T(s["means"]), None, T(s["scales"]),
                                                        T(s["quats"]), T(s["opac"]), W, H)
    dep = dep.clone()
    dep[:k] = -dep[:k]
    ntx, nty = (W + 15) // 16, (H + 15) // 16
    off = torch.full((nty, ntx), -7, dtype=torch.int32, device=dev)
    tpg, ids, fl = _C.isect_regular_tiles(m2, radii, dep, W, H, 16, 16, tile_offsets=off)
    hids = np_(ids)
    first_neg = int(np.argmax(hids < 0)) if (hids < 0).any() else hids.size
    n_neg = int((hids < 0).sum())
    print("entries", hids.size, "negative-depth entries", n_neg, "from index", first_neg, flush=True)
    assert n_neg > 20 and np.all(hids[first_neg:] < 0)
    got = _render_and_judge(dev, s, off, fl, 16, 16, "negative-depth", np.random.default_rng(43))
    # the last tile's pixels do composite entries past the last non-negative key
    assert int((got[3] >= first_neg).sum()) > 0


def test_eval3d_bwd_clamp_band(dev):
    """Pairs with op * vis in (0.99, 0.999): forward alpha unclamped, backward at 0.99 with no geometry
    or opacity gradient (eval3d_bwd.cu:38, 202, 243). Gaussians centred on pixel rays with opacities
    in that band make most of their pairs fall there."""
    s = _pinhole_scene(dev, 51)
    W, H = s["W"], s["H"]
    g = np.random.default_rng(52)
    k = 60
    pi, pj = g.integers(0, H, k), g.integers(0, W, k)
    t = g.uniform(3.0, 15.0, k)
    s["means"][:k] = (s["ro"][pi, pj] + t[:, None] * s["rd"][pi, pj]).astype(np.float32)
    s["opac"][:k] = g.uniform(0.9905, 0.9989, k).astype(np.float32)
    s["scales"][:k] = np.exp(g.uniform(np.log(0.03), np.log(0.1), (k, 3))).astype(np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    cam = frame.make_camera(s["spec"], dev)
    flags, radii, m2, dep = cam.ext_cls.projection_utgs(cam.pack, T(s["means"]), None, T(s["scales"]),
                                                        T(s["quats"]), T(s["opac"]), W, H)
    ntx, nty = (W + 15) // 16, (H + 15) // 16
    off = torch.full((nty, ntx), -7, dtype=torch.int32, device=dev)
    _, ids, fl = _C.isect_regular_tiles(m2, radii, dep, W, H, 16, 16, tile_offsets=off)
    got = _render_and_judge(dev, s, off, fl, 16, 16, "clamp-band", np.random.default_rng(53))
    # the band is exercised: on the pixels the Gaussians are centred on, alpha passes 0.99
    in_band = int((got[2][pi, pj] > 0.99).sum())
    print("pixels with alpha above 0.99 at a band Gaussian's centre:", in_band, "of", k, flush=True)
    assert in_band >= k // 3


@pytest.mark.parametrize("timing", ["global", "rolling_pos", "rolling_neg"])
def test_ut_phm_seam_cases(dev, timing):
    """The phase-modelled UT on the seam cases pinned on the CPU (tests/test_oracle_phm.py): far from
    the seams, straddling the image seam, straddling u_pose, a footprint crossing the image edge, and
    the half-turn camera's one-sided case; flags and the stored side's outputs against the oracle."""
    from tests.test_oracle_phm import seam_cases
    for name, spec, mu, q, s, op, flag, side in seam_cases(timing):
        cam = frame.make_camera(spec, dev)
        T = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)
        got = cam.ext_cls.projection_utgs_phm(cam.pack, T(mu[None]), None, T([s]), T([q]), T([op]), spec.width,
                                              spec.height)
        f, r, m2, d = (np_(x) for x in got)
        rf, rr, rm, rd = O.project_utgs(spec, mu[None].astype(np.float32), np.array([s], np.float32),
                                        np.array([q], np.float32), np.array([op], np.float32), spec.width,
                                        spec.height, phm=True)
        print(timing, name, "gpu", int(f[0]), m2[0], r[0], "| oracle", int(rf[0]), rm[0], rr[0], flush=True)
        assert int(f[0]) == int(rf[0]) == flag, name
        assert np.allclose(m2, rm, atol=2e-2) and np.allclose(r, rr, atol=2e-2, rtol=1e-4), name
        assert np.allclose(d, rd, rtol=1e-6), name


@pytest.mark.parametrize("timing", ["global", "rolling_pos", "rolling_neg"])
@pytest.mark.parametrize("kind", ["lidar", "spherical"])
def test_seam_spans_gpu(dev, kind, timing):
    """The seam Gaussians pinned on the CPU (tests/test_oracle_seam.py), projected and binned on the GPU:
    flag 2, both spans' tile sets equal to the float64 restatement's (the second span past the tile
    boundary on the shutter's side, each branch of phm_lidar_tiling.cu:207-217 /
    phm_spherical_tiling.cu:147-157), every key carrying its Gaussian's stored depth bits (a static
    camera's re-projected depth is the stored one), and keys and ids bit-exact against the oracle's
    binning of the same projections."""
    from tests import test_oracle_seam as TS
    spec = TS._spec(kind, timing)
    cases = TS._cases()
    n = len(cases)
    pts = np.array([c[1] for c in cases], np.float32)
    scl = np.array([c[2] for c in cases], np.float32)
    quat = np.tile(np.array(TS.Q, np.float32), (n, 1))
    opac = np.array([c[3] for c in cases], np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    cam = frame.make_camera(spec, dev)
    W, H = TS.W, TS.H
    flags, radii, m2, dep = cam.ext_cls.projection_utgs_phm(cam.pack, T(pts), None, T(scl), T(quat), T(opac), W, H)
    hf, hr, hm2, hd = (np_(x) for x in (flags, radii, m2, dep))
    assert np.all(hf == 2), hf
    elev = TS._elev(spec) if kind == "lidar" else None
    if kind == "lidar":
        tpg, ids, fl = _C.isect_lidar_tiles(cam.pack, T(pts), None, T(scl), T(quat), T(opac), flags, m2, radii, dep,
                                            T(elev), TS.TSX, W, H, sort=False)
    else:
        tpg, ids, fl = _C.isect_spherical_tiles(cam.pack, T(pts), None, T(scl), T(quat), T(opac), flags, m2, radii,
                                                dep, TS.TSX, TS.TSY, W, H, sort=False)
    tpg, ids, fl = np_(tpg), np_(ids), np_(fl)
    (f_lo, f_hi), (s_lo, s_hi) = TS._span_bounds(spec)
    n_az = math.ceil(W / TS.TSX)
    for i in range(n):
        pos = TS._ut_mode(spec, pts[i].astype(np.float64), TS.Q, scl[i].astype(np.float64), float(opac[i]),
                          "positive")
        first = TS._tiles(kind, spec, hm2[i].astype(np.float64), hr[i].astype(np.float64), f_lo, f_hi)
        second = TS._tiles(kind, spec, pos[1], pos[2], s_lo, s_hi)
        mine = ids[fl == i]
        got = sorted((int(k >> 32) // n_az, int(k >> 32) % n_az) for k in mine)
        print(kind, timing, cases[i][0], "tiles", int(tpg[i]), "first", len(first), "second", len(second), flush=True)
        assert tpg[i] == len(first) + len(second) and got == sorted(first + second), (cases[i][0], got)
        assert np.all((mine & 0xFFFFFFFF).astype(np.uint32) == np.float32(hd[i]).view(np.uint32)), cases[i][0]
    unsorted = O.isect_spherical_family(kind, spec, pts, scl, quat, opac, hf, hm2, hr, hd, TS.TSX, TS.TSY, W, H,
                                        elev=elev, sort=False)
    n_tiles = n_az * (len(elev) if kind == "lidar" else math.ceil(H / TS.TSY))
    rtpg, rids, rfl = J.with_input_depths(unsorted, hd, n_tiles)
    sk, sv = O.sort_pairs(ids, fl, 32 + O.tile_n_bits(n_tiles))
    assert np.array_equal(tpg, rtpg) and np.array_equal(sk, rids) and np.array_equal(sv, rfl)


@pytest.mark.parametrize("case", ["regular", "batched", "lidar", "spherical", "cfg3"])
def test_fill_without_keys(dev, cfg0, case):
    """keys=False (the renderer's binning: it takes the tile offsets) writes the same flatten ids and
    offsets as a fill that writes the keys, and returns no keys; the offsets equal isect_offset_encode
    of the written keys."""
    def run(fn, keys):
        off = torch.full(shape, -7, dtype=torch.int32, device=dev)
        tpg, ids, fl = fn(off, keys)
        torch.cuda.synchronize()
        return tpg, ids, fl, off
    if case in ("regular", "batched"):
        sc, st = cfg0
        spec = sc.cameras[0]
        _, (flags, radii, m2, dep) = _ut(st, spec, dev)
        ntx, nty = (spec.width + 15) // 16, (spec.height + 15) // 16
        if case == "regular":
            shape, n_cams = (nty, ntx), 1
            fn = lambda off, keys: _C.isect_regular_tiles(m2, radii, dep, spec.width, spec.height, 16, 16,
                                                          tile_offsets=off, keys=keys)
        else:
            shape, n_cams = (2, nty, ntx), 2
            m2b, rb, db = (torch.stack([x, x]).contiguous() for x in (m2, radii, dep))
            m2b[1] += 9.5
            fn = lambda off, keys: _C.isect_regular_tiles_batched(m2b, rb, db, spec.width, spec.height, 16, 16,
                                                                  tile_offsets=off, keys=keys)
    else:
        if case == "cfg3":
            sc = synthetic.make_cfg3(n=200_000)
            st = frame.prepare(sc, dev, requires_grad=False)
            spec = sc.cameras[0]
            cam, (flags, radii, m2, dep) = _ut(st, spec, dev, True)
            means, scales, quats, opac = st.means, torch.exp(st.log_scales), st.quats, torch.sigmoid(st.opacity_logits)
            tsx, tsy = sc.tile_size
        else:
            z = np.load(os.path.join(os.path.dirname(__file__), "golden", f"{'lidar_phm' if case == 'lidar' else case}.npz"))
            f = {k: z[k] for k in z.files}
            w, h = (int(x) for x in f["cam_size"])
            spec = synthetic.CameraSpec(case, w, h, f["cam_q"].tolist(), f["cam_t"].tolist(), f["cam_impl"].tolist(),
                                        rolling=f["cam_rolling"].tolist(), trigger_time=float(f["cam_times"][0]),
                                        pose_time=float(f["cam_times"][1]),
                                        beam_v=torch.from_numpy(f["cam_beam_v"]) if "cam_beam_v" in f else None)
            cam = frame.make_camera(spec, dev)
            T = lambda k: torch.from_numpy(np.ascontiguousarray(f[k], np.float32)).to(dev)
            means, scales, quats, opac = T("means"), T("scales"), T("quats"), T("opacity")
            flags, radii, m2, dep = cam.ext_cls.projection_utgs_phm(cam.pack, means, None, scales, quats, opac,
                                                                    spec.width, spec.height)
            tsx, tsy = (int(x) for x in f["tile"])
        ntx, nty = (spec.width + tsx - 1) // tsx, (spec.height + tsy - 1) // tsy
        shape, n_cams = (nty, ntx), 1
        fn = lambda off, keys: cam.isect_gs_tiles(means, scales, quats, spec.width, spec.height, flags, radii, m2, dep,
                                                  opacity=opac, tile_size_x=tsx, tile_size_y=tsy, tile_offsets=off,
                                                  keys=keys)
    tpg_k, ids_k, fl_k, off_k = run(fn, True)
    tpg_n, ids_n, fl_n, off_n = run(fn, False)
    print(case, "intersections", fl_k.numel(), flush=True)
    assert fl_k.numel() > 500
    assert ids_n.numel() == 0 and ids_n.dtype == torch.int64
    assert torch.equal(tpg_k, tpg_n) and torch.equal(fl_k, fl_n) and torch.equal(off_k, off_n)
    enc = _C.isect_offset_encode(ids_k, shape[-1], shape[-2], n_cams)
    assert np.array_equal(np_(enc).reshape(-1), np_(off_k).reshape(-1))
    if case == "regular":  # nothing visible: no keys, no ids, every offset 0
        off0 = torch.full(shape, -7, dtype=torch.int32, device=dev)
        tpg0, ids0, fl0 = _C.isect_regular_tiles(m2 + 1e6, radii, dep, spec.width, spec.height, 16, 16,
                                                 tile_offsets=off0, keys=False)
        assert ids0.numel() == 0 and fl0.numel() == 0 and int(tpg0.abs().max()) == 0
        assert int(off0.abs().max()) == 0
    with pytest.raises(RuntimeError, match="keys=False needs tile_offsets"):
        _C.isect_regular_tiles(m2.reshape(-1, 2)[:100].contiguous(), radii.reshape(-1, 2)[:100].contiguous(),
                               dep.reshape(-1)[:100].contiguous(), 64, 64, 16, 16, keys=False)


@pytest.mark.parametrize("case", ["moving_lidar", "moving_spherical", "point_velocity", "static_large"])
def test_ut_phm_pose_kinds(dev, case):
    """The phase-modelled UT has one kernel for static poses and one for moving poses or moving points
    (ut_phm_kernels.h:13-114 for both); the launch runs both and the device's camera picks which one
    writes. Moving lidar / spherical poses (linear and angular velocity, rolling shutter), per-point
    velocities under a static pose, and a static cfg3 scene of 300k Gaussians (more than the moving
    kernel's grid covers in one pass) against the oracle (tests/_judge.py)."""
    if case == "static_large":
        sc = synthetic.make_cfg3(n=300_000)
        spec = sc.cameras[0]
        means, scales, quats, opac = (sc.means.numpy(), sc.scales.numpy(), sc.quats.numpy(),
                                      sc.opacity.numpy())
        vel = None
    else:
        z = np.load(os.path.join(os.path.dirname(__file__), "golden",
                                 "spherical.npz" if case == "moving_spherical" else "lidar_phm.npz"))
        f = {k: z[k] for k in z.files}
        w, h = (int(x) for x in f["cam_size"])
        kind = "spherical" if case == "moving_spherical" else "lidar"
        moving = case != "point_velocity"
        spec = synthetic.CameraSpec(kind, w, h, [0.9950042, 0.0, 0.0, 0.0998334], [0.4, -0.3, 0.2],
                                    f["cam_impl"].tolist(),
                                    v=[2.5, -1.0, 0.3] if moving else [0.0, 0.0, 0.0],
                                    w=[0.02, -0.01, 0.6] if moving else [0.0, 0.0, 0.0],
                                    rolling=[0.1, 0.0], trigger_time=0.0, pose_time=0.05,
                                    beam_v=torch.from_numpy(f["cam_beam_v"]) if "cam_beam_v" in f else None)
        means, scales, quats, opac = f["means"], f["scales"], f["quats"], f["opacity"]
        vel = None
        if case == "point_velocity":
            vel = np.random.default_rng(11).normal(0.0, 3.0, means.shape).astype(np.float32)
    cam = frame.make_camera(spec, dev)
    T = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)
    got = cam.ext_cls.projection_utgs_phm(cam.pack, T(means), T(vel), T(scales), T(quats), T(opac), spec.width,
                                          spec.height)
    out = J.judge_ut(got, spec, means, scales, quats, opac, spec.width, spec.height, phm=True, vel=vel, label=case)
    assert out["visible_gpu"] > out["n"] // 4


def test_eval3d_tile_over_1024_pixels_rejected(dev):
    """Tiles above the 1024-thread workgroup limit fail as the reference's launch setup does
    (tile_shared_memory.h:8-26)."""
    s = _pinhole_scene(dev, 61, n=20)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    W, H = s["W"], s["H"]
    off = torch.zeros((2, 2), dtype=torch.int32, device=dev)
    fl = torch.zeros(0, dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="Failed to set maximum shared memory size"):
        _C.rasterize_eval3d_fwd(T(s["means"]), T(s["quats"]), T(s["scales"]), T(s["colors"]).unsqueeze(0),
                                T(s["opac"]).view(1, -1), W, H, 33, 32, T(s["ro"]), T(s["rd"]), off, fl)
