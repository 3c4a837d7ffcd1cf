"""GPU parity of the scene-assembly producers against the CPU oracle: the packed instance mask
(bit-exact), the rigid per-instance copy (float32 forward within 1e-6, gradients within 1e-3 relative
with a 1e-5 absolute floor scaled by the largest value, since the per-instance sums add thousands of
terms in float32 atomics), the autograd function and its torch twin."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests._util import GRAD_ATOL, GRAD_RTOL, np_, report
from xsimgs_amd import _C
from xsimgs_amd.nodes import rigid_transform_and_put, rigid_transform_and_put_torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [0, 1, 31, 32, 33, 63, 64, 65, 1000, 1_000_007])
def test_packed_mask_bitexact(dev, n):
    g = np.random.default_rng(n)
    k = 37
    ids = g.integers(-3, k + 3, n).astype(np.int32)
    mask = g.integers(0, 3, k).astype(np.uint8).astype(bool)
    out = _C.packed_mask_from_instances(torch.from_numpy(ids).to(dev), torch.from_numpy(mask).to(dev))
    ref = O.packed_mask_from_instances(ids, mask)
    assert out.dtype == torch.uint32 and out.shape == ((n + 31) // 32,)
    np.testing.assert_array_equal(out.cpu().view(torch.int32).numpy().view(np.uint32), ref)


def test_packed_mask_feeds_mask_radii(dev):
    n, k = 5000, 9
    g = np.random.default_rng(3)
    ids = g.integers(-1, k, n).astype(np.int32)
    mask = np.zeros(k, bool)
    mask[::2] = True
    packed = _C.packed_mask_from_instances(torch.from_numpy(ids).to(dev), torch.from_numpy(mask).to(dev))
    radii = torch.ones(n, 2, device=dev)
    _C.mask_radii_packed(packed, radii)
    keep = (ids < 0) | mask[np.clip(ids, 0, k - 1)]
    np.testing.assert_array_equal(np_(radii)[:, 0] != 0, keep)


def _scene(g, n, k, sorted_ids):
    pos = g.standard_normal((n, 3)).astype(np.float32)
    rot = g.standard_normal((n, 4)).astype(np.float32)
    iq = g.standard_normal((k, 4))
    iq = (iq / np.linalg.norm(iq, axis=1, keepdims=True)).astype(np.float32)
    it, iv, iw = (g.standard_normal((k, 3)).astype(np.float32) for _ in range(3))
    ids = np.sort(g.integers(0, k, n)) if sorted_ids else g.integers(0, k, n)
    ids = ids.astype(np.int32)
    im = np.ones(k, bool)
    im[k // 3] = False
    return pos, rot, ids, iq, it, iv, iw, im


def _offsets(ids, k, g):
    counts = np.bincount(ids, minlength=k)
    per_inst = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int32)
    gs_off = np.zeros(ids.size, np.int32)
    for j in range(k):
        sel = np.nonzero(ids == j)[0]
        gs_off[sel] = g.permutation(sel.size)
    return per_inst, gs_off


def _t(dev, *arrs):
    return [None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in arrs]


@pytest.mark.parametrize("with_offsets", [False, True])
@pytest.mark.parametrize("with_vel_mask", [False, True])
def test_rigid_fwd(dev, with_offsets, with_vel_mask):
    g = np.random.default_rng(5)
    n, k, off = 100_003, 40, 17
    pos, rot, ids, iq, it, iv, iw, im = _scene(g, n, k, False)
    po, go = _offsets(ids, k, g) if with_offsets else (None, None)
    if with_offsets:
        go[:5] = 2 ** 30     # rows past the buffers: skipped, not written
    b = n + off
    init = lambda shape: np.full(shape, 3.0, np.float32)
    out = [init((b, 3)), init((b, 4)), init((b, 3)) if with_vel_mask else None,
           np.zeros(b, bool) if with_vel_mask else None]
    td = _t(dev, pos, rot, ids, iq, it, iv, iw, im, *out, po, go)
    _C.copy_gs_rigid_transform_fwd(*td[:12], off, td[12], td[13])
    ref = O.rigid_fwd(pos, rot, ids, iq, it, iv, iw, im, *out, off, po, go)
    for name, a, r in zip(("positions", "rotations", "velocities", "mask"), td[8:12], ref):
        if r is None:
            continue
        print(report(name, np_(a).astype(np.float64), r.astype(np.float64)), flush=True)
        if name == "mask":
            np.testing.assert_array_equal(np_(a), r)
        else:
            np.testing.assert_allclose(np_(a), r, atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("sorted_ids", [True, False])
@pytest.mark.parametrize("with_offsets,with_vel", [(False, True), (True, True), (True, False)])
def test_rigid_bwd(dev, sorted_ids, with_offsets, with_vel):
    print("case", sorted_ids, with_offsets, with_vel, flush=True)
    g = np.random.default_rng(7)
    n, k, off = 200_000, 50, 9
    pos, rot, ids, iq, it, iv, iw, im = _scene(g, n, k, sorted_ids)
    po, go = _offsets(ids, k, g) if with_offsets else (None, None)
    b = n + off
    vp, vr = g.standard_normal((b, 3)).astype(np.float32), g.standard_normal((b, 4)).astype(np.float32)
    vv = g.standard_normal((b, 3)).astype(np.float32) if with_vel else None
    td = _t(dev, pos, rot, ids, iq, iw, im, po, go, vp, vr, vv)
    got = _C.copy_gs_rigid_transform_bwd(*td[:6], off, *td[6:])
    ref = O.rigid_bwd(pos, rot, ids, iq, iw, im, off, po, go, vp, vr, vv, prec="f64")
    for name, a, r in zip(("g_pos", "g_rot", "g_q", "g_t", "g_v", "g_w"), got, ref):
        a = np_(a).astype(np.float64)
        print(report(name, a, r), flush=True)
        atol = GRAD_ATOL * max(1.0, np.abs(r).max())
        bad = np.abs(a - r) > atol + GRAD_RTOL * np.abs(r)
        assert not bad.any(), (name, np.argwhere(bad)[:5])


def test_rigid_autograd_and_torch_twin(dev):
    g = np.random.default_rng(11)
    n, k = 4099, 6
    pos, rot, ids, iq, it, iv, iw, im = _scene(g, n, k, True)
    po, go = _offsets(ids, k, g)

    def leaves():
        return [t.requires_grad_(True) for t in _t(dev, pos, rot, iq, it, iv, iw)]

    ids_t, im_t, po_t, go_t = _t(dev, ids, im, po, go)
    x = leaves()
    out = rigid_transform_and_put(x[0], x[1], ids_t, x[2], x[3], x[4], x[5], im_t, buffer_offset=0,
                                  per_instance_offsets=po_t, gs_inst_offsets=go_t)
    y = leaves()
    z3, z4 = torch.zeros(n, 3, device=dev), torch.zeros(n, 4, device=dev)
    twin = rigid_transform_and_put_torch(y[0], y[1], ids_t, y[2], y[3], y[4], y[5], im_t, z3, z4,
                                         torch.zeros(n, 3, device=dev), torch.zeros(n, dtype=torch.bool, device=dev),
                                         0, po_t, go_t)
    for a, b in zip(out, twin):
        assert torch.allclose(a, b, atol=1e-6), float((a.float() - b.float()).abs().max())
    w = [torch.randn(o.shape, device=dev, generator=torch.Generator(dev).manual_seed(i)) for i, o in
         enumerate(out[:3])]
    sum((o * wi).sum() for o, wi in zip(out[:3], w)).backward()
    sum((o * wi).sum() for o, wi in zip(twin[:3], w)).backward()
    for name, a, b in zip(("pos", "rot", "q", "t", "v", "w"), x, y):
        print(report(name, np_(a.grad), np_(b.grad)), flush=True)
        scale = max(1.0, float(b.grad.abs().max()))
        assert torch.allclose(a.grad, b.grad, rtol=1e-4, atol=1e-5 * scale), name


def _ulps(a, b):
    """Largest distance in float32 units in the last place between two tensors of finite values."""
    ia = a.detach().float().cpu().contiguous().view(torch.int32).long()
    ib = b.detach().float().cpu().contiguous().view(torch.int32).long()
    ia = torch.where(ia < 0, -(ia & 0x7fffffff), ia)
    ib = torch.where(ib < 0, -(ib & 0x7fffffff), ib)
    return int((ia - ib).abs().max()) if ia.numel() else 0


@pytest.mark.parametrize("n", [0, 1, 63, 1000, 1_000_003])
def test_activate_gaussians_is_torch_exp_and_sigmoid(dev, n):
    """The fused activation op against torch.exp / torch.sigmoid and their autograd on the GPU (the
    same float expressions: the same bits), and against float64 within a float32 rounding; logits and
    log-scales far into the saturated ranges included."""
    from xsimgs_amd.rendering import activate_gaussians
    g = torch.Generator().manual_seed(n)
    ls = torch.randn(n, 3, generator=g) * 3
    lg = torch.randn(n, generator=g) * 6
    if n >= 63:
        ls[:5, 0] = torch.tensor([-100.0, -87.5, 0.0, 60.0, 88.5])
        lg[:6] = torch.tensor([-1e4, -100.0, -17.0, 0.0, 30.0, 1e4])
    ls, lg = ls.to(dev).requires_grad_(), lg.to(dev).requires_grad_()
    vs, vo = torch.randn(n, 3, generator=g).to(dev), torch.randn(n, generator=g).to(dev)
    s, o = activate_gaussians(ls, lg)
    rs, ro = torch.exp(ls), torch.sigmoid(lg)
    gls, glg = torch.autograd.grad((s, o), (ls, lg), (vs, vo))
    rls, rlg = torch.autograd.grad((rs, ro), (ls, lg), (vs, vo))
    d = {k: _ulps(a, b) for k, a, b in (("exp", s, rs), ("sigmoid", o, ro), ("v_log_scales", gls, rls),
                                        ("v_logits", glg, rlg))}
    print(f"activate n={n} ulps against torch: {d}")
    assert all(v == 0 for v in d.values()), d
    s64 = torch.exp(ls.detach().double())
    o64 = torch.sigmoid(lg.detach().double())
    fin = torch.isfinite(s64.float()) & (s64 > 1e-37)
    np.testing.assert_allclose(np_(s)[np_(fin)], np_(s64)[np_(fin)], rtol=2.4e-7)
    np.testing.assert_allclose(np_(o), np_(o64), rtol=3.6e-7, atol=1e-38)


def test_activate_gaussians_one_sided_gradients(dev):
    """A gradient that reaches only the scales (or only the opacities) leaves the other input's None,
    and the one computed equals torch's."""
    from xsimgs_amd.rendering import activate_gaussians
    n = 4097
    g = torch.Generator().manual_seed(5)
    ls = (torch.randn(n, 3, generator=g)).to(dev).requires_grad_()
    lg = (torch.randn(n, 1, generator=g) * 4).to(dev).requires_grad_()
    s, o = activate_gaussians(ls, lg)
    assert s.shape == (n, 3) and o.shape == (n, 1)
    gls, glg = torch.autograd.grad((s * 2).sum(), (ls, lg), allow_unused=True)
    assert glg is None and torch.equal(gls, torch.autograd.grad((torch.exp(ls) * 2).sum(), ls)[0])
    s, o = activate_gaussians(ls, lg)
    gls, glg = torch.autograd.grad((o ** 2).sum(), (ls, lg), allow_unused=True)
    assert gls is None and torch.equal(glg, torch.autograd.grad((torch.sigmoid(lg) ** 2).sum(), lg)[0])


@pytest.mark.parametrize("n_cams,n", [(1, 1), (1, 1000), (1, 100_003), (3, 4097)])
def test_packed_visibility_mask(dev, n_cams, n):
    """The visibility mask of the regular tilings (an extension): bit i set iff some camera's radii of
    Gaussian i are not (r.x <= 0 or r.y <= 0), the test by which the tiling gives an instance no tile;
    zeros, negatives and NaNs included. Packed as numpy packbits (little bit order)."""
    g = np.random.default_rng(n + n_cams)
    r = g.choice(np.array([0.0, -1.0, 0.5, 3.0, np.nan, -0.0], np.float32), size=(n_cams, n, 2))
    radii = torch.from_numpy(r if n_cams > 1 else r[0]).to(dev)
    out = _C.packed_visibility_mask(radii)
    keep = (~((r[..., 0] <= 0) | (r[..., 1] <= 0))).any(axis=0)
    want = np.packbits(np.pad(keep, (0, 32 * ((n + 31) // 32) - n)), bitorder="little").view(np.uint32)
    assert out.dtype == torch.uint32 and out.shape == ((n + 31) // 32,)
    np.testing.assert_array_equal(out.cpu().view(torch.int32).numpy().view(np.uint32), want)
