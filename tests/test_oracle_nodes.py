"""Oracle pins for the scene-assembly producers that feed the rasterization path.

packed_mask_from_instances against numpy's packbits (little bit order: bit i % 32 of word i / 32);
the rigid copy's forward against scipy's rotations (rotation of the positions, composition of the
orientations, rigid-body velocity v + w x (R p)); its backward against float64 central differences of
the forward.
"""
import numpy as np
import pytest
from scipy.spatial.transform import Rotation

from oracle import oracle as O


def _packbits32(bits):
    n = bits.size
    padded = np.zeros(((n + 31) // 32) * 32, np.uint8)
    padded[:n] = bits
    return np.packbits(padded, bitorder="little").view("<u4")


@pytest.mark.parametrize("n", [0, 1, 31, 32, 33, 1000, 4097])
def test_packed_mask_is_packbits(n):
    g = np.random.default_rng(n)
    k = 7
    ids = g.integers(-3, k + 2, n).astype(np.int32)          # negatives: no instance; >= k: out of range
    mask = g.integers(0, 3, k).astype(np.uint8)                # any non-zero byte enables
    bits = np.where((ids < 0) | (ids >= k), 1, mask[np.clip(ids, 0, k - 1)] != 0).astype(np.uint8)
    np.testing.assert_array_equal(O.packed_mask_from_instances(ids, mask), _packbits32(bits))


def _scene(g, n=60, k=5, unit=True):
    pos = g.standard_normal((n, 3))
    rot = g.standard_normal((n, 4))
    iq = g.standard_normal((k, 4))
    if unit:
        iq /= np.linalg.norm(iq, axis=1, keepdims=True)
    it, iv, iw = g.standard_normal((k, 3)), g.standard_normal((k, 3)), g.standard_normal((k, 3))
    ids = g.integers(0, k, n).astype(np.int32)
    im = np.ones(k, np.uint8)
    im[1] = 0
    return pos, rot, ids, iq, it, iv, iw, im


def _offsets(ids, k, g):
    counts = np.bincount(ids, minlength=k)
    per_inst = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int32)
    gs_off = np.zeros(ids.size, np.int32)
    for j in range(k):
        sel = np.nonzero(ids == j)[0]
        gs_off[sel] = g.permutation(sel.size)
    return per_inst, gs_off


@pytest.mark.parametrize("with_offsets", [False, True])
def test_rigid_fwd_against_scipy(with_offsets):
    g = np.random.default_rng(1)
    pos, rot, ids, iq, it, iv, iw, im = _scene(g)
    n, k = pos.shape[0], iq.shape[0]
    off = 5
    po, go = _offsets(ids, k, g) if with_offsets else (None, None)
    b = n + off + 3
    out_p, out_r, out_v = np.full((b, 3), 7.0), np.full((b, 4), 7.0), np.full((b, 3), 7.0)
    out_m = np.zeros(b, np.uint8)
    op, orot, ov, om = O.rigid_fwd(pos, rot, ids, iq, it, iv, iw, im, out_p, out_r, out_v, out_m, off, po, go,
                                   prec="f64")
    rows = off + (po[ids] + go if with_offsets else np.arange(n))
    on = im[ids] != 0
    R = Rotation.from_quat(iq[ids[on]], scalar_first=True)
    pr = R.apply(pos[on])
    np.testing.assert_allclose(op[rows[on]], pr + it[ids[on]], atol=1e-12)
    np.testing.assert_allclose(ov[rows[on]], iv[ids[on]] + np.cross(iw[ids[on]], pr), atol=1e-12)
    # orientation: the Hamilton product q_k (x) q, i.e. the composition R_k R (rot is not unit: compare
    # after normalising, sign included)
    want = (R * Rotation.from_quat(rot[on], scalar_first=True)).as_quat(scalar_first=True, canonical=False)
    got = orot[rows[on]] / np.linalg.norm(rot[on], axis=1, keepdims=True)
    np.testing.assert_allclose(got, want, atol=1e-12)
    assert om[rows[on]].all()
    untouched = np.setdiff1d(np.arange(b), rows[on])
    assert np.all(op[untouched] == 7.0) and np.all(orot[untouched] == 7.0) and not om[untouched].any()


def _loss(args, vp, vr, vv, off, po, go, b):
    pos, rot, ids, iq, it, iv, iw, im = args
    z3, z4 = np.zeros((b, 3)), np.zeros((b, 4))
    op, orot, ov, _ = O.rigid_fwd(pos, rot, ids, iq, it, iv, iw, im, z3, z4, z3, None, off, po, go, prec="f64")
    return float((op * vp).sum() + (orot * vr).sum() + (ov * vv).sum())


@pytest.mark.parametrize("with_offsets,with_vel", [(False, True), (True, True), (True, False)])
def test_rigid_bwd_matches_finite_differences(with_offsets, with_vel):
    g = np.random.default_rng(2)
    args = list(_scene(g, n=40, k=4, unit=False))
    pos, rot, ids, iq, it, iv, iw, im = args
    n, k = pos.shape[0], iq.shape[0]
    off = 3
    po, go = _offsets(ids, k, g) if with_offsets else (None, None)
    b = n + off
    vp, vr = g.standard_normal((b, 3)), g.standard_normal((b, 4))
    vv = g.standard_normal((b, 3)) if with_vel else np.zeros((b, 3))
    got = O.rigid_bwd(pos, rot, ids, iq, iw, im, off, po, go, vp, vr, vv if with_vel else None, prec="f64")
    eps = 1e-6
    for slot, grad in zip((0, 1, 3, 4, 5, 6), got):
        x = args[slot]
        fd = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            keep = x[idx]
            x[idx] = keep + eps
            lp = _loss(args, vp, vr, vv, off, po, go, b)
            x[idx] = keep - eps
            lm = _loss(args, vp, vr, vv, off, po, go, b)
            x[idx] = keep
            fd[idx] = (lp - lm) / (2 * eps)
        np.testing.assert_allclose(grad, fd, rtol=1e-6, atol=1e-6)
    # disabled instance: no gradient, and its particles get zeros
    assert np.all(got[2][1] == 0) and np.all(got[0][ids == 1] == 0)
