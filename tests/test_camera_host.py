"""Host-side camera logic (no GPU): pack layouts of the distorted / fisheye models and the
max-radius bound of the distorted model (the fold of the radial map, or a margin past the image
corner, whichever comes first)."""
import math

import torch

from xsimgs_amd.cameras import CameraPose, DistortedPerspectiveCamera, FisheyeCamera, max_valid_radius

STEP = 16.0 / 8191   # the radius grid the bound is read from


def test_fold_radius_closed_form():
    # rho(r) = r (1 - r^2 / 2) stops rising at r = sqrt(2/3); a long lens keeps the corner far away
    got = max_valid_radius(torch.tensor([0.1, 0.1, 0.5, 0.5]), torch.tensor([-0.5, 0, 0, 0, 0, 0, 0, 0.0]))
    assert abs(float(got) - math.sqrt(2 / 3)) <= STEP


def test_corner_radius_without_distortion():
    # no distortion: rho(r) = r, the farthest corner is at hypot(0.5 / 2, 0.53 / 2.5)
    intr = torch.tensor([2.0, 2.5, 0.5, 0.47])
    got = max_valid_radius(intr, torch.zeros(8), margin=1.5)
    corner = math.hypot(0.5 / 2.0, 0.53 / 2.5)
    assert abs(float(got) - 1.5 * corner) <= 1.5 * STEP


def test_rational_denominator_folds_earlier():
    # k4 > 0 divides the radial map down: rho(r) = r / (1 + r^2) peaks at r = 1
    got = max_valid_radius(torch.tensor([0.05, 0.05, 0.5, 0.5]), torch.tensor([0, 0, 0, 0, 0, 1.0, 0, 0]))
    assert abs(float(got) - 1.0) <= STEP


def test_pack_layouts():
    pose = CameraPose.make(device="cpu")
    d = DistortedPerspectiveCamera(pose, torch.tensor([0.9, 1.2, 0.5, 0.47]), torch.arange(8.0) * 0.01)
    assert d.pack.shape == (1, 30)
    assert torch.allclose(d.pack[0, 21:29], torch.arange(8.0) * 0.01)
    assert torch.allclose(d.pack[0, 29], d.max_radius.square()[0])
    f = FisheyeCamera(pose, torch.tensor([0.3, 0.4, 0.5, 0.5]), torch.tensor([0.1, 0.2, 0.3, 0.4]))
    assert f.pack.shape == (1, 25)
    assert torch.allclose(f.pack[0, 17:], torch.tensor([0.3, 0.4, 0.5, 0.5, 0.1, 0.2, 0.3, 0.4]))
    assert d.undistort().pack.shape == (1, 21)
