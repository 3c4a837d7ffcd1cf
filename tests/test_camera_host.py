"""Host-side camera logic (no GPU): pack layouts of the distorted / fisheye models, the
max-radius bound of the distorted model (the fold of the radial map, or a margin past the image
corner, whichever comes first) and the lidar pack's beam-table address."""
import math

import torch

from xsimgs_amd.cameras import CameraPose, DistortedPerspectiveCamera, FisheyeCamera, LidarCamera, max_valid_radius

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


def _packed_address(pack):
    lo, hi = (int(b) & 0xffffffff for b in pack[0, -2:].contiguous().view(torch.int32))
    return lo | (hi << 32)


def test_lidar_pack_carries_the_beam_table_address():
    # the pack's last two floats are beam_v's address (two float32 bit patterns); the address tensor is
    # built once per address (a blocking host-to-device copy on a GPU) and rebuilt when beam_v moves
    cam = LidarCamera(CameraPose.make(device="cpu"), torch.tensor([0.0, 2 * math.pi, -0.3, 0.6]),
                      torch.linspace(0.0, 1.0, 16))
    first = cam.pack
    assert first.shape == (1, 23)
    assert _packed_address(first) == cam.beam_v.data_ptr()
    assert cam._beam_addr() is cam._beam_addr()
    old = cam.beam_v
    cam.beam_v = torch.linspace(0.0, 1.0, 16) * 0.5
    assert cam.beam_v.data_ptr() != old.data_ptr()
    assert _packed_address(cam.pack) == cam.beam_v.data_ptr()
    cam.beam_v.mul_(2.0)  # values changed in place: the address, and so the pack's address, stay
    assert _packed_address(cam.pack) == cam.beam_v.data_ptr()
