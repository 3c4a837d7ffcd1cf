"""xsg_sh_bwd_noalloc (the SH backward that allocates nothing) against xsg_sh_bwd, through the C-ABI.

Both entry points run the same kernels; the allocation-free one keeps the per-block d_origin
partials in the library's per-GPU device array instead of a caller workspace, so every output must
be bit-identical. Two calls in a row, the second on a smaller input (the array keeps the first
call's partials beyond the second's), then an empty input, and a size over the limit (rejected
before anything runs).
"""
import ctypes as C
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "xsimgs_amd", "libxsimgs_hip.so")
MAX_N = 1 << 25          # XSG_SH_BWD_NOALLOC_MAX_N
XSG_ERR_INVALID = -1


@pytest.fixture(scope="module")
def lib(dev):
    import xsimgs_amd  # noqa: F401  (loads torch's HIP runtime and this library as the package does)
    lib = C.CDLL(LIB)
    vp = C.c_void_p
    common = [C.c_int, vp, C.c_int64, C.c_int, vp, vp, vp, C.c_int, vp, C.c_int, vp, vp, vp, vp]
    lib.xsg_sh_bwd.argtypes = common + [vp, vp]
    lib.xsg_sh_bwd.restype = C.c_int
    lib.xsg_sh_bwd_noalloc.argtypes = common + [vp]
    lib.xsg_sh_bwd_noalloc.restype = C.c_int
    lib.xsg_sh_bwd_workspace_bytes.argtypes = [C.c_int64]
    lib.xsg_sh_bwd_workspace_bytes.restype = C.c_size_t
    lib.xsg_last_error.restype = C.c_char_p
    return lib


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _inputs(dev, n, degree, layout_3kn, with_dc, with_mask, seed):
    g = torch.Generator().manual_seed(seed)
    bands = (degree + 1) ** 2 + 1 - (1 if with_dc else 0)   # one unused band: must come back zero
    pos = torch.randn(n, 3, generator=g) * 5
    coeffs = torch.randn(3, bands, n, generator=g) if layout_3kn else torch.randn(n, bands, 3, generator=g)
    dc = None
    if with_dc:
        dc = torch.randn(3, n, generator=g) if layout_3kn else torch.randn(n, 3, generator=g)
    mask = (torch.randint(-2**31, 2**31 - 1, ((n + 31) // 32,), generator=g, dtype=torch.int32)
            if with_mask else None)
    d_out = torch.randn(n, 3, generator=g)
    origin = torch.tensor([0.3, -0.2, 0.1])
    D = lambda t: None if t is None else t.to(dev).contiguous()
    return dict(degree=degree, origin=D(origin), pos=D(pos), coeffs=D(coeffs), dc=D(dc), mask=D(mask),
                layout=int(layout_3kn), d_out=D(d_out), bands=bands)


def _run(lib, noalloc, x):
    n = x["pos"].shape[0]
    nan = float("nan")
    d_coeffs = torch.full_like(x["coeffs"], nan)     # every band must be written
    d_dc = torch.full_like(x["dc"], nan) if x["dc"] is not None else None
    d_pos = torch.full_like(x["pos"], nan)
    d_origin = torch.full((3,), nan, device=x["pos"].device)
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [x["degree"], _ptr(x["origin"]), n, x["bands"], _ptr(x["pos"]), _ptr(x["coeffs"]), _ptr(x["mask"]),
            x["layout"], _ptr(x["d_out"]), int(x["dc"] is not None), _ptr(d_coeffs), _ptr(d_dc), _ptr(d_pos),
            _ptr(d_origin)]
    if noalloc:
        rc = lib.xsg_sh_bwd_noalloc(*args, stream)
    else:
        ws = torch.empty(max(1, lib.xsg_sh_bwd_workspace_bytes(n)), dtype=torch.uint8, device=x["pos"].device)
        rc = lib.xsg_sh_bwd(*args, _ptr(ws), stream)
    assert rc == 0, lib.xsg_last_error()
    torch.cuda.synchronize()
    return d_coeffs, d_dc, d_pos, d_origin


def test_noalloc_equals_workspace_entry_point(lib, dev):
    cases = [  # n, degree, layout [3, K, N], separate DC, mask -- the second call is smaller
        (300_001, 3, False, False, False),
        (4_097, 2, True, True, True),
    ]
    for i, (n, degree, l3, dc, mk) in enumerate(cases):
        print(f"call {i}: n={n} degree={degree} layout_3kn={l3} dc={dc} mask={mk}", flush=True)
        x = _inputs(dev, n, degree, l3, dc, mk, seed=100 + i)
        ref = _run(lib, False, x)
        got = _run(lib, True, x)
        for name, a, b in zip(("d_coeffs", "d_coeffs_dc", "d_positions", "d_origin"), got, ref):
            if b is None:
                assert a is None
                continue
            assert torch.isfinite(a).all(), name
            assert torch.equal(a, b), f"call {i} {name}: max |diff| {float((a - b).abs().max()):.3e}"


def test_noalloc_empty_and_limit(lib, dev):
    x = _inputs(dev, 0, 1, False, False, False, seed=7)
    _, _, _, d_origin = _run(lib, True, x)
    assert torch.equal(d_origin, torch.zeros(3, device=dev))
    # over the limit: rejected on the host before any pointer is used or any kernel runs
    rc = lib.xsg_sh_bwd_noalloc(3, None, MAX_N + 1, 16, None, None, None, 0, None, 0, None, None, None, None, None)
    assert rc == XSG_ERR_INVALID
    assert b"scratch limit" in lib.xsg_last_error()
