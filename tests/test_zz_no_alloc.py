"""spc_map_build_noalloc -- the map build on the library's static per-device
scratch, for callers that cannot allocate -- through the C ABI, against
spc_map_build with a caller-owned workspace: bit-identical tables, masks and
argsort on two calls in a row (the second smaller, so stale scratch from the
first must not leak in), device-side errors reported with SPC_MAP_SYNC and
cleared by the next call, and sizes above the scratch's maximum refused."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MAX_N = 1 << 20


def _lib(spc):
    L = spc._native.lib()
    P, I64, I32, U32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_uint32
    L.spc_map_build_noalloc.argtypes = [P, P, I64, I32, U32, P, P, P, P, P]
    L.spc_map_build_noalloc.restype = ctypes.c_int
    return L


def _noalloc(spc, coords, flags, resolution=0):
    import torch

    n = coords.shape[0]
    dev = coords.device
    e = lambda k: torch.full((k,), -7, dtype=torch.int32, device=dev)  # noqa: E731
    outs = [e(27 * n), e(27 * n), e(n), e(n), e(n)]
    st = _lib(spc).spc_map_build_noalloc(torch.cuda.current_stream().cuda_stream,
                                         coords.data_ptr(), n, resolution, flags,
                                         *[o.data_ptr() for o in outs])
    torch.cuda.synchronize()
    return st, outs


def test_noalloc_matches_workspace_build(spc, dev):
    import torch

    nat = spc._native
    wl = spc.workloads
    # config-2 batch (62,710 voxels), then the smaller sphere shell (21,766)
    for name, c in (("4 ellipsoid shells", wl.ellipsoid_batch()),
                    ("sphere shell", wl.sphere_shell())):
        print(f"[case] spc_map_build_noalloc {name} N={c.shape[0]}", flush=True)
        cd = torch.from_numpy(c).to(dev)
        st, (tm, om, ms, ar, mn) = _noalloc(spc, cd, nat.MAP_SYNC)
        assert st == nat.OK, _lib(spc).spc_last_error()
        ref = nat.map_build(cd)
        torch.cuda.synchronize()
        assert torch.equal(tm, ref.token_major)
        assert torch.equal(om, ref.offset_major)
        assert torch.equal(ms, ref.mask_sorted)
        assert torch.equal(ar, ref.argsort)
        assert torch.equal(mn, ref.mask_natural)


def test_noalloc_status_and_limits(spc, dev):
    import torch

    nat = spc._native
    L = _lib(spc)
    print("[case] spc_map_build_noalloc status word and size limit", flush=True)
    # mesh semantics: a duplicate coordinate is reported with SPC_MAP_SYNC ...
    c = spc.workloads.random_voxels(3000, 30, batches=1, seed=5)
    dup = np.concatenate([c, c[:1]], 0)
    st, _ = _noalloc(spc, torch.from_numpy(np.ascontiguousarray(dup)).to(dev),
                     nat.MAP_MESH | nat.MAP_SYNC, 32)
    assert st == nat.DUP_COORD
    # ... and the next call's init clears the shared status word
    cd = torch.from_numpy(c).to(dev)
    st, (tm, *_) = _noalloc(spc, cd, nat.MAP_MESH | nat.MAP_SYNC, 32)
    assert st == nat.OK
    assert torch.equal(tm, nat.map_build(cd, mesh_resolution=32).token_major)
    # above the scratch's maximum: refused on the host, outputs untouched
    big = torch.zeros((MAX_N + 1, 4), dtype=torch.int32, device=dev)
    st, outs = _noalloc(spc, big, nat.MAP_SYNC)
    assert st == nat.BAD_SHAPE
    assert b"static scratch" in L.spc_last_error()
    assert bool((outs[0] == -7).all())
