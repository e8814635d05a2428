"""C-ABI checks that need no GPU: the library loads, exports every function
include/sam3d_spconv_amd.h declares, and its pure-host queries answer."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "sam3d_spconv_amd.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*([a-z_0-9]+)\s*\(", text, re.M)
    return sorted(set(n for n in names if n not in ("if", "return")))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for must in ["spc_map_build", "spc_downsample_map", "spc_subdivide_map", "spc_sparse_conv",
                 "sam3d_spconv_f16_forward", "spc_q8_0_repack", "spc_scatter_mean",
                 "spc_gather_rows", "spc_map_workspace_bytes", "spc_last_error"]:
        assert must in names


def test_library_exports_every_declared_symbol(spc):
    lib = ctypes.CDLL(str(spc._native.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_host_queries(spc):
    L = spc._native.lib()
    assert L.spc_version() >= 1
    assert L.spc_status_string(3) == b"duplicate coordinate"
    for n in (1, 1000, 62710, 1 << 20):
        assert L.spc_map_workspace_bytes(n) > 12 * n
        assert L.spc_downsample_workspace_bytes(n) > 16 * n
        assert L.spc_subdivide_workspace_bytes(n) > 8 * n
        assert L.spc_scatter_mean_workspace_bytes(n, n // 8 + 1) > 4 * n


def test_cpu_tensors_are_rejected(spc):
    """No CPU fallback: the product path refuses host tensors."""
    import torch

    c = torch.zeros((4, 4), dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU only"):
        spc._native.map_build(c)
    x = torch.zeros((4, 32), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        spc._native.sparse_conv(x, torch.zeros((32, 27, 32), dtype=torch.bfloat16), None,
                                torch.zeros(108, dtype=torch.int32), ntaps=27, n_out=4)


def test_block_entries_validate_before_device_work(spc):
    """The block entry points reject bad shapes on the host, with a message,
    before any device work (no GPU needed)."""
    nat = spc._native
    L = nat.lib()
    fake = 1 << 12  # aligned, never dereferenced: validation fails first
    assert L.spc_subdivide_tap_classes(None, fake, 1000, 1000, fake, fake) == nat.BAD_SHAPE
    assert b"multiple of" in L.spc_last_error()
    assert L.spc_subdivide_tap_classes(None, fake, 1000, 768, fake, fake) == nat.BAD_SHAPE
    assert L.spc_subdivide_neighbors(None, fake, -1, fake) == nat.BAD_SHAPE
    assert L.spc_compose_rows(None, fake, 10, fake, -1, fake) == nat.BAD_SHAPE
    assert L.spc_compose_rows(None, fake + 4, 10, fake, 5, fake) == nat.BAD_ARG  # misaligned idx
    # weight classes: class_rows must be a positive multiple of 256 covering n_out
    args = (None, nat.BF16, fake, fake, None, fake, fake, nat.IDX_TOKEN_MAJOR, None, None, 8)
    assert L.spc_sparse_conv_classes(*args, 1024, 64, 64, 32, 0, 8, None) == nat.BAD_ARG
    assert L.spc_sparse_conv_classes(*args, 1024, 64, 64, 32, 100, 8, None) == nat.BAD_ARG
    assert L.spc_sparse_conv_classes(*args, 4096, 64, 64, 32, 256, 8, None) == nat.BAD_ARG
    assert b"class_rows" in L.spc_last_error()
    # GroupNorm shapes
    ws = L.spc_group_norm_workspace_bytes(1, 21766, 32)
    assert ws >= 32 * 2 * 8 * (21766 // 1024)
    assert L.spc_group_norm_stats(None, nat.BF16, fake, 1028, 32, fake, 1, 100, 1e-5, fake, fake,
                                  ws) == nat.BAD_SHAPE
    assert L.spc_group_norm_stats(None, nat.BF16, fake, 96, 32, fake, 1, 100, 1e-5, fake, fake,
                                  0) == nat.BAD_ARG  # workspace too small
    assert L.spc_group_norm_silu(None, nat.BF16, fake, 10, 100, 32, fake, 1, fake, None, None, 1,
                                 None, 10, fake) == nat.BAD_SHAPE  # c not a multiple of groups


def test_dense_map_bounds_the_grid_on_the_host(spc):
    """spc_map_build_dense takes at most 2^32 grid cells; the bound holds at
    the domain's ends, where n_batch * resolution^3 reaches 2^63 (2^18
    batches of 32768^3), and is checked before any device work."""
    nat = spc._native
    L = nat.lib()
    fake = 1 << 12
    assert L.spc_map_dense_workspace_bytes(100, 4, 1024) >= 4 << 30  # 2^32 cells: the limit
    for nb, res in ((5, 1024), (1 << 18, 1 << 15), (1, 1 << 15), (0, 64), (1, 0), (1 << 19, 1)):
        assert L.spc_map_dense_workspace_bytes(100, nb, res) == 0
        st = L.spc_map_build_dense(None, fake, 100, nb, res, 0, fake, None, None, None, None, fake,
                                   1 << 40)
        assert st == nat.BAD_SHAPE, (nb, res)
        assert b"out of range" in L.spc_last_error()
