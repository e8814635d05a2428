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
