"""MI355X-native sparse-voxel convolution for SAM 3D Objects.

The package mirrors the reference's sparse operator surface
(sam3d_objects/model/backbone/tdfy_dit/modules/sparse: SparseTensor,
SparseConv3d, SparseDownsample, SparseUpsample, SparseSubdivide) on top of
hand-written gfx950 HIP kernels reached through the C ABI of
lib/libsam3d_spconv_amd.so (include/sam3d_spconv_amd.h).  `tables` builds
the reference's SlatTables / MeshTables index structs on the GPU; `gguf`
reads converted checkpoints and attaches their conv weights; `blocks` has
the SLAT sparse residual block on the fused norm / conv-epilogue kernels.

The directory name is not a Python identifier; load it with
`__graft_entry__.load()` (registered as the module `sam3d_amd`).
"""
from . import _native, workloads  # noqa: F401

BACKEND = "hip"


def __getattr__(name):
    # the torch.nn modules import lazily so that the map/oracle tooling does
    # not pay for them
    if name in ("sparse", "tables", "gguf", "blocks"):
        import importlib

        return importlib.import_module(f".{name}", __name__)
    raise AttributeError(name)
