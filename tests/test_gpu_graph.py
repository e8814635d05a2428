"""The conv path under HIP graph capture: a SLAT residual block's kernels
(LayerNorm32 + SiLU, conv with the norm / modulation / SiLU epilogue, conv
with the residual epilogue) captured once and replayed on new inputs, with
eager work and synchronisations between the replays; every replay must
equal the eager result bit for bit.  Maps, tile plans and packed weights
are built before capture (they are per coordinate set / weight)."""
import numpy as np
import pytest

from helpers import bf16_bits, to_dev_bf16

pytestmark = pytest.mark.gpu


def test_res_block_kernels_replay_in_a_hip_graph(spc, orc, dev):
    import torch

    nat, sp = spc._native, spc.sparse
    coords = spc.workloads.random_voxels(6000, 24, batches=2, seed=41)
    n = coords.shape[0]
    print(f"[case] HIP graph replay of the residual-block kernels N={n} C=128", flush=True)
    torch.manual_seed(3)
    blk = spc.blocks.SparseResBlock3d(128, 64, 128).to(dev)
    with torch.no_grad():
        for p in blk.conv2.parameters():
            p.normal_(0, 0.02)
    blk = blk.to(torch.bfloat16)
    blk.norm1.float()
    c_dev = torch.from_numpy(coords).to(dev)
    emb = torch.randn(2, 64, device=dev).bfloat16()
    with torch.no_grad():
        scale, shift = torch.chunk(blk.emb_layers(emb).float(), 2, dim=1)
    inputs = [to_dev_bf16(bf16_bits(orc, spc.workloads.normal((n, 128), 1.0, seed=50 + r)), dev)
              for r in range(4)]

    base = sp.SparseTensor(inputs[0], c_dev)  # replace() shares its maps and plans

    def chain(feats):
        x = base.replace(feats)
        h = x.replace(nat.layernorm_silu(x.feats, blk.norm1.weight, blk.norm1.bias,
                                         eps=blk.norm1.eps))
        h = blk.conv1.forward_fused(h, norm_mod=(scale, shift, blk.norm2.eps))
        return blk.conv2.forward_fused(h, residual=x.feats).feats

    with torch.no_grad():
        eager = [chain(f).clone() for f in inputs]  # builds maps, plans, packed weights
        static_in = inputs[0].clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            chain(static_in)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_out = chain(static_in)
        for r in (1, 3, 2, 0, 1):
            static_in.copy_(inputs[r])
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(static_out, eager[r]), f"replay with input {r}"
            # eager work between replays
            assert torch.equal(chain(inputs[(r + 1) % 4]), eager[(r + 1) % 4])
            torch.cuda.synchronize()
