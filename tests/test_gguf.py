"""GGUF reader and conv-weight loader (the reference's converted-checkpoint
format: cpp_ggml/src/gguf_loader.cpp, cpp_ggml/scripts/gguf_schema.py,
convert_sam3d_to_gguf.py).  Files are written by tests/gguf_writer.py from
the published GGUF layout; the Q8_0 blocks come from the oracle's
restatement of the converter's quantize_q8_0 (pinned by its own tests)."""
import importlib

import numpy as np
import pytest

from gguf_writer import bf16_bytes, f16_bytes, f32_bytes, write_gguf


@pytest.fixture(scope="module")
def gg(spc):
    return importlib.import_module(spc.__name__ + ".gguf")


def test_header_metadata_and_tensors(gg, tmp_path):
    rng = np.random.default_rng(0)
    a32 = rng.standard_normal((3, 5)).astype(np.float32)
    a16 = rng.standard_normal((2, 8)).astype(np.float16)
    abf = rng.standard_normal((4, 4)).astype(np.float32)
    q8 = rng.integers(0, 256, size=2 * 34, dtype=np.uint8)
    kv = [("general.architecture", "str", "sam3d"), ("sam3d.graph_format", "u32", 1),
          ("cemb.proj_multiplier", "f32", 4.0), ("flag", "bool", True),
          ("cemb.pos_groups", "arr", ("str", ["a", "bc"])), ("big", "u64", 2 ** 40),
          ("neg", "i32", -7), ("ratio", "f64", 0.125)]
    tensors = [("t.f32", "F32", (5, 3), f32_bytes(a32)), ("t.f16", "F16", (8, 2), f16_bytes(a16)),
               ("t.bf16", "BF16", (4, 4), bf16_bytes(abf)), ("t.q8", "Q8_0", (64,), q8.tobytes())]
    for align in (None, 64):
        p = tmp_path / f"a{align}.gguf"
        write_gguf(p, kv, tensors, alignment=align)
        with gg.GGUFReader(p) as r:
            assert r.version == 3 and r.alignment == (align or 32)
            assert r.data_offset % r.alignment == 0
            for key, _, v in kv:
                want = list(v[1]) if isinstance(v, tuple) else v
                assert r.kv[key] == pytest.approx(want) if isinstance(v, float) else r.kv[key] == want
            assert set(r.tensors) == {"t.f32", "t.f16", "t.bf16", "t.q8"}
            assert r.info("t.f32").shape == (3, 5) and r.info("t.f32").ne == (5, 3)
            assert np.array_equal(r.array("t.f32"), a32)
            assert np.array_equal(r.array("t.f16"), a16)
            bits = r.array("t.bf16")
            assert bits.dtype == np.uint16
            back = (bits.astype(np.uint32) << 16).view(np.float32)
            assert np.allclose(back, abf, rtol=2 ** -8)
            assert r.info("t.q8").type_name == "Q8_0" and r.info("t.q8").nbytes == 68
            assert np.array_equal(r.array("t.q8"), q8.reshape(2, 34))
            for t in r.tensors.values():
                assert t.offset % r.alignment == 0


def test_bad_files(gg, tmp_path):
    p = tmp_path / "x.gguf"
    write_gguf(p, [], [("t", "F32", (4,), f32_bytes(np.zeros(4)))], magic=b"GGUX")
    with pytest.raises(gg.GGUFError, match="magic"):
        gg.GGUFReader(p)
    write_gguf(p, [], [("t", "F32", (4,), f32_bytes(np.zeros(4)))], version=1)
    with pytest.raises(gg.GGUFError, match="version"):
        gg.GGUFReader(p)
    write_gguf(p, [], [("t", "F32", (4,), f32_bytes(np.zeros(4)))])
    data = p.read_bytes()
    p.write_bytes(data[:40])
    with pytest.raises(gg.GGUFError):
        gg.GGUFReader(p)
    # a tensor that runs past the end of the file
    write_gguf(p, [], [("t", "F32", (4,), f32_bytes(np.zeros(4)))])
    p.write_bytes(p.read_bytes()[:-24])  # 16 bytes of padding + half the data
    with pytest.raises(gg.GGUFError, match="past the end"):
        gg.GGUFReader(p)


def _conv_gguf(tmp_path, name, tensors):
    p = tmp_path / name
    write_gguf(p, [("general.architecture", "str", "sam3d")], tensors)
    return p


def test_load_slat_mesh_and_1x1(spc, gg, tmp_path):
    import torch

    sp = spc.sparse
    rng = np.random.default_rng(1)
    cin, cout = 64, 32
    w = (rng.standard_normal((cout, 27, cin)) * 0.02).astype(np.float32)  # KRSC
    b = rng.standard_normal(cout).astype(np.float32)
    slat = w.reshape(cout, 27 * cin)                               # rows [Cout, 27*Cin]
    mesh = np.ascontiguousarray(w.transpose(1, 0, 2)).reshape(27, cout * cin)  # [27, Cout*Cin]
    w1 = rng.standard_normal((cout, 1, 1, 1, cin)).astype(np.float32)
    p = _conv_gguf(tmp_path, "c.gguf", [
        ("dit.input_blocks.0.conv1.conv.weight", "F16", (27 * cin, cout), f16_bytes(slat)),
        ("dit.input_blocks.0.conv1.conv.bias", "F32", (cout,), f32_bytes(b)),
        ("dec.upsample.0.out_layers.0.conv.weight", "F32", (cout * cin, 27), f32_bytes(mesh)),
        ("dec.upsample.0.out_layers.0.conv.bias", "F16", (cout,), f16_bytes(b)),
        ("dec.upsample.0.skip_connection.conv.weight", "F16", (cout * cin, 1), f16_bytes(w1)),
        ("dec.upsample.0.skip_connection.conv.bias", "F32", (cout,), f32_bytes(b)),
    ])
    with gg.GGUFReader(p) as r:
        c1 = sp.SparseConv3d(cin, cout, 3)
        gg.load_sparse_conv(c1, r, "dit.input_blocks.0.conv1.conv")  # inferred: slat
        got = c1.conv.weight.detach().numpy().reshape(cout, 27, cin)
        assert np.array_equal(got, w.astype(np.float16).astype(np.float32))
        assert np.array_equal(c1.conv.bias.detach().numpy(), b)
        c2 = sp.SparseConv3d(cin, cout, 3)
        gg.load_sparse_conv(c2, r, "dec.upsample.0.out_layers.0.conv")  # inferred: mesh
        assert np.array_equal(c2.conv.weight.detach().numpy().reshape(cout, 27, cin), w)
        assert np.array_equal(c2.conv.bias.detach().numpy(), b.astype(np.float16).astype(np.float32))
        c3 = sp.SparseConv3d(cin, cout, 1)
        gg.load_sparse_conv(c3, r, "dec.upsample.0.skip_connection.conv")
        # the saved buffer in saved order; the conv applies the raw view itself
        assert np.array_equal(c3.conv.weight.detach().numpy(), w1.astype(np.float16).astype(np.float32))
        with pytest.raises(gg.GGUFError, match="does not match"):
            gg.load_sparse_conv(sp.SparseConv3d(cin, cout, 3), r, "dit.input_blocks.0.conv1.conv",
                                layout="mesh")
        with pytest.raises(gg.GGUFError, match="weights"):
            gg.load_sparse_conv(sp.SparseConv3d(cin, 2 * cout, 3), r, "dit.input_blocks.0.conv1.conv")
        with pytest.raises(KeyError):
            gg.load_sparse_conv(c1, r, "missing")


def test_load_q8_0_blocks(spc, orc, gg, tmp_path):
    import torch

    sp = spc.sparse
    rng = np.random.default_rng(2)
    cin, cout = 64, 32
    w = (rng.standard_normal((cout, 27, cin)) * 0.02).astype(np.float32)
    slat_q = orc.q8_0_quantize(w)                                     # rows [Cout, 27*Cin]
    mesh_q = orc.q8_0_quantize(np.ascontiguousarray(w.transpose(1, 0, 2)))  # rows [27, Cout*Cin]
    w1 = rng.standard_normal((cout, cin)).astype(np.float32)
    q1 = orc.q8_0_quantize(w1)
    p = _conv_gguf(tmp_path, "q.gguf", [
        ("a.conv.weight", "Q8_0", (27 * cin, cout), slat_q.tobytes()),
        ("b.conv.weight", "Q8_0", (cout * cin, 27), mesh_q.tobytes()),
        ("c.conv.weight", "Q8_0", (cout * cin, 1), q1.tobytes()),
    ])
    with gg.GGUFReader(p) as r:
        ca = sp.SparseConv3d(cin, cout, 3, bias=False)
        gg.load_sparse_conv(ca, r, "a.conv")
        blocks, layout = ca._q8
        assert layout == "slat" and np.array_equal(blocks.numpy(), slat_q)
        cb = sp.SparseConv3d(cin, cout, 3, bias=False)
        gg.load_sparse_conv(cb, r, "b.conv")
        blocks, layout = cb._q8
        assert layout == "mesh" and np.array_equal(blocks.numpy(), mesh_q)
        # 1x1x1 Q8_0: dequantised once (the raw view spans block boundaries)
        cc = sp.SparseConv3d(cin, cout, 1, bias=False)
        gg.load_sparse_conv(cc, r, "c.conv")
        import oracle

        deq = orc.q8_0_dequant(q1, oracle.F32)
        assert cc._q8 is None
        assert np.array_equal(cc.conv.weight.detach().numpy().reshape(-1), deq.reshape(-1))


@pytest.mark.gpu
def test_gguf_q8_0_conv_matches_direct_load(spc, orc, dev, tmp_path):
    """A mesh-layout Q8_0 conv loaded from a GGUF file gives bit-identical
    output to the same blocks attached directly, and matches the oracle."""
    import oracle
    import torch
    from helpers import bf16_bits, from_dev, max_rel

    gg = importlib.import_module(spc.__name__ + ".gguf")
    sp = spc.sparse
    coords = spc.workloads.random_voxels(2000, 16, batches=1, seed=23)
    n = coords.shape[0]
    print(f"[case] GGUF Q8_0 mesh conv N={n} 64->64", flush=True)
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((64, 27, 64)) * 0.02).astype(np.float32)
    b = (rng.standard_normal(64) * 0.01).astype(np.float32)
    mesh_q = orc.q8_0_quantize(np.ascontiguousarray(w.transpose(1, 0, 2)))
    p = _conv_gguf(tmp_path, "m.gguf", [
        ("dec.conv.weight", "Q8_0", (64 * 64, 27), mesh_q.tobytes()),
        ("dec.conv.bias", "F32", (64,), f32_bytes(b)),
    ])
    xb = bf16_bits(orc, spc.workloads.normal((n, 64), 1.0, seed=9))
    xt = sp.SparseTensor(torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16),
                         torch.from_numpy(coords).to(dev))
    with gg.GGUFReader(p) as r:
        conv = sp.SparseConv3d(64, 64, 3)
        gg.load_sparse_conv(conv, r, "dec.conv")
    conv = conv.to(dev).to(torch.bfloat16)
    direct = sp.SparseConv3d(64, 64, 3).to(dev)
    with torch.no_grad():
        direct.conv.bias.copy_(torch.from_numpy(b))
    direct.load_q8_0(torch.from_numpy(mesh_q), layout="mesh")
    direct = direct.to(torch.bfloat16)
    with torch.no_grad():
        y = conv(xt)
        yd = direct(xt.replace(xt.feats))
    assert torch.equal(y.feats, yd.feats)
    wq = orc.q8_0_dequant(mesh_q, oracle.F16).reshape(27, 64, 64).transpose(1, 0, 2)
    bb = bf16_bits(orc, b)
    ref = orc.sparse_conv(xb, np.ascontiguousarray(wq), bb, orc.conv_table_slat(coords), ntaps=27,
                          n_out=n, idx_layout=1, out_dtype=oracle.F32, x_dtype=oracle.BF16,
                          w_dtype=oracle.F16, b_dtype=oracle.BF16)
    assert max_rel(from_dev(y.feats), ref) <= 2e-2
