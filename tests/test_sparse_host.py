"""CPU tests of the operator surface's host logic: SparseTensor bookkeeping
(shape, layout, scale, spatial cache, replace, indexing, cat / unbind,
batch broadcast) as SP/basic.py defines it, module construction and
state-dict layout (SP/conv/conv_spconv.py), and that every kernel-backed
op refuses CPU tensors instead of falling back."""
import pytest
import torch


@pytest.fixture(scope="module")
def sp(spc):
    return spc.sparse


def _toy(sp):
    coords = torch.tensor([[0, 1, 2, 3], [0, 1, 2, 4], [0, 5, 5, 5], [1, 0, 0, 0], [1, 7, 1, 2]],
                          dtype=torch.int32)
    feats = torch.arange(5 * 3, dtype=torch.float32).reshape(5, 3)
    return sp.SparseTensor(feats, coords)


def test_shape_layout_scale(sp):
    x = _toy(sp)
    assert x.shape == torch.Size([2, 3]) and x.dim() == 2
    assert x.layout == [slice(0, 3), slice(3, 5)]
    assert x._scale == (1, 1, 1) and x._spatial_cache == {}
    assert x.data.spatial_shape == [8, 6, 6] and x.data.batch_size == 2
    assert x.dtype == torch.float32 and x.device.type == "cpu"
    # keyword form and explicit shape / layout
    y = sp.SparseTensor(feats=x.feats, coords=x.coords, shape=torch.Size([3, 3]),
                        layout=x.layout)
    assert y.shape[0] == 3 and y.layout is x.layout


def test_replace_keeps_bookkeeping(sp):
    x = _toy(sp)
    x._scale = (2, 2, 2)
    x.register_spatial_cache("k", 7)
    y = x.replace(x.feats[:, :2] * 2)
    assert y.shape == torch.Size([2, 2]) and y.layout == x.layout
    assert y._scale == (2, 2, 2) and y.get_spatial_cache("k") == 7
    assert y.coords is x.coords and y.data.indice_dict is x.data.indice_dict
    c2 = x.coords.clone()
    z = x.replace(x.feats, c2)
    assert z.coords is c2


def test_spatial_cache_is_keyed_by_scale(sp):
    x = _toy(sp)
    x.register_spatial_cache("a", 1)
    assert x.get_spatial_cache() == {"a": 1}
    x._scale = (2, 2, 2)
    assert x.get_spatial_cache("a") is None
    x.register_spatial_cache("a", 2)
    assert x._spatial_cache == {"(1, 1, 1)": {"a": 1}, "(2, 2, 2)": {"a": 2}}


def test_elemwise_keeps_only_the_left_operands_cache(sp):
    """SP/basic.py:349-364 replaces a SparseTensor operand by its feats
    before its cache check, so `x + y` carries x's spatial cache alone and
    neither operand's cache dicts change."""
    x, y = _toy(sp), _toy(sp)
    x.register_spatial_cache("a", 1)
    y.register_spatial_cache("b", 2)
    before_x = {k: dict(v) for k, v in x._spatial_cache.items()}
    z = x + y
    assert torch.equal(z.feats, 2 * x.feats)
    assert z.get_spatial_cache("a") == 1 and z.get_spatial_cache("b") is None
    assert x._spatial_cache == before_x and y.get_spatial_cache() == {"b": 2}
    w = x * 3.0 - y
    assert torch.equal(w.feats, 2 * x.feats) and w.get_spatial_cache("b") is None


def test_map_cache_validates_coordinates(sp):
    x = _toy(sp)
    calls = []
    build = lambda c: calls.append(1) or len(calls)  # noqa: E731
    assert x.data.cached("m", build) == 1
    assert x.data.cached("m", build) == 1          # same tensor, same version
    x.coords.add_(0)                                # in-place write bumps the version
    assert x.data.cached("m", build) == 2
    x.coords = x.coords.clone()                     # a new tensor
    assert x.data.cached("m", build) == 3


def test_getitem_cat_unbind(sp):
    x = _toy(sp)
    b1 = x[1]
    assert b1.shape == torch.Size([1, 3])
    assert torch.equal(b1.coords[:, 0], torch.zeros(2, dtype=torch.int32))
    assert torch.equal(b1.feats, x.feats[3:5])
    sel = x[torch.tensor([True, False])]
    assert torch.equal(sel.feats, x.feats[:3])
    cat = sp.sparse_cat([x, x])
    assert cat.shape == torch.Size([4, 3])
    assert cat.coords[:, 0].tolist() == [0, 0, 0, 1, 1, 2, 2, 2, 3, 3]
    cat1 = sp.sparse_cat([x, x], dim=1)
    assert cat1.feats.shape == (5, 6)
    parts = x.unbind(0)
    assert [p.feats.shape[0] for p in parts] == [3, 2]
    cols = x.unbind(1)
    assert len(cols) == 3 and torch.equal(cols[1].feats, x.feats[:, 1])
    rev = x[torch.tensor([1, 0])]  # items renumbered in selection order
    assert rev.coords[:, 0].tolist() == [0, 0, 1, 1, 1]
    assert torch.equal(rev.feats, torch.cat([x.feats[3:5], x.feats[:3]]))
    assert torch.equal(x[::-1].feats, rev.feats)
    with pytest.raises(ValueError):
        x[torch.tensor([0.5])]


def test_elementwise_and_batch_broadcast(sp):
    x = _toy(sp)
    per_batch = torch.tensor([[10.0, 20.0, 30.0], [1.0, 2.0, 3.0]])
    y = x + per_batch
    exp = x.feats.clone()
    exp[:3] += per_batch[0]
    exp[3:] += per_batch[1]
    assert torch.equal(y.feats, exp)
    assert torch.equal((x * 2).feats, x.feats * 2)
    assert torch.equal((1 - x).feats, 1 - x.feats)
    assert torch.equal((x / 2).feats, x.feats / 2)
    assert torch.equal((-x).feats, -x.feats)
    assert torch.equal((x - x).feats, torch.zeros_like(x.feats))
    z = sp.sparse_batch_op(x, per_batch, torch.mul)
    assert torch.equal(z.feats[4], x.feats[4] * per_batch[1])


def test_dense(sp):
    x = _toy(sp)
    d = x.dense()
    assert d.shape == (2, 3, 8, 6, 6)
    assert torch.equal(d[1, :, 7, 1, 2], x.feats[4])
    assert float(d.sum()) == float(x.feats.sum())


def test_full(sp):
    t = sp.SparseTensor.full([0, 0, 0, 1, 1, 2], (2, 4), 1.5)
    assert t.coords.shape == (2 * 2 * 2 * 3, 4) and t.shape == torch.Size([2, 4])
    assert torch.all(t.feats == 1.5)


def test_conv_module_surface(sp):
    c = sp.SparseConv3d(64, 96, 3)
    assert list(c.state_dict()) == ["conv.weight", "conv.bias"]
    assert c.conv.weight.shape == (96, 3, 3, 3, 64) and c.conv.out_channels == 96
    assert c.conv.subm and c.stride == (1, 1, 1)
    c1 = sp.SparseConv3d(64, 32, 1, bias=False)
    assert list(c1.state_dict()) == ["conv.weight"] and c1.conv.weight.shape == (32, 1, 1, 1, 64)
    s = sp.SparseConv3d(64, 128, 2, stride=2)
    assert not s.conv.subm and s.stride == (2, 2, 2)
    inv = sp.SparseInverseConv3d(128, 64, 2, stride=2)
    assert inv.conv.weight.shape == (64, 2, 2, 2, 128)
    for bad in (dict(kernel_size=3, stride=2), dict(kernel_size=5),
                dict(kernel_size=3, dilation=2), dict(kernel_size=3, padding=1)):
        with pytest.raises(NotImplementedError):
            sp.SparseConv3d(32, 32, **bad)
    with pytest.raises(NotImplementedError):
        sp.SparseInverseConv3d(32, 32, 3)


def test_q8_0_load_checks(sp):
    c = sp.SparseConv3d(32, 32, 3)
    with pytest.raises(ValueError):
        c.load_q8_0(torch.zeros(10, dtype=torch.uint8))
    with pytest.raises(ValueError):
        c.load_q8_0(torch.zeros(27 * 32 * 32 // 32 * 34, dtype=torch.uint8), layout="x")
    c.load_q8_0(torch.zeros(27 * 32 * 32 // 32 * 34, dtype=torch.uint8), layout="mesh")


def test_kernel_ops_refuse_cpu_tensors(sp, spc):
    x = _toy(sp)
    x32 = x.replace(torch.zeros(5, 32))
    for op in (sp.SparseConv3d(32, 32, 3), sp.SparseConv3d(32, 32, 1),
               sp.SparseConv3d(32, 32, 2, stride=2), sp.SparseDownsample(2),
               sp.SparseSubdivide()):
        with pytest.raises(RuntimeError, match="GPU only"):
            with torch.no_grad():
                op(x32)
    with pytest.raises(ValueError, match="Upsample cache not found"):
        sp.SparseUpsample(2)(x32)
    with pytest.raises(RuntimeError, match="GPU only"):
        spc.tables.SlatTables.build(x.coords)
