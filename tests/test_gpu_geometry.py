"""The conv kernel's three tile geometries (SPC_TILES_WIDE: 256-row tiles over
a double-buffered 895-row stage; SPC_TILES_SMALL: 128-row tiles, 64 for 8
taps, over a single 511-row stage, several workgroups per CU;
SPC_TILES_TALL: 256-row tiles over a single 559-row stage, reading the wide
plan) compute every output row with the same sequence of MFMA steps --
chunks outer, active taps ascending, absent taps adding exact zeros -- so
their outputs are equal value for value, with and without a tile plan, for
every dtype, epilogue and staging path.  The small and the tall tiles are
also checked against the oracle."""
import numpy as np
import pytest

from helpers import bf16_bits, check_16bit, from_dev, oracle_threads, to_dev_bf16

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[case] {name}", flush=True)


@pytest.fixture()
def geo(spc):
    nat = spc._native
    yield nat
    nat.set_tile_geometry(nat.TILES_AUTO)


def _both(nat, fn):
    """fn() under the wide, then the small tiles (with a fresh plan each)."""
    import torch

    out = []
    for g in (nat.TILES_WIDE, nat.TILES_SMALL):
        nat.set_tile_geometry(g)
        out.append(fn())
    torch.cuda.synchronize()
    nat.set_tile_geometry(nat.TILES_AUTO)
    return out


def _all(nat, fn):
    """fn() under the wide, the small and the tall tiles (the tall ones
    apply to 27 taps; elsewhere the conv keeps its choice by shape)."""
    import torch

    out = []
    for g in (nat.TILES_WIDE, nat.TILES_SMALL, nat.TILES_TALL):
        nat.set_tile_geometry(g)
        out.append(fn())
    torch.cuda.synchronize()
    nat.set_tile_geometry(nat.TILES_AUTO)
    return out


def _inputs(spc, orc, n_in, cin, cout, ntaps, seed, dt="bf16"):
    import torch

    wl = spc.workloads
    x = wl.normal((n_in, cin), 1.0, seed=seed)
    w = wl.normal((cout, ntaps, cin), 0.05, seed=seed + 1)
    b = wl.normal((cout,), 0.1, seed=seed + 2)
    if dt == "bf16":
        x, w, b = (bf16_bits(orc, a) for a in (x, w, b))
        return (x, w, b), tuple(to_dev_bf16(a, "cuda:0") for a in (x, w, b))
    if dt == "f16":
        x, w, b = (a.astype(np.float16) for a in (x, w, b))
    return (x, w, b), tuple(torch.from_numpy(a).to("cuda:0") for a in (x, w, b))


@pytest.mark.parametrize("dt,cin,cout,nvox,grid", [
    ("bf16", 32, 32, 40000, 48), ("bf16", 64, 64, 30000, 40), ("bf16", 64, 128, 30000, 40),
    ("bf16", 128, 128, 12000, 30), ("bf16", 128, 256, 12000, 30), ("bf16", 96, 160, 9000, 28),
    ("f32", 64, 64, 20000, 36), ("f32", 32, 96, 20000, 36), ("f16", 64, 128, 15000, 32)])
def test_subm_wide_equals_small(spc, orc, dev, geo, dt, cin, cout, nvox, grid):
    import oracle
    import torch

    nat = geo
    coords = spc.workloads.random_voxels(nvox, grid, batches=2, seed=cin + cout)
    n = coords.shape[0]
    _case(f"subm {dt} N={n} {cin}->{cout}: wide vs small vs tall tiles")
    (xh, wh, bh), (x, w, b) = _inputs(spc, orc, n, cin, cout, 27, seed=cin * 7 + cout, dt=dt)
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    pw = nat.pack_weights(w)

    def run():
        plan = nat.conv_plan(m.token_major, ntaps=27, n_out=n)
        return (nat.sparse_conv(x, pw, b, m.token_major, ntaps=27, n_out=n, plan=plan),
                nat.sparse_conv(x, pw, b, m.token_major, ntaps=27, n_out=n))

    (wp, wn), (sp_, sn), (tp, tn_) = _all(nat, run)
    assert torch.equal(wp, wn) and torch.equal(sp_, sn) and torch.equal(tp, tn_)
    assert torch.equal(wp, sp_) and torch.equal(wp, tp)
    tm = m.token_major.cpu().numpy()
    code = {"bf16": oracle.BF16, "f16": oracle.F16, "f32": oracle.F32}[dt]
    ref = orc.sparse_conv(xh, wh, bh, tm, ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.F32,
                          x_dtype=code, w_dtype=code, b_dtype=code, nthreads=oracle_threads(),
                          blocked=True)
    if dt == "f32":
        assert np.all(np.abs(sp_.cpu().numpy() - ref) <= 1e-5 + 1e-4 * np.abs(ref))
    else:
        check_16bit(f"small tiles {dt} {cin}->{cout}", from_dev(sp_), ref)


@pytest.mark.parametrize("dt,cin,cout", [("bf16", 128, 128), ("bf16", 64, 64), ("bf16", 64, 32),
                                         ("bf16", 32, 64), ("bf16", 96, 32), ("bf16", 128, 1024),
                                         ("f16", 128, 128), ("f32", 64, 64)])
def test_stride2_wide_equals_small(spc, orc, dev, geo, dt, cin, cout):
    """The 2x2x2 stride-2 conv on the config-2 coords: the wide tiles' 256
    coarse rows overflow their stage (per-tap fallback), the small tiles'
    64 coarse rows (about 340 fine rows) take the staged path, and so do the
    four-buffer tiles the shape picks where its tiles fit one round (every
    case here but 128 -> 1024)."""
    import oracle
    import torch

    nat = geo
    coords = spc.workloads.ellipsoid_batch()
    nf = coords.shape[0]
    d = nat.downsample_map(torch.from_numpy(coords).to(dev), 4, 64)
    _case(f"stride-2 {dt} nf={nf} nc={d.nc} {cin}->{cout}: wide vs small vs by-shape tiles")
    (xh, wh, bh), (x, w, b) = _inputs(spc, orc, nf, cin, cout, 8, seed=cin + 3 * cout, dt=dt)
    pw = nat.pack_weights(w)

    def run():
        plan = nat.conv_plan(d.stride2_taps, ntaps=8, n_out=d.nc, n_in=nf)
        return nat.sparse_conv(x, pw, b, d.stride2_taps, ntaps=8, n_out=d.nc, plan=plan)

    yw, ys, yq = _all(nat, run)
    assert torch.equal(yw, ys) and torch.equal(yw, yq)
    code = {"bf16": oracle.BF16, "f16": oracle.F16, "f32": oracle.F32}[dt]
    ref = orc.sparse_conv(xh, wh, bh, d.stride2_taps.cpu().numpy(), ntaps=8, n_out=d.nc,
                          idx_layout=1, out_dtype=oracle.F32, x_dtype=code, w_dtype=code,
                          b_dtype=code, nthreads=oracle_threads(), blocked=True)
    if dt == "f32":
        got = yq.cpu().numpy()
        assert np.all(np.abs(got - ref) <= 1e-5 + 1e-4 * np.abs(ref))
    else:
        check_16bit(f"by-shape tiles stride-2 {dt} {cin}->{cout}", from_dev(yq), ref)


@pytest.mark.parametrize("n", [1, 5, 127, 130, 300])
def test_ragged_and_tiny(spc, orc, dev, geo, n):
    """Row counts below and just past a tile; rows with no neighbours."""
    import torch

    nat = geo
    coords = spc.workloads.random_voxels(n, 5 if n < 100 else 9, batches=1, seed=n)[:n]
    n = coords.shape[0]
    _case(f"ragged N={n}: wide vs small vs tall tiles")
    _, (x, w, b) = _inputs(spc, orc, n, 64, 64, 27, seed=n + 11)
    m = nat.map_build(torch.from_numpy(np.ascontiguousarray(coords)).to(dev))
    pw = nat.pack_weights(w)
    yw, ys, yt = _all(nat, lambda: nat.sparse_conv(x, pw, b, m.token_major, ntaps=27, n_out=n,
                                                   plan=nat.conv_plan(m.token_major, ntaps=27,
                                                                      n_out=n)))
    assert torch.equal(yw, ys) and torch.equal(yw, yt)


@pytest.mark.parametrize("n", [1, 9, 70, 700])
def test_stride2_ragged_and_tiny(spc, orc, dev, geo, n):
    """Stride-2 convs over a few fine rows (one partial 64-row tile, dead
    waves, coarse rows with one child): the wide, small and four-buffer
    tiles agree with each other and with the oracle."""
    import oracle
    import torch

    nat = geo
    coords = spc.workloads.random_voxels(n, 6 if n < 100 else 14, batches=1, seed=n + 3)[:n]
    coords = np.ascontiguousarray(coords)
    nf = coords.shape[0]
    d = nat.downsample_map(torch.from_numpy(coords).to(dev), 1, 16)
    _case(f"stride-2 ragged nf={nf} nc={d.nc} 128->128")
    (xh, wh, bh), (x, w, b) = _inputs(spc, orc, nf, 128, 128, 8, seed=n + 21)
    pw = nat.pack_weights(w)
    yw, ys, yq = _all(nat, lambda: nat.sparse_conv(
        x, pw, b, d.stride2_taps, ntaps=8, n_out=d.nc,
        plan=nat.conv_plan(d.stride2_taps, ntaps=8, n_out=d.nc, n_in=nf)))
    assert torch.equal(yw, ys) and torch.equal(yw, yq)
    ref = orc.sparse_conv(xh, wh, bh, d.stride2_taps.cpu().numpy(), ntaps=8, n_out=d.nc,
                          idx_layout=1, out_dtype=oracle.F32, x_dtype=oracle.BF16,
                          w_dtype=oracle.BF16, b_dtype=oracle.BF16, nthreads=oracle_threads(),
                          blocked=True)
    check_16bit(f"stride-2 ragged nf={nf}", from_dev(yq), ref)


@pytest.mark.parametrize("seed", range(6))
def test_stride2_random(spc, orc, dev, geo, seed):
    """Seeded random stride-2 convs (voxel count, grid, batches, 1-4 channel
    chunks, output width): the four-buffer tiles the shape picks (whole-chunk
    weight ring, each chunk staged one ahead) equal the wide and small tiles
    bit for bit and the oracle."""
    import oracle
    import torch

    nat = geo
    rng = np.random.default_rng(1000 + seed)
    n = int(rng.integers(500, 12000))
    res = int(rng.choice([24, 32, 48]))
    batches = int(rng.integers(1, 4))
    cin = int(rng.choice([32, 64, 96, 128]))
    cout = int(rng.choice([32, 64, 128]))
    coords = spc.workloads.random_voxels(n, res, batches=batches, seed=seed + 40)
    nf = coords.shape[0]
    d = nat.downsample_map(torch.from_numpy(coords).to(dev), batches, res)
    _case(f"stride-2 random seed={seed} nf={nf} nc={d.nc} res={res} B={batches} {cin}->{cout}")
    (xh, wh, bh), (x, w, b) = _inputs(spc, orc, nf, cin, cout, 8, seed=seed + 60)
    pw = nat.pack_weights(w)
    yw, ys, yq = _all(nat, lambda: nat.sparse_conv(
        x, pw, b, d.stride2_taps, ntaps=8, n_out=d.nc,
        plan=nat.conv_plan(d.stride2_taps, ntaps=8, n_out=d.nc, n_in=nf)))
    assert torch.equal(yw, ys) and torch.equal(yw, yq)
    ref = orc.sparse_conv(xh, wh, bh, d.stride2_taps.cpu().numpy(), ntaps=8, n_out=d.nc,
                          idx_layout=1, out_dtype=oracle.F32, x_dtype=oracle.BF16,
                          w_dtype=oracle.BF16, b_dtype=oracle.BF16, nthreads=oracle_threads(),
                          blocked=True)
    check_16bit(f"stride-2 random seed={seed}", from_dev(yq), ref)


def test_stride2_q8_0(spc, orc, dev, geo):
    """Stride-2 128 -> 128 with Q8_0 weights on the config-2 coords: the
    four-buffer tiles the shape picks (their weight ring holds the block
    scales too) equal the wide and small tiles and the oracle on the
    kernel's operands bf16(f32(d) * q)."""
    import oracle
    import torch

    nat = geo
    coords = spc.workloads.ellipsoid_batch()
    nf = coords.shape[0]
    d = nat.downsample_map(torch.from_numpy(coords).to(dev), 4, 64)
    _case(f"stride-2 Q8_0 nf={nf} nc={d.nc} 128->128: wide vs small vs by-shape tiles")
    (xh, _, bh), (x, _, b) = _inputs(spc, orc, nf, 128, 128, 8, seed=77)
    blocks = orc.q8_0_quantize(spc.workloads.normal((128, 8, 128), 0.05, seed=78))
    qs, dsc = nat.q8_0_repack(torch.from_numpy(blocks).to(dev))
    pq = nat.pack_weights(qs, dsc, cin=128, cout=128, ntaps=8)
    yw, ys, yq = _all(nat, lambda: nat.sparse_conv(
        x, pq, b, d.stride2_taps, ntaps=8, n_out=d.nc,
        plan=nat.conv_plan(d.stride2_taps, ntaps=8, n_out=d.nc, n_in=nf)))
    assert torch.equal(yw, ys) and torch.equal(yw, yq)
    wq = orc.q8_0_dequant(blocks, oracle.BF16)
    ref = orc.sparse_conv(xh, wq, bh, d.stride2_taps.cpu().numpy(), ntaps=8, n_out=d.nc,
                          idx_layout=1, out_dtype=oracle.F32, x_dtype=oracle.BF16,
                          w_dtype=oracle.BF16, b_dtype=oracle.BF16, nthreads=oracle_threads(),
                          blocked=True)
    check_16bit("stride-2 Q8_0 by-shape tiles", from_dev(yq), ref)


def test_q8_0_wide_equals_small(spc, orc, dev, geo):
    import torch

    nat = geo
    coords = spc.workloads.random_voxels(15000, 32, batches=2, seed=5)
    n = coords.shape[0]
    _case(f"Q8_0 N={n} 64->128: wide vs small vs tall tiles")
    g = torch.Generator(device="cpu").manual_seed(3)
    x = torch.randn((n, 64), generator=g).to(dev, torch.bfloat16)
    blocks = nat.q8_0_quantize((torch.randn((128, 27, 64), generator=g) * 0.02).to(dev))
    qs, dsc = nat.q8_0_repack(blocks)
    pw = nat.pack_weights(qs, dsc, cin=64, cout=128)
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    yw, ys, yt = _all(nat, lambda: nat.sparse_conv(x, pw, None, m.token_major, ntaps=27,
                                                   n_out=n, plan=nat.conv_plan(
                                                       m.token_major, ntaps=27, n_out=n)))
    assert torch.equal(yw, ys) and torch.equal(yw, yt)


def test_wide_span_and_fallback_small(spc, orc, dev, geo):
    """Small tiles whose sources span beyond the bitmap window (the LDS hash
    dedupe) and tiles in random row order (union beyond the 511-row stage:
    the per-tap fallback) equal the wide tiles; so do the tall tiles (the
    shuffled shell's 256-row unions exceed their 511-row stage too)."""
    import torch

    nat = geo
    g = np.stack(np.meshgrid([0], [0, 1], np.arange(2048), np.arange(16), indexing="ij"), -1)
    slabs = np.ascontiguousarray(g.reshape(-1, 4), dtype=np.int32)
    shell = spc.workloads.ellipsoid_batch(1, seed=5)
    shuffled = np.ascontiguousarray(shell[np.random.default_rng(6).permutation(len(shell))])
    for name, coords in (("two slabs", slabs), ("shuffled shell", shuffled)):
        n = coords.shape[0]
        _case(f"{name} N={n}: wide vs small vs tall tiles")
        _, (x, w, b) = _inputs(spc, orc, n, 32, 64, 27, seed=n % 1000)
        m = nat.map_build(torch.from_numpy(coords).to(dev))
        pw = nat.pack_weights(w)
        yw, ys, yt = _all(nat, lambda: nat.sparse_conv(
            x, pw, b, m.token_major, ntaps=27, n_out=n,
            plan=nat.conv_plan(m.token_major, ntaps=27, n_out=n)))
        assert torch.equal(yw, ys) and torch.equal(yw, yt)


@pytest.mark.parametrize("cout", [32, 64])
def test_epilogues_wide_equal_small(spc, orc, dev, geo, cout):
    """Residual and norm / modulation / SiLU epilogues on the small tiles,
    the residual one on the tall tiles (the norm epilogue keeps its choice
    by shape there)."""
    import torch

    nat = geo
    coords = spc.workloads.random_voxels(20000, 36, batches=3, seed=cout)
    n = coords.shape[0]
    _case(f"epilogues N={n} 64->{cout}: wide vs small vs tall tiles")
    _, (x, w, b) = _inputs(spc, orc, n, 64, cout, 27, seed=cout + 1)
    cd = torch.from_numpy(coords).to(dev)
    m = nat.map_build(cd)
    pw = nat.pack_weights(w)
    r = torch.randn((n, cout), device=dev).bfloat16()
    sc = (torch.randn((3, cout), device=dev) * 0.3).bfloat16().float()
    sh = (torch.randn((3, cout), device=dev) * 0.3).bfloat16().float()

    def run():
        plan = nat.conv_plan(m.token_major, ntaps=27, n_out=n)
        return (nat.sparse_conv(x, pw, b, m.token_major, ntaps=27, n_out=n, plan=plan,
                                residual=r),
                nat.sparse_conv(x, pw, b, m.token_major, ntaps=27, n_out=n, plan=plan,
                                norm_mod=(sc, sh, cd, 1e-6)))

    (rw, nw), (rs, ns), (rt, nt_) = _all(nat, run)
    assert torch.equal(rw, rs) and torch.equal(nw, ns)
    assert torch.equal(rw, rt) and torch.equal(nw, nt_)


def test_weight_classes_small(spc, orc, dev, geo):
    """The merged-tap child conv (8 taps, 8 weight classes, class-major row
    order) on the small tiles equals the wide tiles."""
    import torch

    nat = geo
    coords = spc.workloads.random_voxels(3000, 24, batches=1, seed=9)
    n = coords.shape[0]
    _case(f"weight classes N_parent={n}: wide vs small tiles")
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    idx, perm, class_rows = nat.subdivide_tap_classes(m.token_major, n)
    g = torch.Generator(device="cpu").manual_seed(4)
    x = torch.randn((n, 64), generator=g).to(dev, torch.bfloat16)
    w = (torch.randn((64, 64, 64), generator=g) * 0.05).to(dev, torch.bfloat16)
    pw = nat.pack_weights(w)

    def run():
        plan = nat.conv_plan(idx, ntaps=8, n_out=8 * class_rows, n_in=n, row_perm=perm)
        return nat.sparse_conv(x, pw, None, idx, ntaps=8, n_out=8 * class_rows, row_perm=perm,
                               plan=plan, class_rows=class_rows, n_classes=8,
                               out=torch.empty((8 * n, 64), dtype=torch.bfloat16, device=dev))

    yw, ys = _both(nat, run)
    assert torch.equal(yw, ys)


def test_plan_sections(spc, orc, dev, geo):
    """A plan built for one geometry only (spc_conv_plan_sections): convs of
    either geometry over it equal the convs over a full plan -- the skipped
    section's tiles carry no marker, so those convs set their tiles up
    themselves; spc_conv_tile_geometry names the section a conv reads."""
    import torch

    nat = geo
    coords = spc.workloads.ellipsoid_batch(2, seed=12)
    n = coords.shape[0]
    _case(f"plan sections N={n} 64->64")
    _, (x, w, b) = _inputs(spc, orc, n, 64, 64, 27, seed=13)
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    pw = nat.pack_weights(w)
    full = nat.conv_plan(m.token_major, ntaps=27, n_out=n)
    outs = {}
    for g in (nat.TILES_WIDE, nat.TILES_SMALL, nat.TILES_TALL):
        nat.set_tile_geometry(g)
        want = nat.PLAN_SMALL if g == nat.TILES_SMALL else nat.PLAN_WIDE
        assert nat.plan_section(torch.bfloat16, ntaps=27, n_out=n, cin=64, cout=64) == want
        for sec in (nat.PLAN_WIDE, nat.PLAN_SMALL, nat.PLAN_WIDE | nat.PLAN_SMALL):
            p = nat.conv_plan(m.token_major, ntaps=27, n_out=n, sections=sec)
            outs[(g, sec)] = nat.sparse_conv(x, pw, b, m.token_major, ntaps=27, n_out=n, plan=p)
        outs[(g, 0)] = nat.sparse_conv(x, pw, b, m.token_major, ntaps=27, n_out=n, plan=full)
    nat.set_tile_geometry(nat.TILES_AUTO)
    torch.cuda.synchronize()
    ref = outs[(nat.TILES_WIDE, 0)]
    for k, v in outs.items():
        assert torch.equal(v, ref), k
    # by shape: C=64 bf16 is one or two channel chunks -> small tiles
    assert nat.plan_section(torch.bfloat16, ntaps=27, n_out=n, cin=64, cout=64) == nat.PLAN_SMALL
    assert nat.plan_section(torch.bfloat16, ntaps=27, n_out=n, cin=128, cout=128) == nat.PLAN_WIDE
    assert nat.plan_section(torch.bfloat16, ntaps=8, n_out=n, cin=128, cout=128) == nat.PLAN_SMALL
    # one-chunk rows with C_out <= 64 -> tall tiles, which read the wide section
    tg = nat.tile_geometry(torch.bfloat16, ntaps=27, n_out=n, cin=32, cout=32)
    assert tg == nat.TILES_TALL
    assert nat.plan_section(torch.bfloat16, ntaps=27, n_out=n, cin=32, cout=64) == nat.PLAN_WIDE
    # short rows into 128 output columns: the wide tiles' double-buffered stage
    assert nat.tile_geometry(torch.bfloat16, ntaps=27, n_out=n, cin=32, cout=128) == nat.TILES_WIDE
    assert nat.tile_geometry(torch.bfloat16, ntaps=27, n_out=n, cin=64, cout=128) == nat.TILES_WIDE
    assert nat.tile_geometry(torch.bfloat16, ntaps=27, n_out=n, cin=64, cout=64) == nat.TILES_SMALL


@pytest.mark.parametrize("r", [1, 6, 15, 16, 17, 31, 32, 33, 64, 65, 129, 255])
def test_partial_tile_live_blocks(spc, orc, dev, geo, r):
    """A partial last row tile of 2 * 256 + r rows: its waves whose rows end
    inside their first row block (16 rows in 16-bit) run that block's MFMAs
    only.  bf16
    128 -> 128 on the wide tiles (64-row waves), the small tiles (64-row
    waves over 128-row tiles), the tall tiles (64-row waves over 256-row
    tiles) and Q8_0 128 -> 128 (128-row waves), every row against the
    oracle."""
    import oracle
    import torch

    nat = geo
    n = 512 + r
    coords = spc.workloads.random_voxels(n + 400, 14, batches=1, seed=r)[:n]
    coords = np.ascontiguousarray(coords)
    _case(f"partial tile N={n} (r={r}): bf16 wide / small / tall, Q8_0")
    (xh, wh, bh), (x, w, b) = _inputs(spc, orc, n, 128, 128, 27, seed=r + 5)
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    tm = m.token_major.cpu().numpy()
    pw = nat.pack_weights(w)
    yw, ys, yt = _all(nat, lambda: nat.sparse_conv(x, pw, b, m.token_major, ntaps=27, n_out=n,
                                                   plan=nat.conv_plan(m.token_major, ntaps=27,
                                                                      n_out=n)))
    ref = orc.sparse_conv(xh, wh, bh, tm, ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.F32,
                          x_dtype=oracle.BF16, w_dtype=oracle.BF16, b_dtype=oracle.BF16,
                          nthreads=oracle_threads(), blocked=True)
    check_16bit(f"partial tile wide N={n}", from_dev(yw), ref)
    check_16bit(f"partial tile small N={n}", from_dev(ys), ref)
    check_16bit(f"partial tile tall N={n}", from_dev(yt), ref)
    # Q8_0 weights (in-register dequantisation: 4 waves of 128 x 64 rows)
    blocks = orc.q8_0_quantize(spc.workloads.normal((128, 27, 128), 0.05, seed=r + 9))
    qs, dsc = nat.q8_0_repack(torch.from_numpy(blocks).to(dev))
    pq = nat.pack_weights(qs, dsc, cin=128, cout=128)
    nat.set_tile_geometry(nat.TILES_WIDE)
    yq = nat.sparse_conv(x, pq, b, m.token_major, ntaps=27, n_out=n)
    torch.cuda.synchronize()
    nat.set_tile_geometry(nat.TILES_AUTO)
    # the kernel's operands bf16(f32(d) * q): one bf16 rounding per element
    wq = orc.q8_0_dequant(blocks, oracle.BF16)
    refq = orc.sparse_conv(xh, wq, bh, tm, ntaps=27, n_out=n, idx_layout=1, out_dtype=oracle.F32,
                           x_dtype=oracle.BF16, w_dtype=oracle.BF16, b_dtype=oracle.BF16,
                           nthreads=oracle_threads(), blocked=True)
    check_16bit(f"partial tile Q8_0 wide N={n}", from_dev(yq), refq)


def _slab_block(nx, ny, nz):
    """Dense block of voxels, lexicographic rows: a tile's x +- 1 neighbours
    lie ny * nz rows away."""
    g = np.stack(np.meshgrid(np.arange(nx), np.arange(ny), np.arange(nz), indexing="ij"),
                 -1).reshape(-1, 3)
    c = np.zeros((g.shape[0], 4), np.int32)
    c[:, 1:] = g
    return c


@pytest.mark.parametrize("dims,path", [((2, 256, 60), "32768-row bitmap"),
                                       ((2, 768, 60), "65536-row bitmap"),
                                       ((2, 1120, 60), "LDS hash")])
def test_dedupe_paths(spc, orc, dev, geo, dims, path):
    """The tile setup's three deduplication paths, chosen per tile from the
    span of its source rows: dense 2 x ny x 60 blocks whose x-slabs hold
    15,360 / 46,080 / 67,200 rows put every tile's sources within 32,768,
    within 65,536 and beyond 65,536 rows (tests/test_oracle_maps.py checks the
    spans on the CPU), each union within the stage.  All paths give the same
    ascending union, so the wide, small and tall tiles, with and without a
    plan, agree bit for bit, and with the oracle."""
    import oracle
    import torch

    nat = geo
    coords = _slab_block(*dims)
    n = coords.shape[0]
    _case(f"dedupe via the {path}: N={n} bf16 32->32")
    (xh, wh, bh), (x, w, b) = _inputs(spc, orc, n, 32, 32, 27, seed=dims[1])
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    pw = nat.pack_weights(w)

    def run():
        plan = nat.conv_plan(m.token_major, ntaps=27, n_out=n)
        return (nat.sparse_conv(x, pw, b, m.token_major, ntaps=27, n_out=n, plan=plan),
                nat.sparse_conv(x, pw, b, m.token_major, ntaps=27, n_out=n))

    (wp, wn), (sp_, sn), (tp, tn_) = _all(nat, run)
    for y in (wn, sp_, sn, tp, tn_):
        assert torch.equal(y, wp)
    ref = orc.sparse_conv(xh, wh, bh, m.token_major.cpu().numpy(), ntaps=27, n_out=n,
                          idx_layout=1, out_dtype=oracle.F32, x_dtype=oracle.BF16,
                          w_dtype=oracle.BF16, b_dtype=oracle.BF16, nthreads=oracle_threads(),
                          blocked=True)
    check_16bit(f"dedupe via the {path}", from_dev(wp), ref)
