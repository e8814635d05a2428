"""Seeded random parity sweep of the conv entry points against the oracle:
dtypes, channel widths (including the 96 / 192 wide tiles and widths 128
does not divide), 27- and 8-tap maps, row counts that give ragged and
>= 256 row tiles, coordinate sets whose tiles span more than the setup's
bitmap window, with and without a plan, with and without the residual
epilogue.  Rows are sampled for the oracle (its cost is linear in them)."""
import numpy as np
import pytest

from helpers import bf16_bits, from_dev, max_rel, row_subset, to_dev_bf16

pytestmark = pytest.mark.gpu

CASES = [
    # (seed, dtype, cin, cout, ntaps, n_target, grid, batches, plan, residual)
    (1, "bf16", 96, 160, 27, 3000, 20, 2, True, False),
    (2, "bf16", 64, 192, 27, 90000, 64, 2, True, True),
    (3, "f16", 32, 96, 27, 90000, 64, 2, True, False),
    (4, "bf16", 224, 64, 27, 5000, 24, 3, False, False),
    (5, "f32", 64, 96, 27, 4000, 24, 1, True, False),
    (6, "bf16", 128, 192, 8, 300000, 128, 1, True, False),
    (7, "f16", 160, 32, 8, 20000, 48, 2, False, False),
    (8, "bf16", 32, 32, 27, 1, 4, 1, True, True),
    (9, "bf16", 256, 256, 27, 257, 10, 1, True, True),
    (10, "bf16", 64, 64, 27, -1, 0, 0, True, True),   # two far-apart slabs (wide-span setup)
]


def _coords(spc, seed, n_target, grid, batches):
    if n_target == -1:
        g = np.stack(np.meshgrid([0], [0, 1], np.arange(2048), np.arange(16), indexing="ij"), -1)
        return np.ascontiguousarray(g.reshape(-1, 4), dtype=np.int32)
    return spc.workloads.random_voxels(n_target, grid, batches=batches, seed=seed)


@pytest.mark.parametrize("case", CASES, ids=[f"case{c[0]}" for c in CASES])
def test_random_conv_case(spc, orc, dev, case):
    import oracle
    import torch

    seed, dt, cin, cout, ntaps, n_target, grid, batches, use_plan, use_res = case
    nat, wl = spc._native, spc.workloads
    coords = _coords(spc, seed, n_target, grid, batches)
    c_dev = torch.from_numpy(coords).to(dev)
    if ntaps == 27:
        m = nat.map_build(c_dev)
        idx, n_in = m.token_major, coords.shape[0]
        n_out = n_in
    else:
        d = nat.downsample_map(c_dev, int(coords[:, 0].max()) + 1, grid)
        idx, n_in, n_out = d.stride2_taps, coords.shape[0], d.nc
    print(f"[case] random conv case{seed}: {dt} {cin}->{cout} ntaps={ntaps} n_in={n_in} "
          f"n_out={n_out} plan={use_plan} residual={use_res}", flush=True)
    code = {"bf16": oracle.BF16, "f16": oracle.F16, "f32": oracle.F32}[dt]
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dt]
    x = oracle.round_to(orc, wl.normal((n_in, cin), 1.0, seed=seed + 100), code)
    w = oracle.round_to(orc, wl.normal((cout, ntaps, cin), 0.03, seed=seed + 200), code)
    b = oracle.round_to(orc, wl.normal((cout,), 0.05, seed=seed + 300), code)
    dev_t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(tdt)  # noqa: E731
    xd, wd, bd = dev_t(x), dev_t(w), dev_t(b)
    plan = nat.conv_plan(idx, ntaps=ntaps, n_out=n_out, n_in=n_in) if use_plan else None
    r = None
    if use_res:
        r = oracle.round_to(orc, wl.normal((n_out, cout), 1.0, seed=seed + 400), code)
    y = nat.sparse_conv(xd, nat.pack_weights(wd), bd, idx, ntaps=ntaps, n_out=n_out, plan=plan,
                        residual=None if r is None else dev_t(r))
    torch.cuda.synchronize()
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([[0, n_out - 1], rng.integers(0, n_out, size=min(n_out, 600))]))
    bits = {oracle.BF16: orc.f32_to_bf16, oracle.F16: orc.f32_to_f16,
            oracle.F32: lambda a: np.ascontiguousarray(a, np.float32)}[code]
    ref = orc.sparse_conv(bits(x), bits(w), bits(b), row_subset(idx.cpu().numpy(), n_in, rows, ntaps),
                          ntaps=ntaps, n_out=len(rows), idx_layout=1, out_dtype=oracle.F32,
                          x_dtype=code, w_dtype=code, b_dtype=code)
    ref = oracle.round_to(orc, ref, code)
    if r is not None:
        ref = oracle.round_to(orc, ref + r[rows], code)
    got = from_dev(y)[rows]
    if dt == "f32":
        assert np.allclose(got, ref, rtol=1e-4, atol=1e-5)
    else:
        assert max_rel(got, ref) <= 2e-2
