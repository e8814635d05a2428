#!/usr/bin/env python3
"""One-GPU sparse-conv benchmark (MI355X).

Default workload: submanifold 3x3x3 sparse conv, bf16 features and weights
with F32 accumulation, C_in = C_out = 128, batch of 4 ellipsoid shells in a
64^3 grid (semi-axes U(16,28), Haar rotations, seed 2024; N = 62,710 voxels,
1,306,542 valid taps).  A step is one conv forward over the whole batch with
the kernel map already built and every input resident in HBM -- the SLAT IO
block loop reuses one map for every conv of every sampling step.

Reported:
  value          Mvoxel/s = N / t_step
  tflops         algorithmic TFLOP/s = 2 * pairs * C_in * C_out / t_step
  roofline       the conv kernel against the dense bf16 MFMA peak (2.5 PFLOP/s)
  map_build_ms   GPU neighbour-map build (hash + 27-offset query + stable mask
                 argsort) for the same coordinates
  cpu_baseline   the oracle's restatement of the ggml CPU op (F32 accumulate,
                 token partition) on the host cores, over a bounded sample of
                 output rows
Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--config 2]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "sparse-conv Mvoxel/s + TFLOP/s (% bf16 MFMA peak), 64³ shell N≈20k C=128"
PEAK_BF16_TFLOPS = 2500.0
PEAK_F32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=2, choices=[0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10],
                    help="2 = the headline workload; others print diagnostic lines (0 = one "
                         "sphere shell, N = 21,766, bf16 C = 128; 9 = feature ops' HBM GB/s)")
    ap.add_argument("--order", choices=["natural", "mask"], default="natural",
                    help="row processing order of the conv kernel")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--headline-only", action="store_true",
                    help="configs 0, 1, 2, 5: time the conv only (no single-shell, bridge, "
                         "f16-operand or library-GEMM lines), for counter runs")
    ap.add_argument("--fused-only", action="store_true",
                    help="configs 6 / 7: time the fused block only (no unfused comparison)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="target duration of the all-core CPU baseline sample (5 runs)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only time a 256 MiB device copy (PMC traffic calibration)")
    ap.add_argument("--tiles", choices=["auto", "wide", "small", "tall"], default="auto",
                    help="conv tile geometry (auto: each conv picks by shape)")
    ap.add_argument("--bf16-weights", action="store_true",
                    help="config 5: the same conv with bf16 weights (no Q8_0 dequantisation)")
    ap.add_argument("--q8-in-registers", action="store_true",
                    help="config 5: dequantise Q8_0 in the conv's registers (once per row tile) "
                         "instead of expanding the packed weights once per step")
    return ap.parse_args()


def bf16_dev(orc, a, dev):
    import torch

    bits = orc.f32_to_bf16(np.ascontiguousarray(a, dtype=np.float32))
    return torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16), bits


class ConvCall:
    """Pre-extracted arguments of one spc_sparse_conv launch (keeps Python
    overhead per step at a single ctypes call)."""

    def __init__(self, nat, x, w, bias, y, idx, *, ntaps, n_out, layout, perm=None,
                 w_scale=None, wdt=None, plan=None, expand_q8=False):
        import torch

        self.fn = nat.lib().spc_sparse_conv_plan
        self.stream = torch.cuda.current_stream().cuda_stream
        dt = nat.dtype_code(x.dtype)
        self.expand = None
        if expand_q8:
            # each step: packed Q8_0 -> packed bf16 (one HBM pass), then the
            # bf16 conv on the expansion
            wx = nat.expand_q8_0(w)
            self.expand = (nat.lib().spc_conv_expand_q8_0,
                           (self.stream, w.data.data_ptr(), w.ntaps, w.cin, w.cout,
                            wx.data.data_ptr()))
            w = wx
        if isinstance(w, nat.PackedWeights):
            wd, layout_w, wptr, sptr = w.w_dtype, nat.W_PACKED, w.data.data_ptr(), None
        else:
            wd = wdt if wdt is not None else dt
            layout_w, wptr = nat.W_KRSC, w.data_ptr()
            sptr = None if w_scale is None else w_scale.data_ptr()
        self.args = (self.stream, dt, x.data_ptr(), wd, layout_w, wptr, sptr,
                     None if bias is None else bias.data_ptr(), y.data_ptr(), idx.data_ptr(),
                     layout, None if perm is None else perm.data_ptr(),
                     None if plan is None else plan.data_ptr(), ntaps, n_out,
                     x.shape[0], x.shape[1], y.shape[1])
        self.nat = nat

    def __call__(self):
        if self.expand is not None:
            st = self.expand[0](*self.expand[1])
            if st != 0:
                self.nat._check("spc_conv_expand_q8_0", st)
        st = self.fn(*self.args)
        if st != 0:
            self.nat._check("spc_sparse_conv", st)


def time_gpu(fn, steps, warmup):
    """Warm-up, then K steps between events recorded on the launch stream."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(stop) / steps, wall


def library_gemm_tflops(dev, dtype, m: int = 8192, steps: int = 20) -> dict:
    """Dense m x m x m GEMM through torch.matmul (the ROCm BLAS libraries,
    hipBLASLt for bf16): a measured ceiling beside the published peak."""
    import torch

    a = torch.randn(m, m, device=dev).to(dtype)
    b = torch.randn(m, m, device=dev).to(dtype)
    ms, _ = time_gpu(lambda: torch.matmul(a, b), steps, 3)
    del a, b
    return {"tflops": 2.0 * m ** 3 / (ms / 1e3) / 1e12, "shape": f"{m}x{m}x{m}",
            "dtype": str(dtype).replace("torch.", ""), "library": "torch.matmul (hipBLASLt)"}


def traffic_from_profile(name: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, calibrated against a copy kernel), if the summary exists."""
    p = ROOT / "profiles" / f"{name}_pmc.md"
    if not p.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch\s*=\s*([0-9.eE+]+)", p.read_text())
    return float(m.group(1)) if m else None


def _host_cpu():
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            m = re.search(r"model name\s*:\s*(.*)", f.read())
            model = m.group(1).strip() if m else ""
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return model, avail


def cpu_baseline(orc, x_bits, w_bits, b_bits, tm, coords, n, cin, cout, target_s, ntaps=27,
                 x_dt=None, w_dt=None):
    """Times the oracle conv (the ggml CPU op's F32-accumulate loop, token
    partition across threads) on the host over the first S output rows, S
    sized so one run lasts about target_s / 5: 1 warm-up, median of 5.  Also
    one thread (the op's likely n_tasks = 1) and the std::map neighbour-map
    build on one thread."""
    import oracle

    x_dt = oracle.BF16 if x_dt is None else x_dt
    w_dt = oracle.BF16 if w_dt is None else w_dt
    threads = min(oracle.cpu_threads(), 16)
    tmr = tm.reshape(n, ntaps)

    def run(rows, th):
        sub = np.ascontiguousarray(tmr[:rows]).reshape(-1)
        t0 = time.perf_counter()
        orc.sparse_conv(x_bits, w_bits, b_bits, sub, ntaps=ntaps, n_out=rows, idx_layout=1,
                        out_dtype=oracle.F32, x_dtype=x_dt, w_dtype=w_dt, b_dtype=x_dt,
                        nthreads=th)
        return time.perf_counter() - t0

    def median_of(k, fn):
        fn()  # warm-up
        return float(np.median([fn() for _ in range(k)]))

    probe = min(n, 64 * threads)
    t = run(probe, threads)
    rows = int(min(n, max(probe, probe * (target_s / 5) / max(t, 1e-6))))
    t_all = median_of(5, lambda: run(rows, threads))
    t1 = run(64, 1)
    rows1 = int(min(n, max(64, 64 * (target_s / 10) / max(t1, 1e-6))))
    t_one = median_of(5, lambda: run(rows1, 1))

    def build_map():
        t0 = time.perf_counter()
        tm_c = orc.conv_table_slat(coords)
        orc.spconv_tables(tm_c, n)
        return time.perf_counter() - t0

    t_map = median_of(5, build_map)
    model, avail = _host_cpu()
    return {
        "value": rows / t_all / 1e6, "unit": "Mvoxel/s", "cores": threads, "kind": "port",
        "sample": f"first {rows} of {n} output rows, {threads} threads (the op's token "
                  f"partition), 1 warm-up + median of 5; host '{model}', {avail} CPUs "
                  "available",
        "single_thread": {"value": rows1 / t_one / 1e6, "unit": "Mvoxel/s", "cores": 1,
                          "sample": f"first {rows1} rows, 1 thread, 1 warm-up + median of 5"},
        "map_build_1thread_ms": {"value": t_map * 1e3, "cores": 1,
                                 "sample": f"std::map 27-offset table + stable mask argsort, "
                                           f"all {n} voxels, median of 5"},
    }


def bench_q8_f16_operands(nat, x, pq8, bias, idx, plan, n, flops, steps=50, warmup=10):
    """Config 5 with the reference's GEMM operands (the sparse module's
    default for Q8_0 under bf16 features): bf16 features cast to f16, the
    packed quants expanded to f16(f32(d) * q), the f16 conv, the output cast
    back to bf16 -- all four launches timed per step."""
    import torch

    L = nat.lib()
    s = torch.cuda.current_stream().cuda_stream
    cout = pq8.cout
    x16 = torch.empty(x.shape, dtype=torch.float16, device=x.device)
    b16 = nat.convert(bias, torch.float16)
    w16 = nat.expand_q8_0(pq8, dtype=torch.float16)
    y16 = torch.empty((n, cout), dtype=torch.float16, device=x.device)
    y = torch.empty((n, cout), dtype=torch.bfloat16, device=x.device)
    conv = ConvCall(nat, x16, w16, b16, y16, idx, ntaps=27, n_out=n, layout=nat.IDX_TOKEN_MAJOR,
                    plan=plan)

    def step():
        st = L.spc_convert(s, nat.BF16, x.data_ptr(), nat.F16, x16.data_ptr(), x.numel())
        st |= L.spc_conv_expand_q8_0_to(s, pq8.data.data_ptr(), 27, pq8.cin, cout, nat.F16,
                                        w16.data.data_ptr())
        conv()
        st |= L.spc_convert(s, nat.F16, y16.data_ptr(), nat.BF16, y.data_ptr(), y.numel())
        if st != 0:
            raise RuntimeError("f16-operand Q8_0 step failed")

    ms, _ = time_gpu(step, steps, warmup)
    ms_conv, _ = time_gpu(conv, steps, warmup)
    return {"ms_per_step": ms, "tflops": flops / (ms / 1e3) / 1e12,
            "conv_only_ms": ms_conv,
            "path": "cast bf16->f16 + expand Q8_0 to f16(d*q) + f16 conv + cast f16->bf16"}


def copy_calibration(steps: int):
    """Plain device-to-device copies of a known size: the FETCH_SIZE /
    WRITE_SIZE scale factors for the conv kernel's PMC traffic."""
    import torch

    nbytes = 256 << 20
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    ms, _ = time_gpu(lambda: dst.copy_(src), steps, 3)
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes,
                      "ms_per_copy": ms, "gbs": 2 * nbytes / (ms / 1e3) / 1e9}))


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE "
              f"{world}); every box here has one GPU and this build has no multi-GPU path. "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        copy_calibration(args.steps)
        return

    import __graft_entry__

    spc = __graft_entry__.load()
    nat = spc._native
    wl = spc.workloads
    import oracle

    orc = oracle.orc()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    nat.set_tile_geometry({"auto": nat.TILES_AUTO, "wide": nat.TILES_WIDE,
                           "small": nat.TILES_SMALL, "tall": nat.TILES_TALL}[args.tiles])
    cfg = args.config
    if cfg == 2:
        coords = wl.ellipsoid_batch()
        cin = cout = 128
        batch = 4
        workload = "subm3x3x3 bf16 C=128, 4 ellipsoid shells 64^3 (N=62,710)"
    elif cfg == 0:
        coords = wl.sphere_shell()
        cin = cout = 128
        batch = 1
        workload = "subm3x3x3 bf16 C=128, one sphere shell r=24 in 64^3 (N=21,766)"
    elif cfg == 10:
        coords = wl.ellipsoid_batch()
        cin = cout = 128
        batch = 4
        workload = ("SLAT IO residual blocks: SparseResBlock3d(128 -> 1024, downsample) on the 4 "
                    "ellipsoid shells (62,710 -> 11,774 rows) and SparseResBlock3d(2048 -> 128, "
                    "upsample) back to the fine rows, bf16")
    elif cfg == 9:
        coords = wl.ellipsoid_batch()
        cin = cout = 128
        batch = 4
        workload = ("feature ops of the SLAT IO blocks on the 4 ellipsoid shells (62,710 fine, "
                    "11,774 coarse rows), bf16")
    elif cfg == 1:
        coords = wl.sphere_shell()
        cin = cout = 64
        batch = 1
        workload = "subm3x3x3 fp32 C=64, sphere shell r=24 in 64^3 (N=21,766)"
    elif cfg == 5:
        coords = wl.sphere_shell()
        cin = cout = 768
        batch = 1
        workload = "subm3x3x3 Q8_0 weights, bf16 activations, C=768, sphere shell 64^3"
    elif cfg == 3:
        coords = wl.ellipsoid_batch()
        cin, cout = 128, 1024
        batch = 4
        workload = "stride-2 2x2x2 conv 128->128 then subm3x3x3 128->1024 at 32^3 (bf16)"
    elif cfg == 6:
        coords = wl.ellipsoid_batch()
        cin = cout = 128
        batch = 4
        workload = ("SLAT sparse residual block (LayerNorm32, SiLU, subm3x3x3, LayerNorm, "
                    "modulation, SiLU, subm3x3x3, + skip), bf16 C=128, 4 ellipsoid shells 64^3")
    elif cfg == 7:
        coords = wl.sphere_shell()
        cin, cout = 768, 192
        batch = 1
        workload = ("mesh-decoder upsample block (GroupNorm32, SiLU, subdivide, subm3x3x3 "
                    "768->192, GroupNorm32, SiLU, subm3x3x3, + 1x1x1 skip), bf16, sphere shell "
                    "64^3 -> 128^3")
    elif cfg == 8:
        # the first block's output support: every sphere-shell voxel's 8 children
        par = wl.sphere_shell()
        kids = np.array([[0, dx, dy, dz] for dx in (0, 1) for dy in (0, 1) for dz in (0, 1)],
                        np.int32)
        coords = (par[:, None, :] * np.array([1, 2, 2, 2], np.int32) + kids[None]).reshape(-1, 4)
        coords = np.ascontiguousarray(coords, dtype=np.int32)
        cin, cout = 192, 96
        batch = 1
        workload = ("mesh-decoder second upsample block (GroupNorm32, SiLU, subdivide, subm3x3x3 "
                    "192->96, GroupNorm32, SiLU, subm3x3x3, + 1x1x1 skip), bf16, subdivided "
                    "sphere shell 128^3 -> 256^3")
    else:
        coords = wl.sphere_shell()
        cin = cout = 64
        batch = 1
        workload = "subdivide x2 (50% pruning) + subm3x3x3 bf16 C=64 @128^3, C=32 @256^3"

    n = coords.shape[0]
    c_dev = torch.from_numpy(coords).to(dev)

    # ---- map build (timed separately; maps are reused by every conv) ----
    # the dense grid when the batch count and the grid bound it (what the
    # sparse module builds), and the hash table for comparison
    n_batch, res = int(coords[:, 0].max()) + 1, int(coords[:, 1:].max()) + 1
    ext = (n_batch, res) if n_batch * res ** 3 <= nat.DENSE_MAX_CELLS else None
    ws = torch.empty(nat.lib().spc_map_workspace_bytes(n), dtype=torch.uint8, device=dev)
    m = nat.map_build(c_dev, workspace=ws)
    map_hash_ms, _ = time_gpu(lambda: nat.map_build(c_dev, sync=False, workspace=ws), 50, 5)
    map_ms = map_hash_ms
    if ext is not None:
        wsd = torch.empty(nat.lib().spc_map_dense_workspace_bytes(n, *ext), dtype=torch.uint8,
                          device=dev)
        md = nat.map_build(c_dev, workspace=wsd, dense=ext)
        if not (torch.equal(md.token_major, m.token_major) and torch.equal(md.argsort, m.argsort)):
            raise RuntimeError("dense and hash map builds differ")
        map_ms, _ = time_gpu(lambda: nat.map_build(c_dev, sync=False, workspace=wsd, dense=ext),
                             50, 5)
    # the token-major table alone (no spconv mask / argsort tables): what the
    # sparse module builds for its convs
    map_token_ms, _ = time_gpu(lambda: nat.map_build(c_dev, sync=False, outputs="token",
                                                     workspace=wsd if ext is not None else ws,
                                                     dense=ext), 50, 5)
    tm_host = m.token_major.cpu().numpy()
    pairs = int((tm_host < n).sum())
    map_bytes = 16 * n + 108 * n + 8 * n

    result = {}
    if cfg in (2, 0, 1, 5):
        torch.manual_seed(0)
        xf = wl.normal((n, cin), 1.0, seed=101)
        wf = wl.normal((cout, 27, cin), 0.02, seed=102)
        bf = wl.normal((cout,), 0.01, seed=103) if cfg != 1 else np.zeros(cout, np.float32)
        y = torch.empty((n, cout), dtype=torch.float32 if cfg == 1 else torch.bfloat16,
                        device=dev)
        perm = m.argsort if args.order == "mask" else None
        idx = m.offset_major if args.order == "mask" else m.token_major
        layout = nat.IDX_OFFSET_MAJOR if args.order == "mask" else nat.IDX_TOKEN_MAJOR
        plan = nat.conv_plan(idx, ntaps=27, n_out=n, idx_layout=layout, row_perm=perm)
        plan_ms, _ = time_gpu(lambda: nat.conv_plan(idx, ntaps=27, n_out=n, idx_layout=layout,
                                                    row_perm=perm), 50, 5)
        if cfg == 1:
            x = torch.from_numpy(xf).to(dev)
            w = torch.from_numpy(wf).to(dev)
            b = torch.from_numpy(bf).to(dev)
            call = ConvCall(nat, x, nat.pack_weights(w), b, y, idx, ntaps=27, n_out=n,
                            layout=layout, perm=perm, plan=plan)
            dtype = "f32"
            peak = PEAK_F32_TFLOPS
            xb, wb, bb = xf, wf, bf
            cpu_dt = (oracle.F32, oracle.F32)
            w_bytes = wf.nbytes
            es = 4
        elif cfg in (2, 0):
            x, xb = bf16_dev(orc, xf, dev)
            w, wb = bf16_dev(orc, wf, dev)
            b, bb = bf16_dev(orc, bf, dev)
            call = ConvCall(nat, x, nat.pack_weights(w), b, y, idx, ntaps=27, n_out=n,
                            layout=layout, perm=perm, plan=plan)
            dtype = "bf16"
            peak = PEAK_BF16_TFLOPS
            cpu_dt = (oracle.BF16, oracle.BF16)
            w_bytes = wb.nbytes
            es = 2
        elif args.bf16_weights:  # config 5's shape with bf16 weights: the dequant's cost
            x, xb = bf16_dev(orc, xf, dev)
            w, wb = bf16_dev(orc, wf, dev)
            b, bb = bf16_dev(orc, bf, dev)
            call = ConvCall(nat, x, nat.pack_weights(w), b, y, idx, ntaps=27, n_out=n,
                            layout=layout, perm=perm, plan=plan)
            dtype = "bf16"
            peak = PEAK_BF16_TFLOPS
            cpu_dt = (oracle.BF16, oracle.BF16)
            w_bytes = wb.nbytes
            es = 2
        else:
            x, xb = bf16_dev(orc, xf, dev)
            b, bb = bf16_dev(orc, bf, dev)
            blocks = orc.q8_0_quantize(wf)
            qs, dsc = nat.q8_0_repack(torch.from_numpy(blocks).to(dev))
            call = ConvCall(nat, x, nat.pack_weights(qs, dsc, cin=cin, cout=cout), b, y, idx,
                            ntaps=27, n_out=n, layout=layout, perm=perm, plan=plan,
                            expand_q8=not args.q8_in_registers)
            dtype = "bf16 x Q8_0"
            peak = PEAK_BF16_TFLOPS
            wb = orc.q8_0_dequant(blocks, oracle.F16)
            cpu_dt = (oracle.BF16, oracle.F16)
            w_bytes = blocks.nbytes
            es = 2
        # The run's other lines are measured first: besides what they report,
        # they hold the GPU under load for ~0.1 s, which brings its clock to
        # the sustained state a serving loop runs in (the power management
        # ramps over ~50 ms of load: config 2 timed after 20 / 200 / 1000 /
        # 3000 warm-up steps from idle took 55.5-56.8 / 51.9 / 49.3 / 49.3 us).
        pre = {}
        if not args.headline_only:
            if dtype == "bf16":
                pre["measured_gemm_peak"] = library_gemm_tflops(dev, torch.bfloat16)
            if cfg == 2:
                pre["bridge"] = bench_bridge(nat, wl, c_dev, dev, args)
                # the metric's named shape (one sphere shell, its own warm-up)
                pre["single_shell"] = bench_single_shell(nat, wl, orc, dev, args)
        ms, wall = time_gpu(call, args.steps, args.warmup)
        t = ms / 1e3
        flops = 2.0 * pairs * cin * cout
        tflops = flops / t / 1e12
        comp_bytes = n * cin * es + n * cout * es + w_bytes + 108 * n
        traffic = traffic_from_profile({2: "conv_bf16_ellipsoids4_c128", 1: "conv_f32_sphere_c64",
                                        5: "conv_q8_0_sphere_c768",
                                        0: "conv_bf16_sphere64_c128"}[cfg])
        result = {
            "metric": METRIC if cfg == 2 else f"config {cfg}: {workload}",
            "value": n / t / 1e6, "unit": "Mvoxel/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": "synthetic",
            "config": {"workload": workload, "n_voxels": n, "pairs": pairs, "cin": cin,
                       "cout": cout, "batch": batch, "ntaps": 27, "row_order": args.order,
                       "tiles": args.tiles,
                       "shell_rule": "|dist to surface| <= 1.5 voxel"},
            "tflops": tflops, "pct_peak": 100.0 * tflops / peak,
            "dense_equiv_tflops": 2.0 * 27 * n * cin * cout / t / 1e12,
            "wall_s": wall, "map_build_ms": map_ms, "map_build_hash_ms": map_hash_ms,
            "map_build_token_only_ms": map_token_ms,
            "map_build_kind": "dense grid" if ext is not None else "hash table",
            "map_build_gbs": map_bytes / (map_ms / 1e3) / 1e9,
            "conv_plan_ms": plan_ms,
            "compulsory_gbs": comp_bytes / t / 1e9,
            "roofline": {"bound": "mfma", "achieved": tflops, "peak": peak, "unit": "TFLOP/s",
                         "frac": tflops / peak, "traffic": traffic,
                         "kernel": "conv_kernel (gather -> MFMA implicit GEMM -> store)",
                         "algorithmic_flops_per_launch": flops},
        }
        if cfg == 5 and not args.bf16_weights:
            result["config"]["q8_path"] = ("dequant in registers" if args.q8_in_registers else
                                           "expand to packed bf16 + bf16 conv, both timed")
            if not args.headline_only:
                result["f16_operands"] = bench_q8_f16_operands(
                    nat, x, nat.pack_weights(qs, dsc, cin=cin, cout=cout), b, idx, plan, n, flops)
        for k in ("single_shell", "bridge"):
            if k in pre:
                result[k] = pre[k]
        if "measured_gemm_peak" in pre:
            g = pre["measured_gemm_peak"]
            g["conv_fraction"] = tflops / g["tflops"]
            result["measured_gemm_peak"] = g
        result["gpu_state"] = ("timed after the run's other lines (" + ", ".join(sorted(pre)) +
                               "), at the sustained clock" if pre else
                               "timed right after the map build and plan (headline only)")
        if not args.no_cpu:
            result["cpu_baseline"] = cpu_baseline(orc, xb, wb, bb, tm_host, coords, n, cin,
                                                  cout, args.cpu_seconds, x_dt=cpu_dt[0],
                                                  w_dt=cpu_dt[1])
    elif cfg == 3:
        d = nat.downsample_map(c_dev, 4, 64)
        nc = d.nc
        mc = nat.map_build(d.coarse_coords)
        pairs_c = int((mc.token_major < nc).sum().item())
        x, _ = bf16_dev(orc, wl.normal((n, cin), 1.0, seed=301), dev)
        w1, _ = bf16_dev(orc, wl.normal((128, 8, cin), 0.02, seed=302), dev)
        w2, _ = bf16_dev(orc, wl.normal((cout, 27, 128), 0.02, seed=303), dev)
        h = torch.empty((nc, 128), dtype=torch.bfloat16, device=dev)
        y = torch.empty((nc, cout), dtype=torch.bfloat16, device=dev)
        p1 = nat.conv_plan(d.stride2_taps, ntaps=8, n_out=nc, n_in=n)
        c1 = ConvCall(nat, x, nat.pack_weights(w1), None, h, d.stride2_taps, ntaps=8, n_out=nc,
                      layout=nat.IDX_TOKEN_MAJOR, plan=p1)
        c2 = ConvCall(nat, h, nat.pack_weights(w2), None, y, mc.token_major, ntaps=27, n_out=nc,
                      layout=nat.IDX_TOKEN_MAJOR, plan=mc.plan())
        ms1, _ = time_gpu(c1, args.steps, args.warmup)
        ms2, _ = time_gpu(c2, args.steps, args.warmup)
        f1 = 2.0 * n * cin * 128
        f2 = 2.0 * pairs_c * 128 * cout
        ms = ms1 + ms2
        # the wide layer as well: SubM 1024 -> 1024 on the same coarse map
        y2 = torch.empty((nc, cout), dtype=torch.bfloat16, device=dev)
        w3, _ = bf16_dev(orc, wl.normal((cout, 27, cout), 0.02, seed=304), dev)
        c3 = ConvCall(nat, y, nat.pack_weights(w3), None, y2, mc.token_major, ntaps=27, n_out=nc,
                      layout=nat.IDX_TOKEN_MAJOR, plan=mc.plan())
        ms3, _ = time_gpu(c3, args.steps, args.warmup)
        f3 = 2.0 * pairs_c * cout * cout
        result = {"metric": f"config 3: {workload}", "value": nc / (ms / 1e3) / 1e6,
                  "unit": "Mvoxel/s", "ms_per_step": ms, "dtype": "bf16",
                  "config": {"workload": workload, "nf": n, "nc": nc, "pairs_coarse": pairs_c},
                  "stride2_ms": ms1, "stride2_tflops": f1 / (ms1 / 1e3) / 1e12,
                  "subm_ms": ms2, "subm_tflops": f2 / (ms2 / 1e3) / 1e12,
                  "pct_peak_subm": 100 * f2 / (ms2 / 1e3) / 1e12 / PEAK_BF16_TFLOPS,
                  "subm1024_ms": ms3, "subm1024_tflops": f3 / (ms3 / 1e3) / 1e12,
                  "pct_peak_subm1024": 100 * f3 / (ms3 / 1e3) / 1e12 / PEAK_BF16_TFLOPS}
    elif cfg == 6:
        result = bench_res_block(spc, nat, wl, orc, coords, c_dev, dev, args, workload)
    elif cfg == 10:
        result = bench_io_blocks(spc, nat, wl, orc, coords, c_dev, dev, args, workload)
    elif cfg == 9:
        result = bench_feature_ops(spc, nat, wl, orc, coords, c_dev, dev, args, workload)
    elif cfg in (7, 8):
        result = bench_subdivide_block(spc, nat, wl, orc, coords, c_dev, dev, args, workload,
                                       cin, cout, res=64 if cfg == 7 else 128)
    else:
        keeps = wl.prune_masks(n)
        lv = []
        cc = c_dev
        for keep, ch in zip(keeps, (64, 32)):
            oc, par = nat.subdivide_map(cc, torch.from_numpy(keep).to(dev))
            res = 128 if ch == 64 else 256
            ml = nat.map_build(oc, mesh_resolution=res)
            nl = oc.shape[0]
            pl = int((ml.token_major < nl).sum().item())
            x, _ = bf16_dev(orc, wl.normal((nl, ch), 1.0, seed=400 + ch), dev)
            w, _ = bf16_dev(orc, wl.normal((ch, 27, ch), 0.02, seed=401 + ch), dev)
            y = torch.empty((nl, ch), dtype=torch.bfloat16, device=dev)
            call = ConvCall(nat, x, nat.pack_weights(w), None, y, ml.token_major, ntaps=27,
                            n_out=nl, layout=nat.IDX_TOKEN_MAJOR, plan=ml.plan())
            msl, _ = time_gpu(call, args.steps, args.warmup)
            tl = msl / 1e3
            byt = nl * ch * 2 * 2 + w.numel() * 2 + 108 * nl
            lv.append({"resolution": res, "n": nl, "pairs": pl, "c": ch, "ms": msl,
                       "mvoxel_s": nl / tl / 1e6, "tflops": 2.0 * pl * ch * ch / tl / 1e12,
                       "compulsory_gbs": byt / tl / 1e9})
            cc = oc
        result = {"metric": f"config 4: {workload}", "levels": lv, "dtype": "bf16"}
    print(json.dumps(result))


def bench_single_shell(nat, wl, orc, dev, args) -> dict:
    """The metric's named shape beside the batch: one 64^3 sphere shell
    (N = 21,766, 453,614 pairs), bf16 C = 128 -> 128, map and tile plan
    built once, the conv timed like the headline step."""
    import torch

    coords = wl.sphere_shell()
    n = coords.shape[0]
    m = nat.map_build(torch.from_numpy(coords).to(dev))
    pairs = m.pairs
    x, _ = bf16_dev(orc, wl.normal((n, 128), 1.0, seed=111), dev)
    w, _ = bf16_dev(orc, wl.normal((128, 27, 128), 0.02, seed=112), dev)
    b, _ = bf16_dev(orc, wl.normal((128,), 0.01, seed=113), dev)
    y = torch.empty((n, 128), dtype=torch.bfloat16, device=dev)
    call = ConvCall(nat, x, nat.pack_weights(w), b, y, m.token_major, ntaps=27, n_out=n,
                    layout=nat.IDX_TOKEN_MAJOR, plan=m.plan())
    # its own warm-up: with 84 CUs idle the clock climbs higher (2.15 GHz in
    # the loop) and takes longer to get there than the full-chip conv's
    warm = max(args.warmup, 500)
    ms, _ = time_gpu(call, args.steps, warm)
    tf = 2.0 * pairs * 128 * 128 / (ms / 1e3) / 1e12
    return {"workload": "subm3x3x3 bf16 C=128, one sphere shell r=24 in 64^3", "n_voxels": n,
            "pairs": pairs, "ms": ms, "mvoxel_s": n / (ms / 1e3) / 1e6, "tflops": tf,
            "pct_peak": 100.0 * tf / PEAK_BF16_TFLOPS, "steps": args.steps, "warmup": warm}


def bench_bridge(nat, wl, c_dev, dev, args) -> dict:
    """The drop-in spconv bridge (sam3d_spconv_f16_forward: f16, unpacked
    KRSC weights packed on every call, offset-major indices, no tile plan)
    on the headline rows and channels, beside the packed-weight f16 conv of
    the same data without and with a tile plan.  Outputs are compared bit
    for bit."""
    import torch

    n = c_dev.shape[0]
    m = nat.map_build(c_dev)
    x = torch.from_numpy(wl.normal((n, 128), 1.0, seed=121)).to(dev).half()
    w = torch.from_numpy(wl.normal((128, 27, 128), 0.02, seed=122)).to(dev).half()
    b = torch.from_numpy(wl.normal((128,), 0.01, seed=123)).to(dev).half()
    y_bridge = torch.empty((n, 128), dtype=torch.float16, device=dev)
    y_packed = torch.empty_like(y_bridge)
    y_plan = torch.empty_like(y_bridge)
    L = nat.lib()
    s = torch.cuda.current_stream().cuda_stream
    bargs = (s, x.data_ptr(), w.data_ptr(), b.data_ptr(), y_bridge.data_ptr(),
             m.offset_major.data_ptr(), m.mask_sorted.data_ptr(), m.argsort.data_ptr(), n, 128,
             128)

    def bridge():
        L.sam3d_spconv_f16_forward(*bargs)

    pw = nat.pack_weights(w)
    packed = ConvCall(nat, x, pw, b, y_packed, m.offset_major, ntaps=27, n_out=n,
                      layout=nat.IDX_OFFSET_MAJOR)
    planned = ConvCall(nat, x, pw, b, y_plan, m.token_major, ntaps=27, n_out=n,
                       layout=nat.IDX_TOKEN_MAJOR, plan=m.plan())
    ms_bridge, _ = time_gpu(bridge, args.steps, args.warmup)
    err = L.spc_last_error().decode(errors="replace")
    if err:
        raise RuntimeError(f"sam3d_spconv_f16_forward: {err}")
    ms_packed, _ = time_gpu(packed, args.steps, args.warmup)
    ms_plan, _ = time_gpu(planned, args.steps, args.warmup)
    # calls alternating between the fine rows and their stride-2 coarse rows
    # (the SLAT IO blocks' two levels): each level keeps its own tile plan
    d = nat.downsample_map(c_dev, int(c_dev[:, 0].max().item()) + 1, 64)
    mc = nat.map_build(d.coarse_coords)
    nc = d.nc
    xc = torch.from_numpy(wl.normal((nc, 128), 1.0, seed=124)).to(dev).half()
    yc = torch.empty((nc, 128), dtype=torch.float16, device=dev)
    cargs = (s, xc.data_ptr(), w.data_ptr(), b.data_ptr(), yc.data_ptr(),
             mc.offset_major.data_ptr(), mc.mask_sorted.data_ptr(), mc.argsort.data_ptr(), nc,
             128, 128)

    def coarse():
        L.sam3d_spconv_f16_forward(*cargs)

    def alternate():
        L.sam3d_spconv_f16_forward(*bargs)
        L.sam3d_spconv_f16_forward(*cargs)

    ms_coarse, _ = time_gpu(coarse, args.steps, args.warmup)
    ms_alt, _ = time_gpu(alternate, args.steps, args.warmup)
    err = L.spc_last_error().decode(errors="replace")
    if err:
        raise RuntimeError(f"sam3d_spconv_f16_forward: {err}")
    torch.cuda.synchronize()
    return {"workload": "sam3d_spconv_f16_forward, f16 C=128 -> 128 on the headline rows",
            "bridge_ms": ms_bridge, "packed_ms": ms_packed, "packed_plan_ms": ms_plan,
            "bridge_over_packed": ms_bridge / ms_packed,
            "bit_identical": bool(torch.equal(y_bridge, y_packed) and
                                  torch.equal(y_bridge, y_plan)),
            "coarse_rows": nc, "bridge_coarse_ms": ms_coarse,
            "alternating_fine_coarse_ms": ms_alt,
            "alternating_over_separate": ms_alt / (ms_bridge + ms_coarse)}


def bench_feature_ops(spc, nat, wl, orc, coords, c_dev, dev, args, workload) -> dict:
    """HBM rates of the non-GEMM kernels of the SLAT IO blocks on the config-2
    rows (bf16): the scatter-mean downsample (fine -> coarse; from the rows'
    coarse index with a sort, and from the map's children lists), the upsample
    gather (coarse -> fine), LayerNorm + SiLU, LayerNorm + modulation + SiLU
    and the GroupNorm pair.  Algorithmic bytes per launch: every input row
    read once and every output row written once (plus 4-byte row indices
    and counts); GB/s = bytes / kernel time."""
    import ctypes

    import torch

    n = coords.shape[0]
    d = nat.downsample_map(c_dev, 4, 64)
    nc = d.nc
    L = nat.lib()
    s = torch.cuda.current_stream().cuda_stream
    BF = nat.BF16
    p = lambda t: t.data_ptr()  # noqa: E731
    out = []

    def rec(name, fn, c_args, nbytes, **kw):
        def call():
            st = fn(*c_args)
            if st != 0:
                nat._check(name, st)
        ms, _ = time_gpu(call, args.steps, args.warmup)
        out.append({"op": name, "ms": ms, "bytes": nbytes, "gbs": nbytes / (ms / 1e3) / 1e9,
                    "pct_hbm": 100.0 * nbytes / (ms / 1e3) / 1e9 / PEAK_HBM_GBS, **kw})

    ws = torch.empty(L.spc_scatter_mean_workspace_bytes(n, nc), dtype=torch.uint8, device=dev)
    f2c, cnt, ch = d.fine_to_coarse.contiguous(), d.counts.contiguous(), d.children.contiguous()
    keep = []
    for c in (128, 1024):
        xf, _ = bf16_dev(orc, wl.normal((n, c), 1.0, seed=900 + c), dev)
        xc, _ = bf16_dev(orc, wl.normal((nc, c), 1.0, seed=901 + c), dev)
        yc = torch.empty((nc, c), dtype=torch.bfloat16, device=dev)
        yf = torch.empty((n, c), dtype=torch.bfloat16, device=dev)
        sc = torch.randn(4, c, device=dev).bfloat16().float()
        keep += [xf, xc, yc, yf, sc]
        rec(f"scatter_mean {n}->{nc} C={c}", L.spc_scatter_mean,
            (s, BF, p(xf), p(f2c), p(cnt), p(yc), c, n, nc, p(ws), ws.numel()),
            n * c * 2 + nc * c * 2 + 4 * n + 4 * nc, rows_in=n, rows_out=nc, channels=c)
        rec(f"children_mean {n}->{nc} C={c}", L.spc_children_mean,
            (s, BF, p(xf), p(ch), p(cnt), p(yc), c, n, nc),
            n * c * 2 + nc * c * 2 + 4 * 8 * nc + 4 * nc, rows_in=n, rows_out=nc, channels=c)
        rec(f"gather (upsample) {nc}->{n} C={c}", L.spc_gather_rows,
            (s, BF, p(xc), p(f2c), p(yf), n, nc, c), nc * c * 2 + n * c * 2 + 4 * n,
            rows_in=nc, rows_out=n, channels=c)
        rec(f"layernorm_silu N={n} C={c}", L.spc_layernorm_silu,
            (s, BF, p(xf), n, c, None, None, ctypes.c_float(1e-6), 1, p(yf)), 2 * n * c * 2,
            rows=n, channels=c)
        rec(f"layernorm_mod_silu N={n} C={c}", L.spc_layernorm_mod_silu,
            (s, BF, p(xf), n, c, ctypes.c_float(1e-6), p(sc), p(sc), p(c_dev), 4, p(yf)),
            2 * n * c * 2 + 4 * n * 4, rows=n, channels=c)
    xg, _ = bf16_dev(orc, wl.normal((n, 768), 1.0, seed=990), dev)
    yg = torch.empty_like(xg)
    offs = spc.sparse.batch_offsets(spc.sparse.SparseTensor(xg, c_dev)).contiguous()
    rows_max = int((offs[1:] - offs[:-1]).max().item())
    stt = torch.empty((4, 32, 2), dtype=torch.float32, device=dev)
    gws = torch.empty(max(8, L.spc_group_norm_workspace_bytes(4, rows_max, 32)),
                      dtype=torch.uint8, device=dev)
    rec(f"group_norm_stats N={n} C=768", L.spc_group_norm_stats,
        (s, BF, p(xg), 768, 32, p(offs), 4, rows_max, ctypes.c_float(1e-5), p(stt), p(gws),
         gws.numel()), n * 768 * 2, rows=n, channels=768)
    rec(f"group_norm_silu N={n} C=768", L.spc_group_norm_silu,
        (s, BF, p(xg), n, 768, 32, p(offs), 4, p(stt), None, None, 1, None, n, p(yg)),
        2 * n * 768 * 2, rows=n, channels=768)
    del keep
    return {"metric": f"config 9: {workload}", "dtype": "bf16", "ops": out,
            "config": {"workload": workload, "n_fine": n, "n_coarse": nc}}


def bench_res_block(spc, nat, wl, orc, coords, c_dev, dev, args, workload):
    """SparseResBlock3d forward on the fused kernels against the same block
    as separate kernels and torch elementwise ops (both with cached maps)."""
    import torch

    n = coords.shape[0]
    torch.manual_seed(0)
    blk = spc.blocks.SparseResBlock3d(128, 512, 128).to(dev)
    with torch.no_grad():
        for p in blk.conv2.parameters():
            p.normal_(0, 0.02)
    blk = blk.to(torch.bfloat16)
    blk.norm1.float()
    x, _ = bf16_dev(orc, wl.normal((n, 128), 1.0, seed=601), dev)
    xt = spc.sparse.SparseTensor(x, c_dev)
    emb = torch.randn(4, 512, device=dev).bfloat16()

    def fused():
        with torch.no_grad():
            return blk(xt, emb)

    def unfused():
        with torch.no_grad():
            emb_out = blk.emb_layers(emb).type(x.dtype)
            scale, shift = torch.chunk(emb_out, 2, dim=1)
            h = xt.replace(nat.layernorm_silu(xt.feats, blk.norm1.weight, blk.norm1.bias))
            h = blk.conv1(h)
            h = h.replace(nat.layernorm_silu(h.feats, silu=False))
            h = h * (1 + scale) + shift
            h = h.replace(torch.nn.functional.silu(h.feats))
            h = blk.conv2(h)
            return h + xt

    ms_f, _ = time_gpu(fused, args.steps, args.warmup)
    ms_u = diff = None
    if not args.fused_only:
        ms_u, _ = time_gpu(unfused, args.steps, args.warmup)
        diff = float((fused().feats.float() - unfused().feats.float()).abs().max())
    return {"metric": f"config 6: {workload}", "value": n / (ms_f / 1e3) / 1e6, "unit": "Mvoxel/s",
            "ms_per_step": ms_f, "unfused_ms": ms_u, "speedup": ms_u / ms_f if ms_u else None,
            "dtype": "bf16", "max_abs_diff_fused_vs_unfused": diff,
            "config": {"workload": workload, "n_voxels": n, "channels": 128, "batch": 4}}


def bench_io_blocks(spc, nat, wl, orc, coords, c_dev, dev, args, workload):
    """The SLAT flow model's IO residual blocks at their real widths
    (structured_latent_flow.py:50-74, 140-200): the input block
    SparseResBlock3d(128, 1024, 1024, downsample=True) -- scatter-mean
    downsample of the 62,710 fine rows to 11,774 coarse rows, LayerNorm32 +
    SiLU, conv 128 -> 1024, the norm2 / modulation / SiLU row pass, conv
    1024 -> 1024 + the 128 -> 1024 skip -- and the output block
    SparseResBlock3d(2048, 1024, 128, upsample=True) -- the coarse -> fine
    gather, conv 2048 -> 128 with the fused norm epilogue, conv 128 -> 128 +
    the 2048 -> 128 skip.  Maps are cached in the tensors' spatial caches
    (built once, as in a sampling loop); the time is the block forward."""
    import torch

    sp = spc.sparse
    n = coords.shape[0]
    out = {}
    for mode, cin, cout in (("down", 128, 1024), ("up", 2048, 128)):
        torch.manual_seed(7 + cin)
        blk = spc.blocks.SparseResBlock3d(cin, 1024, cout, downsample=mode == "down",
                                          upsample=mode == "up").to(dev)
        with torch.no_grad():
            for prm in blk.conv2.parameters():
                prm.normal_(0, 0.02)
        blk = blk.to(torch.bfloat16)
        blk.norm1.float()
        if mode == "down":
            x, _ = bf16_dev(orc, wl.normal((n, cin), 1.0, seed=1001), dev)
            xt = sp.SparseTensor(x, c_dev)
        else:
            ft = sp.SparseTensor(torch.zeros((n, 32), dtype=torch.bfloat16, device=dev), c_dev)
            ct = sp.SparseDownsample(2)(ft)
            x, _ = bf16_dev(orc, wl.normal((ct.coords.shape[0], cin), 1.0, seed=1002), dev)
            xt = ct.replace(x)
        emb = torch.randn(4, 1024, device=dev).bfloat16()

        def fwd():
            with torch.no_grad():
                return blk(xt, emb)

        y = fwd()  # builds and caches the maps and plans
        ms, _ = time_gpu(fwd, args.steps, args.warmup)
        n_in, n_out = xt.feats.shape[0], y.feats.shape[0]
        flops = 0.0
        for conv, rows, ci, co in ((blk.conv1, n_out, cin, cout), (blk.conv2, n_out, cout, cout)):
            flops += 2.0 * ci * co * rows * 27  # dense-equivalent (tap padding included)
        out[mode] = {"block": f"SparseResBlock3d({cin} -> {cout}, {mode}sample)", "rows_in": n_in,
                     "rows_out": n_out, "ms": ms, "mvoxel_s": n_out / (ms / 1e3) / 1e6,
                     "dense_equiv_tflops": flops / (ms / 1e3) / 1e12}
    return {"metric": f"config 10: {workload}", "dtype": "bf16", "blocks": out,
            "config": {"workload": workload, "n_fine": n,
                       "n_coarse": out["down"]["rows_out"]}}


def bench_subdivide_block(spc, nat, wl, orc, coords, c_dev, dev, args, workload, cin, cout, res):
    """SparseSubdivideBlock3d forward (768 -> 192 or 192 -> 96, the mesh
    decoder's upsample blocks) on the fused path against the same block with
    separate GroupNorm, SiLU, gather and residual passes.  Both include the
    child map build, as the block builds it on every call."""
    import torch

    sp = spc.sparse
    n = coords.shape[0]
    torch.manual_seed(0)
    blk = spc.blocks.SparseSubdivideBlock3d(cin, res, cout).to(dev)
    with torch.no_grad():
        for p in blk.out_layers[3].parameters():
            p.normal_(0, 0.02)
    blk = blk.to(torch.bfloat16)
    blk.act_layers[0].float()
    blk.out_layers[1].float()
    x, _ = bf16_dev(orc, wl.normal((n, cin), 1.0, seed=701), dev)
    xt = sp.SparseTensor(x, c_dev)
    gn0, gn1 = blk.act_layers[0], blk.out_layers[1]

    def fused():
        with torch.no_grad():
            return blk(xt)

    def unfused():
        with torch.no_grad():
            coords, parent = blk.sub.map(xt)
            h = nat.group_norm_silu(xt.feats, sp.batch_offsets(xt), 32, gn0.weight, gn0.bias,
                                    gn0.eps, silu=False)
            h = torch.nn.functional.silu(h)
            h = blk.sub.assemble(xt, coords, nat.gather_rows(h, parent))
            xs = blk.sub.assemble(xt, coords, nat.gather_rows(xt.feats, parent))
            h = blk.out_layers[0](h)
            h = h.replace(torch.nn.functional.silu(nat.group_norm_silu(
                h.feats, sp.batch_offsets(h), 32, gn1.weight, gn1.bias, gn1.eps, silu=False)))
            h = blk.out_layers[3](h)
            return h + blk.skip_connection(xs)

    ms_f, _ = time_gpu(fused, args.steps, args.warmup)
    yf = fused()
    nc = yf.feats.shape[0]
    ms_u = diff = None
    if not args.fused_only:
        ms_u, _ = time_gpu(unfused, args.steps, args.warmup)
        diff = float((yf.feats.float() - unfused().feats.float()).abs().max())
    return {"metric": f"config {args.config}: {workload}", "value": nc / (ms_f / 1e3) / 1e6,
            "unit": "Mvoxel/s",
            "ms_per_step": ms_f, "unfused_ms": ms_u, "speedup": ms_u / ms_f if ms_u else None,
            "dtype": "bf16", "max_abs_diff_fused_vs_unfused": diff,
            "config": {"workload": workload, "n_parents": n, "n_children": nc, "cin": cin,
                       "cout": cout}}


if __name__ == "__main__":
    main()
