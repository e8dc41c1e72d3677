"""Benchmark: config 3 sparse residual block on one MI355X.

Workload: 256^3 grid, 1,040,679 active voxels (shell
of a seeded union of 8 ellipsoids), C = 128, bf16 activations and weights
with f32 accumulation.  One step = neighbour-map build for the coords + conv
plan build (row order and per-tile halo tables of the map) + conv3x3x3 ->
LayerNorm -> SiLU (fused into the first conv's epilogue) -> conv3x3x3 -> + x
(fused into the second conv's epilogue), both convs halo-staged.  Inputs are
resident in HBM before timing; the weights are packed once beforehand (layer
constants, as the reference's decoder caches its weights per layer).

Prints one JSON line: value = voxels/s of the whole step (W untimed steps,
then K steps timed with HIP events, no host work in between); roofline = the
dominant kernel (the MFMA conv) at its useful FLOPs 2*P*Cin*Cout per launch
(P = valid (row, offset) pairs) over its mean launch duration, measured with
HIP events on the launch stream between the parts of K further steps;
cpu_baseline = the oracle's restatement of the reference CPU flex path
(HashMap map + im2col + single-thread sgemm) timed on this host over a
bounded sample of query rows.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "sparse-conv voxels/s + TFLOP/s (% bf16 MFMA peak), 256^3 grid ~1M voxels C=128"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0      # MI355X HBM3E


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=25,
                    help="untimed steps right before the timed ones (the GPU's clocks need ~20 steps)")
    ap.add_argument("--cpu-sample", type=int, default=262144,
                    help="query rows of the CPU baseline sample (0 = skip)")
    ap.add_argument("--only", choices=["map", "plan", "mapplan", "conv", "ln", "config5", "map_shuffled",
                                       "map_spread", "conv_f16"], default=None,
                    help="run just this part of the step (or config 5's decoder stack) --steps times "
                         "(for rocprofv3) and exit")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the config 2 / 4 / 5 component timings")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one 1 GiB device-to-device copy (the known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


def queued_ms(fn, iters, warmup=2):
    """GPU time per call of `fn` with the host's per-call cost taken out:
    the calls are enqueued behind a ~2 ms spin kernel (torch.cuda._sleep), so
    by the time the start event is reached every call is already queued and
    the GPU runs them back to back.  For calls whose kernels take less time
    than the host needs to issue them (small inputs, Python in the loop)."""
    import torch
    for _ in range(warmup):
        fn()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    torch.cuda._sleep(5_000_000)
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / iters


def events_ms(fn, iters, warmup=0):
    import torch
    for _ in range(warmup):
        fn()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / iters


def host_cpu():
    """(CPU model, cores this process may run on, threads for the all-cores
    baseline: those cores, capped by OMP_NUM_THREADS when set)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    cores = len(os.sched_getaffinity(0))
    threads = cores
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = max(1, min(cores, int(os.environ["OMP_NUM_THREADS"])))
    return model, cores, threads


def _config3_cpu_step(O, coords, x_f32, w1, w2, sample_rows, threads):
    """Seconds for the map over all coords and for the block over the first
    `sample_rows` query rows, with the flex conv (im2col gather + packed FMA
    sgemm, oracle/sc_fastgemm.c) on `threads` threads."""
    import numpy as np
    O.set_num_threads(threads)
    cfg = O.OracleConfig(128, 128)
    b = np.zeros(128, np.float32)
    t0 = time.perf_counter()
    nbr = O.build_neighbor_rows(cfg, coords, lowest_row_on_duplicate=False)
    t_map = time.perf_counter() - t0
    rows = np.arange(sample_rows)
    t0 = time.perf_counter()
    h = O.conv_flex_fast(cfg, w1, b, x_f32, nbr[rows], threads=threads)
    h = O.silu(O.layer_norm(h, None, None, 1e-6))
    # conv2 reads conv1 output at neighbour rows; the sample's own rows stand in
    # for the rest of the input (same work per row).
    h_full = np.zeros_like(x_f32)
    h_full[rows] = h
    y = O.conv_flex_fast(cfg, w2, b, h_full, nbr[rows], threads=threads) + x_f32[rows]
    t_rest = time.perf_counter() - t0
    assert y.shape == (sample_rows, 128)
    O.set_num_threads(1)
    return t_map, t_rest


def _reference_bench_shape(O, reps=7):
    """The reference's own CPU bench (crates/burn_flex_gmm/benches/
    sparse_subm_conv.rs:37-74: 4,096 line coords [0, x, 0, 0], 3x3x3, Cin 64 ->
    Cout 128, f32, LCG inputs), one thread, median of `reps`: the flex path
    (map + pack + im2col + sgemm) with the packed FMA sgemm and with the
    oracle's separately rounded loop, and the legacy direct loop; beside the
    published ~22.5 ms (flex) and ~44.1 ms (legacy), whose hardware is not
    stated (docs/trellis2_gpu_efficiency_roadmap.md:10-13)."""
    import numpy as np
    cfg = O.OracleConfig(64, 128)
    coords = np.zeros((4096, 4), np.int32)
    coords[:, 1] = np.arange(4096)
    vals = O.Lcg(7).next_f32(4096 * 64 + 128 * 27 * 64 + 128)  # input, weight, bias in the bench's order
    x = vals[:4096 * 64].reshape(4096, 64)
    w = vals[4096 * 64:4096 * 64 + 128 * 27 * 64].reshape(128, 27, 64)
    b = vals[4096 * 64 + 128 * 27 * 64:]
    O.set_num_threads(1)

    def med(fn):
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return 1e3 * sorted(ts)[reps // 2]

    def flex_fast():
        nbr = O.build_neighbor_rows(cfg, coords, lowest_row_on_duplicate=False)
        return O.conv_flex_fast(cfg, w, b, x, nbr, threads=1)

    ms_fast = med(flex_fast)
    ms_oracle = med(lambda: O.conv_flex(cfg, w, b, coords, x))
    ms_legacy = med(lambda: O.conv_legacy(cfg, w, b, coords, x))
    issued = 2.0 * 4096 * 27 * 64 * 128
    return {"shape": "4,096 line coords, 3x3x3, Cin 64 -> Cout 128, f32, 1 thread "
                     "(crates/burn_flex_gmm/benches/sparse_subm_conv.rs:37-74)",
            "flex_ms": ms_fast, "flex_issued_gflops": issued / (ms_fast * 1e-3) / 1e9,
            "flex_oracle_loop_ms": ms_oracle, "legacy_ms": ms_legacy,
            "published_flex_ms": 22.5, "published_legacy_ms": 44.1,
            "note": "flex_ms: packed FMA sgemm (the kind matrixmultiply 0.3.10 runs); flex_oracle_loop_ms: the "
                    "parity oracle's separately rounded loop; published figures from the reference's docs, "
                    "hardware not stated"}


def cpu_baseline(coords, x_f32, w1, w2, sample_rows):
    """The reference CPU path (burn_flex_gmm flex: build_neighbor_rows with a
    HashMap, im2col gather + sgemm) restated in C (oracle/), timed on this
    host: the config-3 step -- map over all N coords, conv1 / LN / SiLU /
    conv2 / + x over `sample_rows` query rows, voxels/s = 1 / (t_map / N +
    t_rest / sample) -- on 1 thread (the reference's matrixmultiply is
    single-threaded: the headline baseline) and on all the host's cores
    (OpenMP over row blocks); and config 1 (64^3 sphere shell, 14,648
    voxels, C = 64, f32: map + conv over every row) on both."""
    import numpy as np
    from bevy_synth_amd import synth
    from oracle import oracle as O
    O.build()
    model, cores, threads = host_cpu()
    n = len(coords)
    ref_shape = _reference_bench_shape(O)
    t_map1, t_rest1 = _config3_cpu_step(O, coords, x_f32, w1, w2, sample_rows, 1)
    t_mapn, t_restn = _config3_cpu_step(O, coords, x_f32, w1, w2, sample_rows, threads)
    # config 1, every row
    c1 = synth.config1_coords()
    rng = np.random.default_rng(1)
    x1 = rng.standard_normal((len(c1), 64)).astype(np.float32)
    wc1 = (rng.standard_normal((64, 27, 64)) / np.sqrt(27 * 64)).astype(np.float32)
    cfg1 = O.OracleConfig(64, 64)
    cfg1_res = {}
    for t in (1, threads):
        O.set_num_threads(t)
        t0 = time.perf_counter()
        nb1 = O.build_neighbor_rows(cfg1, c1, lowest_row_on_duplicate=False)
        y1 = O.conv_flex_fast(cfg1, wc1, np.zeros(64, np.float32), x1, nb1, threads=t)
        dt = time.perf_counter() - t0
        assert y1.shape == (len(c1), 64)
        pairs = int((nb1 >= 0).sum())
        cfg1_res[t] = {"voxels_per_s": len(c1) / dt, "seconds": dt, "useful_gflops": 2.0 * pairs * 64 * 64 / dt / 1e9,
                       "cores": t}
    O.set_num_threads(1)
    return {
        "value": 1.0 / (t_map1 / n + t_rest1 / sample_rows),
        "unit": "voxels/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"config 3 step: map build over all {n} coords ({t_map1:.2f} s) + conv/LN/SiLU/"
                   f"conv/add over the first {sample_rows} query rows ({t_rest1:.2f} s), f32, 1 thread; "
                   f"map and LN/SiLU from oracle/sc_oracle.c, flex conv = its im2col gather + a packed FMA "
                   f"sgemm (oracle/sc_fastgemm.c), restating crates/burn_flex_gmm/src/lib.rs:69-109,242-375"),
        "reference_bench_shape": ref_shape,
        "host": {"cpu_model": model, "cores_available": cores},
        "all_cores": {"value": 1.0 / (t_mapn / n + t_restn / sample_rows), "unit": "voxels/s", "cores": threads,
                      "sample": f"same step; flex conv on {threads} OpenMP threads over row blocks "
                                f"(map {t_mapn:.2f} s, block {t_restn:.2f} s)"},
        "config1": {"voxels": len(c1), "one_thread": cfg1_res[1], "all_cores": cfg1_res[threads],
                    "sample": "config 1 (64^3 sphere shell r=24, C=64, f32): map + flex conv over every row"},
    }


def config5_stack(dev, rng):
    """Config 5's int8 decoder stack (3 stages of 2 residual blocks + fused
    C2S upsample, 512 -> 64 channels) on synthetic bf16 features.  Returns
    (run, res, start voxels): run() executes the stack once and leaves the
    children's neighbourhood and features in res["nb"], res["y"]."""
    import numpy as np
    import torch

    from bevy_synth_amd import decoder as D
    from bevy_synth_amd import synth

    coords5, masks = synth.config5_stack_inputs()
    stack = D.int8_stack([512, 256, 128, 64], 2, seed=5, device=dev)
    x5 = torch.from_numpy(synth.bf16_bits(synth.normal_f32(rng, (len(coords5), 512))).view(np.int16)) \
        .to(dev).view(torch.bfloat16)
    c5 = torch.from_numpy(coords5).to(dev)
    m5 = [torch.from_numpy(m).to(dev) for m in masks]
    res = {}

    def run():
        res["nb"], res["y"] = stack(c5, x5, m5)
    return run, res, len(coords5)


def config_components(dev, st=None, steps: int = 5):
    """The other BASELINE configs on this GPU, for the record (parity cases,
    not the headline): config 2's planned 3x3x3 conv (C = 256, bf16), config
    4's 2x2x2 transposed upsample (a 1x1x1 conv with the child scatter) then
    the children's map + plan + 3x3x3 conv (C = 256), and config 5's int8
    decoder stack (3 stages of 2 residual blocks + fused C2S upsample,
    512 -> 64 channels); the neighbour map in its other table modes; the C2S
    compaction of config 4's parents; a ConvNeXt block at config 2's shape;
    and config 3's conv in f16 (st: the config-3 step, whose map and plan
    it reuses).  ms per call, after one untimed call."""
    import numpy as np
    import torch

    from bevy_synth_amd import decoder as D
    from bevy_synth_amd import flex_gmm as F
    from bevy_synth_amd import synth

    def bf(a):
        return torch.from_numpy(synth.bf16_bits(a).view(np.int16)).to(dev).view(torch.bfloat16)

    def wall_ms(fn, n):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / n

    out = {}
    rng = np.random.default_rng(7)
    # config 2
    c2 = synth.config2_coords()
    C = 256
    cfg = F.SparseSubmConvConfig(C, C)
    nb = D.Neighborhood.build(cfg, torch.from_numpy(c2).to(dev))
    layer = D.ConvLayer(cfg, bf(synth.conv_weight(rng, C, 27, C, 1 / np.sqrt(27 * C))),
                        torch.zeros(C, dtype=torch.float32, device=dev))
    x2 = bf(synth.normal_f32(rng, (len(c2), C)))
    P2 = int((nb.nbr >= 0).sum().item())
    ms = events_ms(lambda: layer(x2, nb), steps, 2)
    out["config2"] = {"voxels": len(c2), "pairs": P2, "conv_ms": ms,
                      "conv_useful_tflops": 2.0 * P2 * C * C / (ms * 1e-3) / 1e12,
                      "map_plus_plan_ms": wall_ms(lambda: D.Neighborhood.build(cfg, nb.coords), steps)}
    # config 4
    g = synth.ShellCubeGeometry()
    parents = g.coords()
    mask = torch.from_numpy(synth.subdivision_mask_near_surface(parents, g)).to(dev)
    pc = torch.from_numpy(parents).to(dev)
    cin, cout = 512, 256
    tl = D.ConvLayer(F.SparseSubmConvConfig(cin, 8 * cout, 1, 1, 1),
                     bf(synth.normal_f32(rng, (8 * cout, 1, cin), 1 / np.sqrt(8 * cin))),
                     torch.zeros(8 * cout, dtype=torch.float32, device=dev))
    xp = bf(synth.normal_f32(rng, (len(parents), cin)))
    ccfg = F.SparseSubmConvConfig(cout, cout)
    cl = D.ConvLayer(ccfg, bf(synth.conv_weight(rng, cout, 27, cout, 1 / np.sqrt(27 * cout))),
                     torch.zeros(cout, dtype=torch.float32, device=dev))
    cc, feats, _ = D.transposed_upsample(pc, xp, tl, mask)
    cnb = D.Neighborhood.build(ccfg, cc)
    P4 = int((cnb.nbr >= 0).sum().item())
    t_up = wall_ms(lambda: D.transposed_upsample(pc, xp, tl, mask), steps)
    t_conv = events_ms(lambda: cl(feats, cnb), steps, 2)
    out["config4"] = {"parents": len(parents), "children": int(cc.shape[0]), "child_pairs": P4,
                      "transposed_upsample_ms": t_up,
                      "child_map_plus_plan_ms": wall_ms(lambda: D.Neighborhood.build(ccfg, cc), steps),
                      "conv_ms": t_conv, "conv_useful_tflops": 2.0 * P4 * cout * cout / (t_conv * 1e-3) / 1e12}
    # config 5
    run5, res, n5 = config5_stack(dev, rng)
    run5()  # a second untimed stack: the first builds the allocator's cache for every size
    t5 = wall_ms(run5, max(4, steps))
    out["config5"] = {"start_voxels": n5, "end_voxels": int(res["y"].shape[0]), "stack_ms": t5,
                      "note": "18 convs (int8 weights, bf16 activations), 4 maps + plans, fused C2S upsamples; "
                              "includes the host syncs of the child counts"}
    del run5, res

    # C2S compaction (sc_subdivision_build_indexed) of config 4's parents:
    # HBM-bound; algorithmic bytes = mask + parent coords read, child coords,
    # linear_idx and the [P, 8] child-row table written
    A = int(cc.shape[0])
    P = len(parents)
    mask_u8 = mask.to(torch.uint8).contiguous()
    sbuf = F.SubdivisionBuffers(P, dev)
    ms_sub = events_ms(lambda: F.subdivision_launch(pc, mask=mask_u8, buffers=sbuf), steps, 2)
    ms_call = events_ms(lambda: F.subdivision_build_indexed(pc, mask=mask_u8), steps, 2)
    sub_bytes = P * 8 + P * 16 + A * (16 + 4) + P * 32
    # the same call over the first 256 parents (the per-call floor)
    pc_t, mask_t = pc[:256].contiguous(), mask_u8[:256].contiguous()
    sbuf_t = F.SubdivisionBuffers(256, dev)
    ms_sub_floor = events_ms(lambda: F.subdivision_launch(pc_t, mask=mask_t, buffers=sbuf_t), steps, 2)
    # the same two launches with the calls queued ahead of the GPU
    ms_sub_gpu = queued_ms(lambda: F.subdivision_launch(pc, mask=mask_u8, buffers=sbuf), steps)
    ms_sub_floor_gpu = queued_ms(lambda: F.subdivision_launch(pc_t, mask=mask_t, buffers=sbuf_t), steps)
    out["c2s_compaction"] = {"parents": P, "children": A, "ms": ms_sub,
                             "gbps": sub_bytes / (ms_sub * 1e-3) / 1e9,
                             "frac_hbm": sub_bytes / (ms_sub * 1e-3) / 8e12,
                             "ms_256_parents": ms_sub_floor,
                             "gpu_ms": ms_sub_gpu, "gpu_ms_256_parents": ms_sub_floor_gpu,
                             "gpu_gbps": sub_bytes / (ms_sub_gpu * 1e-3) / 1e9,
                             "gpu_frac_hbm": sub_bytes / (ms_sub_gpu * 1e-3) / 8e12,
                             "call_ms": ms_call,
                             "note": "ms: the two launches back to back, buffers preallocated (events); ms_256_parents: the "
                                     "same call on 256 parents; gpu_ms: the calls queued behind a spin kernel, so the "
                                     "host's per-call cost is taken out; "
                                     "call_ms: the Python call, which allocates and reads the child count back"}

    # ConvNeXt block (conv -> LN(affine) -> mlp_0 -> SiLU -> mlp_2 + x) at
    # config 2's shape, C = 256, hidden 4C, bf16
    C, H = 256, 1024
    blk = D.ConvNeXtBlock(
        D.ConvLayer(F.SparseSubmConvConfig(C, C), bf(synth.conv_weight(rng, C, 27, C, 1 / np.sqrt(27 * C))),
                    torch.zeros(C, dtype=torch.float32, device=dev)),
        torch.ones(C, dtype=torch.float32, device=dev), torch.zeros(C, dtype=torch.float32, device=dev),
        D.LinearLayer(bf(synth.normal_f32(rng, (H, C), 1 / np.sqrt(C))), torch.zeros(H, dtype=torch.float32,
                                                                                    device=dev)),
        D.LinearLayer(bf(synth.normal_f32(rng, (C, H), 1 / np.sqrt(H))), torch.zeros(C, dtype=torch.float32,
                                                                                    device=dev)))
    ms_cn = events_ms(lambda: blk(x2, nb), steps, 2)
    fl_cn = 2.0 * P2 * C * C + 2 * 2.0 * len(c2) * C * H
    out["convnext_block"] = {"voxels": len(c2), "channels": C, "hidden": H, "ms": ms_cn,
                             "useful_tflops": fl_cn / (ms_cn * 1e-3) / 1e12}

    # config 3's conv (-> LN -> SiLU, planned) in f16 on the step's map and plan
    if st is not None:
        x16 = st.x.to(torch.float16)
        w16 = st.w1_d.to(torch.float16)
        wp16 = F.pack_conv_weight(st.cfg, w16)
        h16 = torch.empty_like(x16)
        P3 = int((st.nbr >= 0).sum().item())

        def conv_f16():
            F.sparse_subm_conv_forward(st.cfg, x16, st.nbr, w16, st.bias, out=h16, layer_norm=True, ln_eps=1e-6,
                                       silu=True, plan=st.plan, packed_weight=wp16)
        # the f16 and the bf16 conv interleaved, each call between its own
        # events, medians: the clock ramps under sustained MFMA load, so timing
        # one precision after the other favours the second
        for _ in range(5):
            conv_f16()
            st.conv1()
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(max(steps, 5))]
        for e0, e1, e2 in ev:
            e0.record()
            conv_f16()
            e1.record()
            st.conv1()
            e2.record()
        torch.cuda.synchronize()
        ms16 = float(np.median([e0.elapsed_time(e1) for e0, e1, _ in ev]))
        ms_bf = float(np.median([e1.elapsed_time(e2) for _, e1, e2 in ev]))
        out["config3_f16_conv"] = {"ms": ms16, "useful_tflops": 2.0 * P3 * st.C * st.C / (ms16 * 1e-3) / 1e12,
                                   "frac_of_fp16_peak": 2.0 * P3 * st.C * st.C / (ms16 * 1e-3) / 1e12 /
                                   PEAK_BF16_TFLOPS, "bf16_ms_same_protocol": ms_bf,
                                   "note": "conv -> LN -> SiLU, planned, outside the step; f16 and bf16 calls "
                                           "interleaved, medians of per-call events"}

    # The neighbour map in its other table modes: config 3's coords shuffled
    # (unsorted rows: the dense grid), spread over a wide box (the hash
    # table) and config 5's last C2S child set (C2S order below a sorted root
    # set: the rank bitmap over octree levels).
    def map_mode(coords_np, what):
        cd = torch.from_numpy(np.ascontiguousarray(coords_np)).to(dev)
        n = len(coords_np)
        mcfg = F.SparseSubmConvConfig(64, 64)
        nbr = torch.empty((n, 27), dtype=torch.int32, device=dev)
        ws = F.NeighborMapWorkspace(dev).get(n)
        ms = events_ms(lambda: F.neighbor_map_build_into(mcfg, cd, nbr, ws), steps, 2)
        F.neighbor_map_check(ws)
        gbps = (n * 16 + n * 27 * 4) / (ms * 1e-3) / 1e9
        return {"coords": what, "voxels": n, "table": F.neighbor_map_table_mode(ws), "map_build_ms": ms,
                "gbps": gbps, "frac_hbm": gbps / PEAK_HBM_GBPS}
    c3 = synth.config3_coords()
    shuffled = c3[np.random.default_rng(11).permutation(len(c3))]
    children, masks5 = synth.config5_stack_inputs()
    for m in masks5:
        children = synth.child_expand(children, m)
    out["map_modes"] = {"config3_shuffled": map_mode(shuffled, "config 3 coords in a random row order"),
                        "config3_spread": map_mode(synth.config3_spread_coords(),
                                                   "config 3's octants 1024 cells apart in x, random row "
                                                   "order (bbox beyond the dense grid)"),
                        "config5_children": map_mode(children, "config 5's last child set (C2S order)")}
    return out


class Config3Step:
    """The timed step of config 3 and its buffers: neighbour map + conv plan
    + conv3x3x3 -> LayerNorm -> SiLU (fused) -> conv3x3x3 -> + x (fused), bf16
    with f32 accumulation, weights packed once.  tests/test_gpu_bench_step.py
    runs this same object and checks its output against the oracle."""

    def __init__(self, dev, seed: int = 2026):
        import numpy as np
        import torch

        from bevy_synth_amd import flex_gmm as F
        from bevy_synth_amd import synth

        self.coords = coords = synth.config3_coords()
        self.n = n = len(coords)
        self.C = C = 128
        rng = np.random.default_rng(seed)
        self.x_f32 = synth.bf16_to_f32(synth.bf16_bits(synth.normal_f32(rng, (n, C))))
        std = 1.0 / np.sqrt(27 * C)
        self.w1 = synth.bf16_to_f32(synth.bf16_bits(synth.conv_weight(rng, C, 27, C, std)))
        self.w2 = synth.bf16_to_f32(synth.bf16_bits(synth.conv_weight(rng, C, 27, C, std)))

        def to_bf16(a):
            return torch.from_numpy(synth.bf16_bits(a).view(np.int16)).to(dev).view(torch.bfloat16)

        self.coords_d = torch.from_numpy(coords).to(dev)
        self.x = to_bf16(self.x_f32)
        self.w1_d, self.w2_d = to_bf16(self.w1), to_bf16(self.w2)
        self.bias = torch.zeros(C, dtype=torch.float32, device=dev)
        self.cfg = cfg = F.SparseSubmConvConfig(C, C)
        self.nbr = torch.empty((n, 27), dtype=torch.int32, device=dev)
        self.ws = F.NeighborMapWorkspace(dev).get(n)
        self.plan_buf = torch.empty(F.conv_plan_bytes(n, 27), dtype=torch.uint8, device=dev)
        self.h = torch.empty((n, C), dtype=torch.bfloat16, device=dev)
        self.out = torch.empty((n, C), dtype=torch.bfloat16, device=dev)
        self.w1_p, self.w2_p = F.pack_conv_weight(cfg, self.w1_d), F.pack_conv_weight(cfg, self.w2_d)
        self.plan = F.ConvPlan(self.plan_buf, n, n, 27)
        self.F = F

    def map_build(self):
        self.F.neighbor_map_build_into(self.cfg, self.coords_d, self.nbr, self.ws)

    def plan_build(self):
        self.F.conv_plan_build_into(self.cfg, self.coords_d, self.nbr, self.plan_buf)

    def map_and_plan(self):
        self.map_build()
        self.plan_build()

    def conv1(self):  # conv -> LayerNorm -> SiLU, fused in the conv epilogue
        self.F.sparse_subm_conv_forward(self.cfg, self.x, self.nbr, self.w1_d, self.bias, out=self.h,
                                        layer_norm=True, ln_eps=1e-6, silu=True, plan=self.plan,
                                        packed_weight=self.w1_p)

    def ln_silu(self):  # the unfused LayerNorm + SiLU kernel, timed for reference only
        self.F.layer_norm(self.h, eps=1e-6, silu=True, out=self.h)

    def conv2(self):  # conv -> + x, fused
        self.F.sparse_subm_conv_forward(self.cfg, self.h, self.nbr, self.w2_d, self.bias, residual=self.x,
                                        out=self.out, plan=self.plan, packed_weight=self.w2_p)

    def step(self):
        self.map_build()
        self.plan_build()
        self.conv1()
        self.conv2()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the sparse-conv path shards by spatial slab with a halo exchange, not built here)",
              file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    from bevy_synth_amd import flex_gmm as F
    from bevy_synth_amd import synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.only == "config5":
        run5, _, _ = config5_stack(dev, np.random.default_rng(7))
        for _ in range(max(args.warmup, 1)):
            run5()
        ms = events_ms(run5, args.steps)
        print(f"[bench] only=config5 {ms:.3f} ms per call", file=sys.stderr, flush=True)
        return
    if args.only in ("map_shuffled", "map_spread"):
        # the map alone in its dense-grid / hash-table mode (for rocprofv3)
        c3 = synth.config3_coords()
        cm = (c3[np.random.default_rng(11).permutation(len(c3))] if args.only == "map_shuffled"
              else synth.config3_spread_coords())
        cd = torch.from_numpy(np.ascontiguousarray(cm)).to(dev)
        mcfg = F.SparseSubmConvConfig(64, 64)
        nbr_m = torch.empty((len(cm), 27), dtype=torch.int32, device=dev)
        ws_m = F.NeighborMapWorkspace(dev).get(len(cm))
        part = lambda: F.neighbor_map_build_into(mcfg, cd, nbr_m, ws_m)
        for _ in range(max(args.warmup, 1)):
            part()
        ms = events_ms(part, args.steps)
        F.neighbor_map_check(ws_m)
        print(f"[bench] only={args.only} table={F.neighbor_map_table_mode(ws_m)} {ms:.3f} ms per call",
              file=sys.stderr, flush=True)
        return
    st = Config3Step(dev)
    n, C, coords, x_f32, w1, w2 = st.n, st.C, st.coords, st.x_f32, st.w1, st.w2
    nbr, ws, h, out = st.nbr, st.ws, st.h, st.out
    map_build, plan_build, map_and_plan = st.map_build, st.plan_build, st.map_and_plan
    conv1, conv2, ln_silu, step = st.conv1, st.conv2, st.ln_silu, st.step

    # One untimed step, then everything that needs the host (the map status
    # check, the pair count, the calibration copy), so that the W warmup
    # steps lead straight into the K timed steps: a host-side gap between them
    # idles the GPU, its clocks drop, and the first timed steps run ~7 % slow.
    step()
    F.neighbor_map_check(ws)
    P = int((nbr >= 0).sum().item())
    if args.calibrate_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        src.fill_(1)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.only == "conv_f16":
        # conv -> LN -> SiLU in f16 and in bf16, alternately (the f16-vs-bf16
        # clock comparison: rocprofv3 --pmc GRBM_GUI_ACTIVE --kernel-trace)
        x16, w16 = st.x.to(torch.float16), st.w1_d.to(torch.float16)
        wp16, h16 = F.pack_conv_weight(st.cfg, w16), torch.empty_like(st.x, dtype=torch.float16)

        def conv1_f16():
            F.sparse_subm_conv_forward(st.cfg, x16, st.nbr, w16, st.bias, out=h16, layer_norm=True, ln_eps=1e-6,
                                       silu=True, plan=st.plan, packed_weight=wp16)
        part = lambda: (conv1_f16(), conv1())
    elif args.only:
        part = {"map": map_build, "plan": plan_build, "mapplan": map_and_plan,
                "conv": lambda: (conv1(), conv2()), "ln": ln_silu}[args.only]
    if args.only:
        for _ in range(max(args.warmup, 1)):
            part()
        ms = events_ms(part, args.steps)
        print(f"[bench] only={args.only} {ms:.3f} ms per call", file=sys.stderr, flush=True)
        return
    print(f"[bench] config3 voxels={n} pairs={P}", file=sys.stderr, flush=True)

    for _ in range(max(args.warmup, 1)):
        step()
    ms_step = events_ms(step, args.steps)
    # Per-part launch durations inside the step: K more steps with HIP events
    # recorded on the launch stream between the parts (a separate pass, so the
    # timed steps above carry no extra events).  The conv's duration in the
    # roofline is its mean over conv1 and conv2 there, under the step's own
    # mix of memory-bound and MFMA-bound kernels.
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    for e in ev:
        e[0].record()
        map_and_plan()
        e[1].record()
        conv1()
        e[2].record()
        conv2()
        e[3].record()
    torch.cuda.synchronize()
    part = [sum(e[j].elapsed_time(e[j + 1]) for e in ev) / args.steps for j in range(3)]
    per_step = sorted(e[0].elapsed_time(e[3]) for e in ev)
    step_median = per_step[len(per_step) // 2]
    step_p90 = per_step[min(len(per_step) - 1, int(0.9 * len(per_step)))]
    ms_map_plan, ms_conv1, ms_conv2 = part
    ms_conv = (ms_conv1 + ms_conv2) / 2.0
    # the map and the plan on their own (the map's GB/s), then the unfused LN
    wu = max(args.warmup, 1)
    ms_map = events_ms(map_build, args.steps, wu)
    ms_plan = events_ms(plan_build, args.steps, wu)
    ms_ln = events_ms(ln_silu, args.steps, wu)
    # The same map and plan calls on the first 256 rows (sorted and unique
    # like the whole set, so the same table and row-order modes), where every
    # kernel has next to nothing to do: the per-call floor of the launch
    # chain as a Python caller sees it (the host's per-call cost bounds it
    # when that exceeds the kernels' time).
    n_t = 256
    cd_t = st.coords_d[:n_t].contiguous()
    nbr_t = torch.empty((n_t, 27), dtype=torch.int32, device=dev)
    ws_t = F.NeighborMapWorkspace(dev).get(n_t)
    plan_t = torch.empty(F.conv_plan_bytes(n_t, 27), dtype=torch.uint8, device=dev)
    map_t = lambda: F.neighbor_map_build_into(st.cfg, cd_t, nbr_t, ws_t)
    plan_tb = lambda: F.conv_plan_build_into(st.cfg, cd_t, nbr_t, plan_t)
    ms_map_floor = events_ms(map_t, args.steps, wu)
    ms_plan_floor = events_ms(plan_tb, args.steps, wu)
    # the same with the calls queued ahead of the GPU: the kernels' own floor
    ms_map_floor_gpu = queued_ms(map_t, args.steps)
    ms_plan_floor_gpu = queued_ms(plan_tb, args.steps)
    ms_map_gpu = queued_ms(map_build, args.steps)
    floor_modes = (F.neighbor_map_table_mode(ws_t), F.neighbor_map_table_mode(ws))
    print(f"[bench] step {ms_step:.3f} ms  map+plan {ms_map_plan:.3f}  conv1 {ms_conv1:.3f}  "
          f"conv2 {ms_conv2:.3f}  (alone: map {ms_map:.3f}  plan {ms_plan:.3f}  unfused ln {ms_ln:.3f}; "
          f"on {n_t} rows: map {ms_map_floor:.3f}  plan {ms_plan_floor:.3f}, queued {ms_map_floor_gpu:.3f} / "
          f"{ms_plan_floor_gpu:.3f}, map queued {ms_map_gpu:.3f}; table {floor_modes[0]} / {floor_modes[1]})",
          file=sys.stderr, flush=True)

    flops = 2.0 * P * C * C
    conv_tflops = flops / (ms_conv * 1e-3) / 1e12
    map_bytes = n * 16 + n * 27 * 4
    map_gbps = map_bytes / (ms_map * 1e-3) / 1e9
    traffic, traffic_source = None, None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tj = json.load(f)
            traffic = tj.get("conv_halo_kernel/config3", None)
            traffic_source = tj.get("source", None)

    configs = None
    if not args.no_configs:
        print("[bench] configs 2 / 4 / 5 ...", file=sys.stderr, flush=True)
        configs = config_components(dev, st)
        print(f"[bench] configs: {json.dumps(configs)}", file=sys.stderr, flush=True)
    cpu = None
    if args.cpu_sample > 0:
        print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
        cpu = cpu_baseline(coords, x_f32, w1, w2, args.cpu_sample)

    line = {
        "metric": METRIC,
        "value": n / (ms_step * 1e-3),
        "unit": "voxels/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "config3 sparse residual block (map build + conv plan + conv3x3x3 -> LN "
                               "-> SiLU -> conv3x3x3 -> +x), 256^3 ellipsoid-union shell",
                   "voxels": n, "channels": C, "kernel": "3x3x3", "valid_pairs": P,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": "conv_halo_kernel<bf16,bf16>",
                     "achieved": conv_tflops, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": conv_tflops / PEAK_BF16_TFLOPS, "traffic": traffic,
                     "traffic_source": f"profile-time figure, not measured in this run: {traffic_source}"},
        "components": {
            "step_ms_median": step_median, "step_ms_p90": step_p90,
            "map_and_plan_ms": ms_map_plan, "map_build_ms": ms_map, "plan_build_ms": ms_plan,
            "conv_ms": ms_conv,
            "conv1_ln_silu_ms": ms_conv1, "conv2_residual_ms": ms_conv2,
            "unfused_ln_silu_ms": ms_ln,
            "map_build_gbps": map_gbps, "map_build_frac_hbm": map_gbps / PEAK_HBM_GBPS,
            "map_build_256_rows_ms": ms_map_floor, "plan_build_256_rows_ms": ms_plan_floor,
            "map_build_queued_ms": ms_map_gpu, "map_build_256_rows_queued_ms": ms_map_floor_gpu,
            "plan_build_256_rows_queued_ms": ms_plan_floor_gpu,
            "conv_useful_tflops": conv_tflops,
            "conv_issued_tflops_dense27": 2.0 * n * 27 * C * C / (ms_conv * 1e-3) / 1e12,
        },
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
