"""Motion-decoder throughput on one MI355X: frames/s at 512x512, f16 weights.

A step decodes one batch of 16 frames (the 250-frame throughput workload is
decoded in launches of 16; consecutive steps walk its AR(1) latent sequence)
with every input resident in HBM: latents in device memory, frames written
to device memory.  Prints ONE JSON line (see the keys below).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch 16]
                    [--ftype f16|f32] [--workload iid|smooth|stress]
                    [--no-cpu-baseline]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "talking-portrait.cpp_amd")
sys.path[:0] = [ROOT, PKG]

PEAK_HBM_GBS = 8000.0
PEAK_TFLOPS = {"f16": 2500.0, "f32": 157.3}
REF_FPS_RTX5070TI = 213.2   # mdec, GGML-CUDA f16 fast graph (docs/vulkan-perf.md:134,143)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.md")
COPY_PROBE_BYTES = 256 << 20   # the calibration copy: reads and writes this many bytes


def measured_traffic(stage):
    """HBM bytes per launch of `stage` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (rows `| stage | fetch KiB | write KiB | ... | bytes |`),
    or None when that stage has no row"""
    try:
        for line in open(TRAFFIC_FILE):
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 6 and cells[0] == stage:
                return int(float(cells[-1]))
    except OSError:
        pass
    return None


def copy_probe():
    """a plain device copy of COPY_PROBE_BYTES, the reference kernel that
    scales the FETCH_SIZE / WRITE_SIZE counters to bytes"""
    import torch
    src = torch.ones(COPY_PROBE_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()


def fused_tail(oc, r, ftype="f16"):
    """stages whose dense conv runs the stage tail in its epilogue: all
    channels in one conv tile, the tile's pixels in one frame (256 channels:
    f16 only)"""
    bn = 256 if oc == 32 else 128
    if oc == 256:
        return ftype == "f16" and (r * r) % 128 == 0
    return oc in (32, 64, 128) and (r * r) % bn == 0


def stage_costs(ic, oc, nframes, ftype):
    """(name, algorithmic FLOPs, algorithmic HBM bytes) of every profiled
    launch group of one decode_batch call, in tpmd_stage_times slot order;
    None for the empty tail slot of a fused stage"""
    sa = 2 if ftype == "f16" else 4   # conv operand / activation bytes
    sw = sa                            # conv weight bytes
    C0 = ic[0]
    # style GEMV + demod + conv1: latents; the modulation weights of all 22
    # modulated convs (f32 rows of 512, one per input channel); S_aug of the
    # 15 demodulated convs ([OC][IC + 1] f32); conv1 weights and its output.
    # FLOPs: conv1, the style GEMVs and the demodulations
    convs = [(C0, C0)] + [(c_in, oc[j]) for j in range(len(ic)) for c_in in (ic[j], oc[j])]
    mod_rows = sum(c_in for c_in, _ in convs) + sum(oc)
    saug = sum(o * (c_in + 1) for c_in, o in convs)
    f0 = 2 * nframes * 16 * 9 * C0 * C0 + 2 * nframes * 512 * mod_rows + 2 * nframes * saug
    b0 = (nframes * 512 * 4 + mod_rows * 512 * 4 + saug * 4 + 9 * C0 * C0 * sw
          + nframes * 16 * C0 * sa)
    slots = [("style+conv1", f0, b0)]
    for j in range(len(ic)):
        r = 8 << j
        IC, OC = ic[j], oc[j]
        last = j + 1 == len(ic)
        px = nframes * r * r
        f_up = 2 * px * 9 * IC * OC
        b_up = nframes * (r // 2) ** 2 * IC * sa + px * OC * sa + 4 * OC * 9 * IC * sw
        f_dn = 2 * px * 9 * OC * OC
        # tail: feats once, previous skips, trunk (next operand), flow and rgb
        b_tl = (r * r * OC * sa + (nframes * 2 * 3 * (r // 2) ** 2 * 4 if j else 0)
                + (0 if last else px * OC * sa + px * 3 * 4) + px * 3 * 4)
        f_tl = px * OC * 2 * 6
        if fused_tail(OC, r, ftype):
            b_dt = px * OC * sa + 9 * OC * OC * sw + b_tl
            slots += [(f"r{r}.upconv", f_up, b_up), (f"r{r}.conv+tail", f_dn + f_tl, b_dt), None]
        else:
            b_dn = px * OC * sa + px * OC * 4 + 9 * OC * OC * sw
            slots += [(f"r{r}.upconv", f_up, b_up), (f"r{r}.conv", f_dn, b_dn),
                      (f"r{r}.tail", f_tl, b_tl + px * OC * 4)]
    return slots


def roofline(name, flops, nbytes, us, ftype):
    ridge = PEAK_TFLOPS[ftype] * 1e12 / (PEAK_HBM_GBS * 1e9)
    ai = flops / max(nbytes, 1)
    if ai >= ridge and flops > 0:
        ach = flops / (us * 1e-6) / 1e12
        return {"name": name, "us": round(us, 2), "bound": "mfma", "achieved": round(ach, 2),
                "peak": PEAK_TFLOPS[ftype], "unit": "TFLOP/s", "frac": round(ach / PEAK_TFLOPS[ftype], 4)}
    ach = nbytes / (us * 1e-6) / 1e9
    return {"name": name, "us": round(us, 2), "bound": "hbm", "achieved": round(ach, 1),
            "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(ach / PEAK_HBM_GBS, 4)}


def encoder_flops(cin, cout, res=512, dim=512):
    """algorithmic FLOPs of one motion-encoder run (conv MACs x 2: stem,
    per ResBlock conv1 3x3, conv2 3x3 stride 2, skip 1x1 stride 2, the final
    4x4 conv, the fc chain and Q)"""
    f = 2 * res * res * 3 * cin[0]
    r = res
    for c, co in zip(cin, cout):
        f += 2 * r * r * 9 * c * c + 2 * (r // 2) ** 2 * (9 + 1) * c * co
        r //= 2
    f += 2 * dim * 16 * cout[-1] + 2 * (4 * dim * dim + 20 * dim) + 2 * dim * 20
    return f


def encoder_timing(ftype, reps=20):
    """the motion encoder (once per portrait) on the synthetic image, device
    resident, synchronous runs: median ms and MFMA fraction"""
    import numpy as np
    import torch
    import synth
    import tpmd
    enc = tpmd.MotionEncoder(ftype)
    enc.set_weights(synth.enc_raw_weights(1004, ftype))
    enc.prepare()
    img = torch.from_numpy(synth.image(1005)).cuda()
    torch.cuda.synchronize()
    for _ in range(3):
        enc.run(img)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        lib = tpmd.lib()
        if lib.tpme_run(enc.h, tpmd._ptr(img), 1) < 0:
            raise tpmd.TpmdError(lib.tpme_last_error(enc.h).decode())
        ts.append(time.perf_counter() - t0)
    ms = float(np.median(ts)) * 1e3
    fl = encoder_flops(enc.ch_in, enc.ch_out)
    peak = 2500.0 if ftype == "f16" else 157.3
    enc.close()
    return {"ms_per_portrait": round(ms, 3), "gflop": round(fl / 1e9, 2),
            "achieved_tflops": round(fl / (ms * 1e-3) / 1e12, 1),
            "mfma_frac": round(fl / (ms * 1e-3) / 1e12 / peak, 4),
            "note": "tpme_run, 512x512 image resident in HBM, synchronous (host clock)"}


def fmt_timing(ftype, reps=5):
    """the flow-matching transformer at its default dims (src/fmt.h:10-16):
    one CFG-batched forward and one 50-frame chunk (nfe - 1 = 9 forwards),
    host in/out, median ms; GEMM FLOPs / forward time against the MFMA peak"""
    import numpy as np
    import synth
    import tpmd
    cfg = synth.FmtConfig()
    fm = tpmd.FlowTransformer(ftype)
    fm.set_weights(synth.fmt_raw_weights(cfg, ftype=ftype))
    fm.prepare()
    io = synth.fmt_chunk_inputs(cfg)
    g = np.random.default_rng(0)
    x60 = g.standard_normal((cfg.total, cfg.dim_w)).astype(np.float32)
    cond = g.standard_normal((3, cfg.total, cfg.dim_c)).astype(np.float32)
    fm.forward(x60, cond, 0.5)
    tf, tc = [], []
    for _ in range(reps):
        t0 = time.perf_counter()
        fm.forward(x60, cond, 0.5)
        tf.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        fm.sample_chunk(io["wr"], io["prev_x"], io["prev_wa"], io["cond_audio"], 1, io["x0"])
        tc.append(time.perf_counter() - t0)
    H, T = cfg.dim_h, cfg.total
    per_tok = cfg.depth * (6 * H * H + 3 * H * H + H * H + 2 * cfg.dim_mlp * H) + 2 * H * H + cfg.dim_w * H \
        + cfg.dim_c * H
    flops = 2.0 * 3 * T * per_tok + 2.0 * T * cfg.dim_w * H
    ms = float(np.median(tf)) * 1e3
    peak = 2500.0 if ftype == "f16" else 157.3
    fm.close()
    return {"forward_ms": round(ms, 3), "chunk_ms": round(float(np.median(tc)) * 1e3, 3),
            "forward_gflop": round(flops / 1e9, 2), "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / peak, 4),
            "note": "tpfm_forward / tpfm_sample_chunk, host buffers, synchronous (host clock)"}


def gather_timing(reps=50):
    """the standalone bilinear gather (tpmd_gather, GGML_OP_BILINEAR_GATHER)
    on device buffers, HIP events on the stream it runs on.  Algorithmic bytes
    per launch: N * 8 (grid) + the feature map once + N * C * 4 (f32 output).
    Grids: i.i.d. U(-a, a) (random taps, the single-stage and stress
    workloads) or a warp (pixel centres plus a smooth displacement of a few
    pixels and sub-pixel jitter, what the decoder's flow heads produce).
    Each shape is timed over 50 launches twice, replayed from a HIP graph
    (kernel nodes only; each replay checked bit for bit against an eager
    launch) and launched back to back from the host; the faster is reported
    and named."""
    import torch
    import tpmd
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(1003)
    rows = []
    for C, R, nf, f16, kind in ((512, 64, 1, False, 1.1), (512, 64, 16, False, 1.1), (512, 64, 16, True, 2.0),
                                (512, 64, 16, True, "warp"), (128, 128, 16, True, "warp"),
                                (64, 256, 16, True, "warp"), (32, 512, 16, True, "warp")):
        N = nf * R * R
        feat = torch.randn(R * R, C, device=dev, generator=g)
        feat = feat.half() if f16 else feat
        if kind == "warp":
            ax = (2 * torch.arange(R, device=dev, dtype=torch.float32) + 1) / R - 1
            gy, gx = torch.meshgrid(ax, ax, indexing="ij")
            jit = (torch.rand(nf, R, R, 2, device=dev, generator=g) - 0.5) / R
            grid = torch.stack([gx + 0.05 * torch.sin(3 * gy), gy + 0.05 * torch.cos(2 * gx)], -1) + jit
            grid = grid.reshape(N, 2).contiguous()
        else:
            grid = (torch.rand(N, 2, device=dev, generator=g) * 2 - 1) * kind
        ref = tpmd.gather(feat, R, R, grid)
        out = torch.empty(N, C, device=dev)
        # the reps captured in one HIP graph: back-to-back launches, so the
        # events time the kernels, not the host's per-call launch cost
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                tpmd.gather(feat, R, R, grid, out=out)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                tpmd.gather(feat, R, R, grid, out=out)
        # every replay is checked against the eager launch, with eager work
        # (clearing the output) between replays
        graph.replay()
        torch.cuda.synchronize()
        same = bool(torch.equal(out, ref))
        out.zero_()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / reps * 1e3
        same = same and bool(torch.equal(out, ref))   # bit for bit
        del graph
        # the same launches from the host, back to back on the stream (the
        # kernels outlast a launch call except at one frame)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            tpmd.gather(feat, R, R, grid, out=out)
        e1.record()
        torch.cuda.synchronize()
        us_eager = e0.elapsed_time(e1) / reps * 1e3
        same = same and bool(torch.equal(out, ref))
        how = "graph replay"
        if us_eager < us:
            us, how = us_eager, "stream launches"

        nbytes = N * 8 + R * R * C * feat.element_size() + N * C * 4
        name = (f"{C}x{R}x{R} {'f16' if f16 else 'f32'} feat, {nf} frame(s), "
                + ("warp grid" if kind == "warp" else f"grid U(-{kind}, {kind})"))
        row = roofline(name, 0, nbytes, us, "f16")
        row["mb"] = round(nbytes / 1e6, 2)
        row["replay_matches_eager"] = same
        row["timing"] = how
        rows.append(row)
        del feat, grid, out, ref
    return rows


def cpu_topology():
    """(logical CPUs this process may run on, physical cores among them),
    from the kernel's CPU topology"""
    cpus = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in cpus:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            cores.add((open(base + "physical_package_id").read().strip(), open(base + "core_id").read().strip()))
        except OSError:
            cores.add(("?", str(c)))
    return len(cpus), len(cores)


def cpu_baseline(ftype_unused=None):
    """the CPU oracle's fast graph (f32, numpy/OpenBLAS + OpenMP C ops) on
    this host, timed with tp-bench's mdec protocol (bench/tp-bench.cpp:
    136-151): batches of 8 frames, two untimed warm-up batches, then
    iters * 5 timed batches (iters = 1 here, a bounded sample), ms per frame
    = total / (batches * 8); threads = the physical cores (the reference's
    best CPU setting, docs/r3-summary.md:29-31)"""
    from threadpoolctl import threadpool_limits
    from oracle import mdec as om
    import synth
    logical, physical = cpu_topology()
    om.set_threads(physical)
    B, iters = 8, 1
    raw, lat, feats = synth.workload("iid", B, "f32")
    dec = om.Decoder(raw, "f32")
    dec.set_feats(feats)
    with threadpool_limits(limits=physical):
        for _ in range(2):
            dec.decode_fast(lat)
        t0 = time.perf_counter()
        for _ in range(iters * 5):
            dec.decode_fast(lat)
        dt = time.perf_counter() - t0
    n = iters * 5 * B
    return {"value": round(n / dt, 4), "unit": "frames/s", "cores": physical, "kind": "port",
            "physical_cores": physical, "logical_cpus": logical,
            "sample": f"tp-bench mdec protocol: {iters * 5} timed batches of {B} frames after 2 warm-up batches, "
                      f"f32 fast-graph oracle at 512x512, i.i.d. workload, {physical} threads "
                      f"(physical cores of the {logical} logical CPUs available)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--ftype", default="f16", choices=["f16", "f32"])
    ap.add_argument("--workload", default="iid", choices=["iid", "smooth", "stress"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--lanes", type=int, default=3, choices=[1, 3],
                    help="3: the library's own lanes (consecutive batches overlap); 1: every launch chain on "
                         "one stream (kernel traces comparable with the per-stage events)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run the 256 MiB calibration copy (for counter runs)")
    ap.add_argument("--no-graphs", action="store_true",
                    help="enqueue each launch chain launch by launch instead of replaying it as a HIP graph")
    ap.add_argument("--decoder-only", action="store_true",
                    help="skip the frame-path, encoder, FMT and gather legs (for counter runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(frames shard across GPUs by batch, with no collective per frame)",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import synth
    import tpmd

    B = args.batch
    n_seq = 250
    raw, lat, feats = synth.workload(args.workload, n_seq, args.ftype)
    dec = tpmd.MotionDecoder(args.ftype, 7, device=0)
    dec.set_weights(raw)
    dec.prepare()
    dec.build(B)
    dec.set_feats(feats)
    lat_dev = torch.from_numpy(np.concatenate([lat, lat[:B]])).cuda()   # wrap-around window
    # one frame buffer per decoder lane: consecutive calls overlap on the GPU,
    # and a call writing a buffer that an in-flight call writes would wait
    imgs_ring = [torch.empty((B, 3, 512, 512), dtype=torch.float32, device="cuda") for _ in range(3)]
    torch.cuda.synchronize()   # inputs resident before the decoder stream reads them
    if args.lanes == 1:
        dec.use_stream(torch.cuda.current_stream())   # a caller's stream: one lane
    if args.no_graphs:
        dec.use_graphs(False)

    def step(k):
        t0 = (k * B) % n_seq
        dec.decode_batch_device(lat_dev[t0:t0 + B], imgs_ring[k % 3])

    for k in range(args.warmup):
        step(k)
    dec.sync()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        step(k)
    dec.sync()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    fps = args.steps * B / dt

    # per-stage durations: HIP events recorded by the library on its stream
    nslot = dec.profile_stages(True)
    acc = np.zeros(nslot)
    nprof = max(5, min(args.steps, 20))
    for k in range(nprof):
        step(k)
        acc += np.array(dec.stage_times())
    dec.profile_stages(False)
    us = acc / nprof
    slots = stage_costs(dec.ic, dec.oc, B, args.ftype)
    stages = [roofline(sl[0], sl[1], sl[2], u, args.ftype) for sl, u in zip(slots, us) if sl is not None]
    dom = max(range(len(stages)), key=lambda i: stages[i]["us"])
    r = dict(stages[dom])
    r["kernel"] = r.pop("name")
    r["traffic"] = measured_traffic(r["kernel"])
    r.pop("us")

    # the f16 MFMA rate this GPU sustains (its clock drops under a matrix
    # load by an amount set by the operand bits): the dominant kernel's
    # fraction of it, beside the fraction of the published peak
    sustained = None
    if args.ftype == "f16":
        tf_rand, ghz_rand = tpmd.probe_mfma_f16(True)
        tf_zero, ghz_zero = tpmd.probe_mfma_f16(False)
        sustained = {"random_operands_tflops": round(tf_rand, 1), "random_operands_core_ghz": round(ghz_rand, 2),
                     "zero_operands_tflops": round(tf_zero, 1), "zero_operands_core_ghz": round(ghz_zero, 2),
                     "note": "back-to-back v_mfma_f32_32x32x16_f16, four waves per SIMD, no memory traffic "
                             "(tpmd_probe_mfma_f16)"}
        if r["bound"] == "mfma":
            r["frac_of_sustained"] = round(r["achieved"] / tf_rand, 4)

    out = {
        "metric": "motion-decoder frames/sec @512x512 f16, 1 GPU",
        "value": round(fps, 2),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,   # set below from the rate that includes the download, as the reference's does
        "dtype": "f16" if args.ftype == "f16" else "f32",
        "data": "synthetic",
        "config": {"workload": f"LIA motion decoder 512x512, {n_seq}-frame AR(1) latent sequence "
                               f"({args.workload} inputs), {B} frames per launch chain",
                   "frames_per_step": B, "resolution": 512, "ftype": args.ftype,
                   "stage_channels_in": list(dec.ic), "stage_channels_out": list(dec.oc)},
        "roofline": r,
        "stages": stages,
        "stage_sum_us": round(float(us.sum()), 1),
        "lanes": args.lanes,
        "graphs": not args.no_graphs,
    }
    if sustained:
        out["mfma_sustained"] = sustained
    if args.decoder_only:
        if args.copy_probe:
            copy_probe()
        print(json.dumps(out))
        return
    # the clip delivered to host memory through the frame output path
    # (downloads overlapped with decoding): reported beside `value`, never as it
    # into one pageable buffer reused call after call, as tp-bench reuses its
    # std::vector (bench/tp-bench.cpp:137-146): its pages are mapped before the
    # timed call; `*_fresh`: a newly allocated buffer per call, whose first
    # touch (page faults) falls inside the timed call
    host = {}
    for name, fmt, shape, dt in (("f32_chw", tpmd.FRAME_F32, (n_seq, 3, 512, 512), np.float32),
                                 ("rgb24", tpmd.FRAME_RGB24, (n_seq, 512, 512, 3), np.uint8)):
        dec.decode_frames(lat[:2 * B], fmt)               # slots allocated, warm
        t0h = time.perf_counter()
        dec.decode_frames(lat, fmt)
        host[name + "_fresh"] = round(n_seq / (time.perf_counter() - t0h), 1)
        buf = np.zeros(shape, dt)
        dec.decode_frames(lat, fmt, out=buf)              # warm, as tp-bench's two warm-up calls
        t0h = time.perf_counter()
        dec.decode_frames(lat, fmt, out=buf)
        host[name] = round(n_seq / (time.perf_counter() - t0h), 1)
        del buf
    # the same into pinned caller buffers, which take the downloads directly
    for name, fmt, shape, dt in (("f32_chw_pinned", tpmd.FRAME_F32, (n_seq, 3, 512, 512), torch.float32),
                                 ("rgb24_pinned", tpmd.FRAME_RGB24, (n_seq, 512, 512, 3), torch.uint8)):
        buf = torch.empty(shape, dtype=dt, pin_memory=True)
        dec.decode_frames(lat, fmt, out=buf)              # warm
        t0h = time.perf_counter()
        dec.decode_frames(lat, fmt, out=buf)
        host[name] = round(n_seq / (time.perf_counter() - t0h), 1)
        del buf
    out["host_delivered_fps"] = {"frames": n_seq, **host,
                                 "note": "host buffers (pageable, reused call after call unless `_fresh`; or pinned "
                                         "where named), PCIe download included"}
    # the reference's figure times decode_batch into a host std::vector, the
    # f32 download included (bench/tp-bench.cpp:133-151): compare like with like
    if args.ftype == "f16":
        out["vs_baseline"] = round(host["f32_chw"] / REF_FPS_RTX5070TI, 3)
        out["vs_baseline_basis"] = ("host_delivered_fps.f32_chw (f32 CHW frames in a reused pageable host buffer) / "
                                    f"{REF_FPS_RTX5070TI} frames/s (GGML-CUDA f16 mdec, RTX 5070 Ti, "
                                    "docs/vulkan-perf.md:134)")
        out["device_resident_vs_reference"] = round(fps / REF_FPS_RTX5070TI, 3)
    out["encoder"] = encoder_timing(args.ftype)
    out["fmt"] = fmt_timing(args.ftype)
    out["gather"] = gather_timing()
    if args.copy_probe:
        copy_probe()
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
