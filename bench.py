"""W4A16 projection benchmark on one MI355X.

Headline: the LM-head GEMV, M = 1, K = 1024,
N = 248320, W4A16 G=128 (N(0, 0.02) weights quantized per group, fp16
scales, bf16 activation ~ N(0, 1)), through the production path: the
load-time repacked weights (cudalm_w4a16_gemv_bf16_prepacked). One step =
one GEMV launch. Four weight copies rotate so each step streams from HBM
and not from the 256 MB MALL. `value` = algorithmic bytes per step /
measured time per step (GB/s).

Also reported (same JSON line, extra keys):
  * the file-layout entry (cudalm_w4a16_gemv_bf16) on the same workload;
  * configs[0] (M=1, 3584x1024) per-launch time;
  * configs[2-3]: the 24-layer decode projection census (186 calls + LM
    head) at M = 1, 8, 32, replayed from a HIP graph: us per decode step,
    and aggregate GB/s;
  * prefill-chunk GEMM, M = 512, per census shape: TFLOP/s;
  * next_rows: the tied bf16 LM head (M = 1, 8; GB/s), the SwiGLU front
    half at 3584x1024 (fused launch vs gate -> up -> silu*mul), and the
    fp16-activation twin on the LM-head workload;
  * cpu_baseline: the oracle's restatement of the reference's CPU path
    (ref_gemv_bf16) on the host cores, LM-head workload.

Synthetic data is generated with torch on the GPU (seeded), not read
from disk. Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "cudalm-agent_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "W4A16 GEMV achieved HBM GB/s (% peak) at M=1/8; µs per decode-step projections"

# 24-layer Qwen3.5-0.8B projection census, per layer in call order
# (benchmarks/profiling/v07b_w4a16_shape_census.txt; src/runtime/
# qwen35_deltanet.cpp:166-251, qwen35_full_attention.cpp:211-340).
DELTANET = [("in_proj_qkv", 6144, 1024), ("in_proj_z", 2048, 1024), ("in_proj_b", 16, 1024),
            ("in_proj_a", 16, 1024), ("out_proj", 1024, 2048)]
FULL_ATTN = [("q_proj", 4096, 1024), ("k_proj", 512, 1024), ("v_proj", 512, 1024),
             ("o_proj", 1024, 2048)]
MLP = [("gate_proj", 3584, 1024), ("up_proj", 3584, 1024), ("down_proj", 1024, 3584)]
LM_HEAD = (248320, 1024)


def layer_kinds():
    # full attention at every 4th layer (3, 7, ..., 23): 6 full, 18 DeltaNet
    return ["full" if (i % 4) == 3 else "delta" for i in range(24)]


def census_calls():
    calls = []
    for li, kind in enumerate(layer_kinds()):
        for name, N, K in (FULL_ATTN if kind == "full" else DELTANET) + MLP:
            calls.append((li, name, N, K))
    return calls


PROFILE_LM_HEAD = os.path.join(REPO, "profiles", "w4a16_stream_lm_head_M1.md")


def measured_traffic():
    """HBM bytes per LM-head launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (copy-calibrated), or None."""
    try:
        for line in open(PROFILE_LM_HEAD):
            if line.startswith("traffic_bytes_per_launch = "):
                return int(float(line.split("=")[1]))
    except OSError:
        return None
    return None


PROFILE_CENSUS = "profiles/w4a16_census_kernel_trace.md"


def census_kernel_sum_us(key: str):
    """(summed kernel durations, graph wall) in us of one census traversal
    `key` (M1, M1_fused, ...), both from the same run of the committed
    rocprofv3 kernel-trace summary, or None."""
    vals = {}
    try:
        for line in open(os.path.join(REPO, PROFILE_CENSUS)):
            for tag in ("sum_kernel_us", "traced_wall_us"):
                if line.startswith(f"{tag}[{key}] = "):
                    vals[tag] = float(line.split("=")[1])
    except OSError:
        return None
    if len(vals) != 2:
        return None
    return vals["sum_kernel_us"], vals["traced_wall_us"]


ROLES = [name for name, _, _ in DELTANET + FULL_ATTN + MLP]


def census_seed(li: int, name: str) -> int:
    """Weight seed of projection `name` of layer li: 0xC0DA0000 + 16 * layer
    + role, the role being the projection's index among the 12 census roles,
    so every matrix of the census is distinct."""
    return 0xC0DA0000 + 16 * li + ROLES.index(name)


def census_groups(fused: bool):
    """Launch groups of one decode step in call order. Fused groups are the
    projections that read the same activations (in_proj_qkv/z/b/a, gate/up,
    q/k/v)."""
    groups = []
    for li, kind in enumerate(layer_kinds()):
        if kind == "full":
            plan = [FULL_ATTN[:3], FULL_ATTN[3:], MLP[:2], MLP[2:]]
        else:
            plan = [DELTANET[:4], DELTANET[4:], MLP[:2], MLP[2:]]
        for grp in plan:
            items = [(li, name, N, K) for name, N, K in grp]
            if fused:
                groups.append(items)
            else:
                groups.extend([[it] for it in items])
    return groups


def algo_bytes(N: int, K: int, M: int) -> int:
    return N * K // 2 + 2 * N * K // 128 + 2 * M * K + 2 * M * N


def synth_weights(torch, N: int, K: int, seed: int, dev):
    """N(0, 0.02) fp32 -> reference quantizer (docs/weight_format.md:135-153)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    Wf = torch.randn((N, K), generator=g, device=dev, dtype=torch.float32) * 0.02
    Wg = Wf.view(N, K // 128, 128)
    s32 = Wg.abs().amax(dim=2) / 7
    zero = s32 == 0
    safe = torch.where(zero, torch.ones_like(s32), s32)
    q = torch.round(Wg / safe.unsqueeze(2)).clamp_(-7, 7)
    q = torch.where(zero.unsqueeze(2), torch.zeros_like(q), q).view(N, K).to(torch.int32)
    packed = (((q[:, 1::2] & 15) << 4) | (q[:, 0::2] & 15)).to(torch.uint8).contiguous()
    scale = s32.to(torch.float16).contiguous()
    del Wf, Wg, q
    return packed, scale


def synth_act(torch, M: int, K: int, seed: int, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16).contiguous()


def time_launches(torch, launches, reps: int, warmup: int, stream):
    """Run `launches` (callables) round-robin; returns (avg seconds per launch
    from per-launch event pairs, total seconds for `reps` launches)."""
    for i in range(warmup):
        launches[i % len(launches)]()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(reps):
        starts[i].record(stream)
        launches[i % len(launches)]()
        ends[i].record(stream)
    t1.record(stream)
    torch.cuda.synchronize()
    per = sum(s.elapsed_time(e) for s, e in zip(starts, ends)) / reps * 1e-3
    return per, t0.elapsed_time(t1) * 1e-3


def stream_time(torch, launches, reps: int, warmup: int, stream):
    """Seconds per launch: `reps` launches back to back (round-robin over
    `launches`) between two HIP events on `stream`, after `warmup`.

    The window holds the host's launch loop: when the host enqueues slower
    than the GPU drains, the GPU waits between launches and the figure rises
    (1.5-4 us on ~25 us kernels after a pass that created many objects, or
    after the CPU idled), while the kernel trace shows the same kernel
    duration and HBM bytes. Callers take the median of several windows."""
    for i in range(warmup):
        launches[i % len(launches)]()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(reps):
        launches[i % len(launches)]()
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) * 1e-3 / reps


def graph_time(torch, fn, reps: int, stream):
    """Capture fn() into a HIP graph, replay `reps` times; seconds per replay."""
    g = torch.cuda.CUDAGraph()
    fn()  # warm
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=stream):
        fn()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(reps):
        g.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) * 1e-3 / reps


def bench_bf16_lm_head(torch, lib, dev, stream, sraw, reps: int = 40):
    """Tied bf16 LM head (bf16_gemv / batch_bf16_gemv), M = 1 and 8, four
    rotating 508 MB weight copies; per-launch event timing. The `_prepacked`
    lines read a tile-major copy made at load time (cudalm_bf16_repack,
    outside the timed region) through cudalm_bf16_gemv_prepacked."""
    Nb, Kb = LM_HEAD
    embs = []
    for c in range(4):
        g = torch.Generator(device=dev)
        g.manual_seed(0xE4B + c)
        embs.append((torch.randn((Nb, Kb), generator=g, device=dev) * 0.02).to(torch.bfloat16))
    bf = {}
    for Mb in (1, 8):
        xb = synth_act(torch, Mb, Kb, 0xB16 + Mb, dev)
        yb = torch.empty((Mb, Nb), dtype=torch.bfloat16, device=dev)
        xbp, ybp = xb.data_ptr(), yb.data_ptr()
        L = [(lambda ep=e.data_ptr(): lib.cudalm_bf16_gemv(ep, xbp, ybp, Nb, Kb, Mb, sraw))
             for e in embs]
        per = stream_time(torch, L, reps, 8, stream)
        byts = 2 * Nb * Kb + 2 * Mb * Kb + 2 * Mb * Nb
        bf[f"M{Mb}"] = {"kernel_us": round(per * 1e6, 2), "GBps": round(byts / per / 1e9, 1),
                        "frac_hbm_peak": round(byts / per / 1e9 / HBM_PEAK_GBS, 4),
                        "algorithmic_bytes": byts}
    packs = []
    for e in embs:
        pk = torch.empty(Nb * Kb, dtype=torch.bfloat16, device=dev)
        assert lib.cudalm_bf16_repack(e.data_ptr(), pk.data_ptr(), Nb, Kb, sraw) == 0
        packs.append(pk)
    torch.cuda.synchronize()
    del embs
    for Mb in (1, 8):
        xb = synth_act(torch, Mb, Kb, 0xB16 + Mb, dev)
        yb = torch.empty((Mb, Nb), dtype=torch.bfloat16, device=dev)
        xbp, ybp = xb.data_ptr(), yb.data_ptr()
        L = [(lambda pp=p.data_ptr(): lib.cudalm_bf16_gemv_prepacked(pp, xbp, ybp, Nb, Kb, Mb, sraw))
             for p in packs]
        per = stream_time(torch, L, reps, 8, stream)
        byts = 2 * Nb * Kb + 2 * Mb * Kb + 2 * Mb * Nb
        bf[f"M{Mb}_prepacked"] = {"kernel_us": round(per * 1e6, 2), "GBps": round(byts / per / 1e9, 1),
                                  "frac_hbm_peak": round(byts / per / 1e9 / HBM_PEAK_GBS, 4),
                                  "algorithmic_bytes": byts}
    del packs
    return bf


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--copies", type=int, default=4, help="rotating weight copies (> MALL)")
    ap.add_argument("--no-census", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-next", action="store_true",
                    help="skip the bf16 LM head, SwiGLU and fp16-twin lines")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--lm-head-only", action="store_true",
                    help="headline workload only (for counter collection)")
    ap.add_argument("--bf16-lm-head-only", action="store_true",
                    help="only the tied bf16 LM head lines (for counter collection)")
    ap.add_argument("--file-lm-head-only", action="store_true",
                    help="only the W4A16 LM head through the file-layout entry, M = 1 then"
                         " M = 8 (for counter collection)")
    ap.add_argument("--cfg0-mib", type=int, default=2048,
                    help="MiB of weight copies the configs[0] line rotates over (profiler runs: 320)")
    ap.add_argument("--only", default="", choices=["", "config0", "lm_head_m8", "lm_head_m32"],
                    help="kernel-trace / counter run: the headline, then only this side line")
    ap.add_argument("--census-mode", default="", metavar="KEY",
                    help="kernel-trace run: only the census traversal KEY (M1, M1_fused, M8, ...),"
                         " graph-replayed as in the full run, then exit")
    ap.add_argument("--prefill-only", action="store_true",
                    help="headline plus the M = 512 prefill lines (for counter collection)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (x5), to scale HBM counters")
    args = ap.parse_args()
    if args.lm_head_only:
        args.no_census = args.no_prefill = args.no_cpu = args.no_next = True
    if args.prefill_only:
        args.no_census = args.no_cpu = args.no_next = True
    if args.census_mode or args.only:
        args.no_prefill = args.no_cpu = args.no_next = True
    if args.only:
        args.no_census = True

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the W4A16 projection path runs on a single "
              "MI355X here (sharding along N across GPUs is a design, not built or run).",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    if args.copy_calibration:
        src = torch.empty(args.copy_calibration << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": args.copy_calibration << 20, "calls": 5}))
        return

    import cudalm_w4a16 as w4

    dev = torch.device("cuda:0")
    # one non-default stream carries every launch (graph capture needs one)
    stream = torch.cuda.Stream(device=dev)
    torch.cuda.set_stream(stream)
    sraw = stream.cuda_stream
    lib = w4.lib()

    if args.bf16_lm_head_only:
        print(json.dumps({"bf16_lm_head": bench_bf16_lm_head(torch, lib, dev, stream, sraw,
                                                             reps=args.steps)}), flush=True)
        return

    if args.file_lm_head_only:
        # the drop-in call on the file's row-major weights (no repack), over
        # the same rotating copies as the headline
        N, K = LM_HEAD
        fw = [synth_weights(torch, N, K, 0x11AD + c, dev) for c in range(args.copies)]
        res = {}
        for Mf in (1, 8):
            xf = synth_act(torch, Mf, K, 0x11AE + Mf, dev)
            yf = torch.empty((Mf, N), dtype=torch.bfloat16, device=dev)
            lf = [(lambda w=w, s=s, xf=xf, yf=yf, Mf=Mf: lib.cudalm_w4a16_gemv_bf16(
                w.data_ptr(), s.data_ptr(), xf.data_ptr(), yf.data_ptr(), N, K, Mf, sraw))
                  for w, s in fw]
            t = stream_time(torch, lf, args.steps, args.warmup, stream)
            nb = algo_bytes(N, K, Mf)
            res[f"M{Mf}"] = {"kernel_us": round(t * 1e6, 2), "GBps": round(nb / t / 1e9, 1),
                             "frac_hbm_peak": round(nb / t / 1e9 / HBM_PEAK_GBS, 4)}
        print(json.dumps({"file_layout_lm_head": res}), flush=True)
        return

    # ---------------- headline: LM head, M = 1, prepacked ----------------
    N, K = LM_HEAD
    M = 1
    packs, ws, ss = [], [], []
    for c in range(args.copies):
        w, s = synth_weights(torch, N, K, 0x11AD + c, dev)
        packs.append(w4.repack(w, s, N, K))
        ws.append(w)
        ss.append(s)
    x = synth_act(torch, M, K, 0x11AE, dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    xp, yp = x.data_ptr(), y.data_ptr()

    def mk_packed(p):
        pp = p.data_ptr()
        return lambda: lib.cudalm_w4a16_gemv_bf16_prepacked(pp, xp, yp, N, K, M, sraw)

    def mk_file(w, s):
        wp_, sp_ = w.data_ptr(), s.data_ptr()
        return lambda: lib.cudalm_w4a16_gemv_bf16(wp_, sp_, xp, yp, N, K, M, sraw)

    # the timed region: K steps bracketed by synchronize on both sides
    launches = [mk_packed(p) for p in packs]
    per_launch, _ = time_launches(torch, launches, min(args.steps, 100), args.warmup, stream)
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t_start = time.perf_counter()
    ev0.record(stream)  # HIP events on the stream the kernels run on
    for i in range(args.steps):
        launches[i % len(launches)]()
    ev1.record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    step_s = elapsed / args.steps
    kern_s = ev0.elapsed_time(ev1) * 1e-3 / args.steps  # back-to-back launches
    nbytes = algo_bytes(N, K, M)
    value = nbytes / step_s / 1e9
    kern_gbs = nbytes / kern_s / 1e9

    extra = {}
    # ---------------- small-M batched decode on the LM head (M = 8, 32) ----------------
    if not args.lm_head_only and not args.census_mode and args.only in ("", "lm_head_m8", "lm_head_m32"):
        small = {}
        for Mb in (8, 32):
            if args.only and args.only != f"lm_head_m{Mb}":
                continue
            xb = synth_act(torch, Mb, K, 0x11B0 + Mb, dev)
            yb = torch.empty((Mb, N), dtype=torch.bfloat16, device=dev)
            xbp, ybp = xb.data_ptr(), yb.data_ptr()
            lb = [(lambda pp=p.data_ptr(): lib.cudalm_w4a16_gemv_bf16_prepacked(pp, xbp, ybp, N, K, Mb, sraw))
                  for p in packs]
            per_b = sorted(stream_time(torch, lb, 100, args.warmup, stream) for _ in range(3))[1]
            nb = algo_bytes(N, K, Mb)
            small[f"M{Mb}"] = {"kernel_us": round(per_b * 1e6, 2), "GBps": round(nb / per_b / 1e9, 1),
                               "frac_hbm_peak": round(nb / per_b / 1e9 / HBM_PEAK_GBS, 4),
                               "algorithmic_bytes": nb}
        extra["lm_head_small_m"] = small
    file_per = float("nan")
    if not args.lm_head_only and not args.census_mode and not args.only:
        file_per = stream_time(torch, [mk_file(w, s) for w, s in zip(ws, ss)],
                               min(args.steps, 100), args.warmup, stream)
    file_gbs = nbytes / file_per / 1e9 if file_per == file_per else None

    # M = 1, N = 3584, K = 1024. The launches rotate over 2 GiB
    # of weight copies by default (1,130 matrices of 1.9 MB: 16 synthesized
    # ones, each at ~70 addresses), more than the 256 MB MALL, so every
    # launch reads its weights from HBM as it would in the census.
    cfg0_s = None
    if not args.lm_head_only and not args.census_mode and args.only in ("", "config0"):
        N0, K0 = 3584, 1024
        base = []
        for c in range(16):
            w, s = synth_weights(torch, N0, K0, 0x3584 + c, dev)
            base.append(w4.repack(w, s, N0, K0))
        ncopies = max(16, -(-(args.cfg0_mib << 20) // base[0].numel()))
        c0 = [base[c % 16] if c < 16 else base[c % 16].clone() for c in range(ncopies)]
        x0 = synth_act(torch, 1, K0, 0x3585, dev)
        y0 = torch.empty((1, N0), dtype=torch.bfloat16, device=dev)
        x0p, y0p = x0.data_ptr(), y0.data_ptr()
        c0_launch = [(lambda pp=p.data_ptr(): lib.cudalm_w4a16_gemv_bf16_prepacked(pp, x0p, y0p, N0, K0, 1, sraw))
                     for p in c0]
        cfg0_s = graph_time(torch, lambda: [f() for f in c0_launch], 20 if len(c0_launch) <= 200 else 5,
                            stream) / len(c0_launch)
        del c0, base

    # ---------------- census: 186 projections + LM head per decode step ----------------
    if not args.no_census:
        calls = census_calls()
        cw, cf = {}, {}
        for li, name, Nc, Kc in calls:
            w, s = synth_weights(torch, Nc, Kc, census_seed(li, name), dev)
            cw[(li, name)] = w4.repack(w, s, Nc, Kc)
            cf[(li, name)] = (w, s)
        census = {}
        for Mc in (1, 8, 32):
            if args.census_mode and not args.census_mode.startswith(f"M{Mc}"):
                continue
            xs = {Kc: synth_act(torch, Mc, Kc, 0xAC70 + Kc + Mc, dev) for Kc in (1024, 2048, 3584)}
            ys = {(li, name): torch.empty((Mc, Nc), dtype=torch.bfloat16, device=dev)
                  for li, name, Nc, Kc in calls}
            xh = synth_act(torch, Mc, K, 0x11AF + Mc, dev)
            yh = torch.empty((Mc, N), dtype=torch.bfloat16, device=dev)
            tot_bytes = sum(algo_bytes(Nc, Kc, Mc) for _, _, Nc, Kc in calls) + algo_bytes(N, K, Mc)
            for fused in (False, True):
                key = f"M{Mc}" + ("_fused" if fused else "")
                if args.census_mode and args.census_mode != key:
                    continue
                launches = []  # (list of (packed_ptr, y_ptr, N), K)
                for group in census_groups(fused):
                    Kc = group[0][3]
                    launches.append(([(cw[(li, nm)].data_ptr(), ys[(li, nm)].data_ptr(), Nc)
                                      for li, nm, Nc, _ in group], Kc))
                launches.append(([(packs[0].data_ptr(), yh.data_ptr(), N)], K))
                arrays = [(w4.proj_array([(pp, None, yy, nn) for pp, yy, nn in items]), len(items),
                           xs[Kc].data_ptr() if (items[0][0] != packs[0].data_ptr()) else xh.data_ptr(), Kc)
                          for items, Kc in launches]

                def traversal(arrays=arrays, Mc=Mc):
                    for arr, cnt, xx, Kc in arrays:
                        if cnt == 1:
                            p0 = arr[0]
                            lib.cudalm_w4a16_gemv_bf16_prepacked(p0.weight, xx, p0.y, p0.N, Kc, Mc, sraw)
                        else:
                            lib.cudalm_w4a16_gemv_bf16_multi(ctypes.cast(arr, ctypes.c_void_p), cnt, xx,
                                                             Kc, Mc, 1, sraw)

                t = graph_time(torch, traversal, 10, stream)
                if args.census_mode:
                    # 1 eager + 3 warm + 10 timed traversals were dispatched
                    print(json.dumps({"census_mode": key, "launches": len(arrays),
                                      "traversals_dispatched": 14,
                                      "us_per_decode_step": round(t * 1e6, 2)}), flush=True)
                    return
                census[key] = {
                    "us_per_decode_step": round(t * 1e6, 2),
                    "launches": len(arrays),
                    "bytes": tot_bytes,
                    "GBps": round(tot_bytes / t / 1e9, 1),
                    "frac_hbm_peak": round(tot_bytes / t / 1e9 / HBM_PEAK_GBS, 4),
                }
                prof = census_kernel_sum_us(key)
                if prof:
                    # census roofline: the summed kernel durations of one
                    # traversal (committed rocprofv3 kernel trace) against this
                    # run's untraced graph wall; a ratio near or above 1 means
                    # the kernels themselves fill the traversal (the tracer
                    # lengthens each dispatch, and its wall depends on the box)
                    ksum = prof[0]
                    census[key].update({
                        "sum_kernel_us_traced": ksum,
                        "sum_kernel_over_wall": round(ksum * 1e-6 / t, 3),
                        "GBps_over_sum_kernel": round(tot_bytes / (ksum * 1e-6) / 1e9, 1),
                        "frac_hbm_peak_over_sum_kernel": round(tot_bytes / (ksum * 1e-6) / 1e9
                                                               / HBM_PEAK_GBS, 4),
                        "source": PROFILE_CENSUS})
            # stage chain: the fused groups as dependent stages of one
            # persistent launch (each waits for the previous one, the
            # runtime's worst case), then the LM head launch. The _swiglu
            # form runs every MLP as the reference's data flow: gate/up as a
            # SwiGLU stage writing act = silu(gate) * up (the
            # qwen35_silu_mul_bf16 step, with no launch of its own), down
            # reading act.
            act = torch.empty((Mc, MLP[0][1]), dtype=torch.bfloat16, device=dev)
            for key in (f"M{Mc}_chain", f"M{Mc}_chain_swiglu"):
                if args.census_mode and args.census_mode != key:
                    continue
                swiglu = key.endswith("_swiglu")
                stages = []
                for gi, group in enumerate(census_groups(True)):
                    Kc = group[0][3]
                    names = [nm for _, nm, _, _ in group]
                    xin = xs[Kc].data_ptr()
                    act_arg = ()
                    if swiglu and names == ["gate_proj", "up_proj"]:
                        act_arg = (act,)
                    elif swiglu and names == ["down_proj"]:
                        xin = act.data_ptr()
                    stages.append(([(cw[(li, nm)].data_ptr(), None, ys[(li, nm)].data_ptr(), Nc)
                                    for li, nm, Nc, _ in group], xin, Kc, gi - 1) + act_arg)
                chain = w4.Chain(stages, Mc, prepacked=True, stream=stream)
                hp, xhp, yhp = packs[0].data_ptr(), xh.data_ptr(), yh.data_ptr()

                def traversal_chain(chain=chain, Mc=Mc):
                    chain.run(stream=stream)
                    lib.cudalm_w4a16_gemv_bf16_prepacked(hp, xhp, yhp, N, K, Mc, sraw)

                t = graph_time(torch, traversal_chain, 10, stream)
                chain.status(stream=stream)
                if args.census_mode:
                    print(json.dumps({"census_mode": key, "launches": 2, "traversals_dispatched": 14,
                                      "us_per_decode_step": round(t * 1e6, 2)}), flush=True)
                    return
                census[key] = {
                    "us_per_decode_step": round(t * 1e6, 2),
                    "launches": 2,
                    "stages": len(stages),
                    **({"swiglu_stages": sum(len(sg) == 5 for sg in stages)} if swiglu else {}),
                    "bytes": tot_bytes,
                    "GBps": round(tot_bytes / t / 1e9, 1),
                    "frac_hbm_peak": round(tot_bytes / t / 1e9 / HBM_PEAK_GBS, 4),
                }
            if Mc == 1 and not args.census_mode:
                # the drop-in case: the reference's 187 call sites unchanged,
                # file-layout weights (no repack), one launch per projection
                fl = [(cf[(li, nm)][0].data_ptr(), cf[(li, nm)][1].data_ptr(),
                       xs[Kc].data_ptr(), ys[(li, nm)].data_ptr(), Nc, Kc) for li, nm, Nc, Kc in calls]

                def traversal_file(fl=fl):
                    for wp_, sp_, xx, yy, nn, kk in fl:
                        lib.cudalm_w4a16_gemv_bf16(wp_, sp_, xx, yy, nn, kk, 1, sraw)
                    lib.cudalm_w4a16_gemv_bf16(ws[0].data_ptr(), ss[0].data_ptr(), xh.data_ptr(),
                                               yh.data_ptr(), N, K, 1, sraw)

                t = graph_time(torch, traversal_file, 10, stream)
                census["M1_file_layout"] = {
                    "us_per_decode_step": round(t * 1e6, 2),
                    "launches": len(fl) + 1,
                    "bytes": tot_bytes,
                    "GBps": round(tot_bytes / t / 1e9, 1),
                    "frac_hbm_peak": round(tot_bytes / t / 1e9 / HBM_PEAK_GBS, 4),
                }
        extra["census"] = census
        del cw, cf

    # ---------------- prefill chunk GEMM, M = 512 ----------------
    if not args.no_prefill:
        pre = {}
        Mp = 512
        for Np, Kp in ((3584, 1024), (1024, 3584), (6144, 1024), (4096, 1024), (2048, 1024),
                       (1024, 2048), (512, 1024)):
            w, s = synth_weights(torch, Np, Kp, 0xBEEF + Np + Kp, dev)
            p = w4.repack(w, s, Np, Kp)
            xpf = synth_act(torch, Mp, Kp, 0xF00D, dev)
            ypf = torch.empty((Mp, Np), dtype=torch.bfloat16, device=dev)
            pp, xx, yy = p.data_ptr(), xpf.data_ptr(), ypf.data_ptr()
            t = graph_time(torch, lambda: [lib.cudalm_w4a16_gemv_bf16_prepacked(pp, xx, yy, Np, Kp, Mp, sraw)
                                           for _ in range(10)], 5, stream) / 10
            fl = 2.0 * Mp * Np * Kp
            pre[f"{Np}x{Kp}"] = {"us": round(t * 1e6, 2), "TFLOPs": round(fl / t / 1e12, 1),
                                 "frac_bf16_peak": round(fl / t / 1e12 / BF16_PEAK_TFLOPS, 4)}
        extra["prefill_M512"] = pre

    # ---------------- next rows: bf16 LM head, SwiGLU epilogue, fp16 twin ----------------
    if not args.no_next:
        nxt = {}
        nxt["bf16_lm_head"] = bench_bf16_lm_head(torch, lib, dev, stream, sraw)
        # SwiGLU front half at the MLP shape: gate, up, silu*mul
        Ng, Kg = 3584, 1024
        gu = []
        for c in range(16):
            w, s = synth_weights(torch, Ng, Kg, 0x5C0 + c, dev)
            gu.append(w4.repack(w, s, Ng, Kg))
        sw = {}
        for Mg in (1, 8, 32):
            xg = synth_act(torch, Mg, Kg, 0x5C1 + Mg, dev)
            tg = torch.empty((Mg, Ng), dtype=torch.bfloat16, device=dev)
            tu, yg = torch.empty_like(tg), torch.empty_like(tg)
            xgp, tgp, tup, ygp = xg.data_ptr(), tg.data_ptr(), tu.data_ptr(), yg.data_ptr()
            pairs = [(gu[2 * c].data_ptr(), gu[2 * c + 1].data_ptr()) for c in range(8)]

            def three(pairs=pairs, Mg=Mg):
                for a, b in pairs:
                    lib.cudalm_w4a16_gemv_bf16_prepacked(a, xgp, tgp, Ng, Kg, Mg, sraw)
                    lib.cudalm_w4a16_gemv_bf16_prepacked(b, xgp, tup, Ng, Kg, Mg, sraw)
                    lib.cudalm_silu_mul_bf16(tgp, tup, ygp, Mg * Ng, sraw)

            def one(pairs=pairs, Mg=Mg):
                for a, b in pairs:
                    lib.cudalm_w4a16_swiglu_bf16(a, None, b, None, xgp, ygp, Ng, Kg, Mg, 1, sraw)

            t3 = graph_time(torch, three, 10, stream) / len(pairs)
            t1 = graph_time(torch, one, 10, stream) / len(pairs)
            sw[f"M{Mg}"] = {"three_launch_us": round(t3 * 1e6, 2), "fused_us": round(t1 * 1e6, 2),
                            "fused_GBps": round(2 * algo_bytes(Ng, Kg, Mg) / t1 / 1e9, 1)}
        nxt["swiglu_gate_up_3584x1024"] = sw
        del gu
        # fp16-activation twin (int4_gemv) on the LM-head workload
        xh16 = torch.randn((1, K), device=dev).to(torch.float16)
        yh16 = torch.empty((1, N), dtype=torch.float16, device=dev)
        L = [(lambda pp=p.data_ptr(): lib.cudalm_w4a16_gemv_f16_prepacked(pp, xh16.data_ptr(),
                                                                          yh16.data_ptr(), N, K, 1,
                                                                          sraw)) for p in packs]
        per = stream_time(torch, L, 100, 8, stream)
        nxt["f16_twin_lm_head_M1"] = {"kernel_us": round(per * 1e6, 2),
                                      "GBps": round(nbytes / per / 1e9, 1)}
        extra["next_rows"] = nxt

    # ---------------- CPU baseline (oracle restatement of ref_gemv_bf16) ----------------
    cpu = None
    if not args.no_cpu:
        import oracle

        Wn = ws[0].cpu().numpy()
        Sn = ss[0].view(torch.int16).cpu().numpy().view(np.uint16)
        Xn = x.view(torch.int16).cpu().numpy().view(np.uint16)
        # the GPU boxes allot 16 host threads per GPU, whatever the host reports
        avail = oracle.hardware_threads()
        threads = min(avail, 16)
        one = oracle.time_gemv_bf16(Wn, Sn, Xn, N, K, 1, threads, 1)
        iters = max(1, int(args.cpu_seconds / max(one, 1e-3)))
        t_cpu = oracle.time_gemv_bf16(Wn, Sn, Xn, N, K, 1, threads, iters)
        cpu = {"value": round(nbytes / t_cpu / 1e9, 2), "unit": "GB/s", "cores": threads,
               "cores_available": avail,
               "kind": "port",
               "sample": f"full LM-head GEMV (N={N}, K={K}, M=1), {iters} calls after 1 warm-up, "
                         f"rows split over {threads} threads (the box's 16-thread share per GPU; "
                         f"the host reports {avail}); {t_cpu * 1e3:.1f} ms per call"}
        # parity of the timed headline kernel: y from packs[0] against the
        # fp64 bound and against the reference's own CPU loop (ref_gemv_bf16)
        lib.cudalm_w4a16_gemv_bf16_prepacked(packs[0].data_ptr(), xp, yp, N, K, M, sraw)
        torch.cuda.synchronize()
        Yg = y.view(torch.int16).cpu().numpy().view(np.uint16).reshape(M, N)
        ok, st = oracle.full_parity(Yg, Wn, Sn, Xn, N, K, M, threads)
        Yr = oracle.gemv_bf16(Wn, Sn, Xn, N, K, M, threads)
        diff = np.abs(oracle.bf16_to_f32(Yg).astype(np.float64) - oracle.bf16_to_f32(Yr).astype(np.float64))
        cpu["parity"] = {"within_tolerance": bool(ok), "max_ulp_vs_fp64": round(st["max_ulp"], 3),
                         "n_over_2ulp": st["n_over_2ulp"], "n": st["n"],
                         "ref_cpu_loop_max_ulp_vs_fp64": round(st["ref_max_ulp"], 3),
                         "ref_cpu_loop_n_over_2ulp": st["ref_n_over_2ulp"],
                         # the north_star's bar as written: bf16 ulps from the
                         # reference loop's fp32 accumulator (ref_gemv_bf16)
                         "max_ulp_vs_fp32_ref": round(st["max_ulp_vs_fp32_ref"], 3),
                         "n_over_2ulp_vs_fp32_ref": st["n_over_2ulp_vs_fp32_ref"],
                         "n_differ_from_ref_cpu_loop": int((Yg != Yr).sum()),
                         "max_abs_diff_vs_ref_cpu_loop": float(diff.max())}
        # single-core form of the reference's loop, on a bounded row sample
        rows = 16384
        t1 = oracle.time_gemv_bf16(Wn[:rows].copy(), Sn[:rows].copy(), Xn, rows, K, 1, 1, 3)
        cpu["single_core_GBps"] = round(algo_bytes(rows, K, 1) / t1 / 1e9, 3)

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xbf16->fp32",
        "data": "synthetic (torch-seeded N(0,0.02) weights quantized W4A16 G=128; N(0,1) bf16 x)",
        "config": {"workload": "LM-head W4A16 GEMV, M=1, K=1024, N=248320 (BASELINE configs[1]), "
                               "prepacked weights, 4 rotating copies",
                   "M": M, "N": N, "K": K, "group": 128, "parallelism": "single-gpu"},
        "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(kern_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(kern_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "traffic_source": "profiles/w4a16_stream_lm_head_M1.md (rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0, copy-calibrated)",
                     "kernel": "w4a16_stream_piece_one_kernel<true, 1, false, 1, ActBf16, 4, true, 4, false>",
                     "kernel_us": round(kern_s * 1e6, 3),
                     "kernel_us_source": "HIP events around the timed K launches / K",
                     "kernel_us_event_pairs": round(per_launch * 1e6, 3),
                     "algorithmic_bytes_per_launch": nbytes},
        "file_layout_entry": ({"kernel_us": round(file_per * 1e6, 3), "GBps": round(file_gbs, 1)}
                              if file_gbs else None),
        "config0_M1_3584x1024": ({"us": round(cfg0_s * 1e6, 3),
                                  "GBps": round(algo_bytes(3584, 1024, 1) / cfg0_s / 1e9, 1)}
                                 if cfg0_s else None),
        "cpu_baseline": cpu,
    }
    out.update(extra)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
