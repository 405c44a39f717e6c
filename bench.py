#!/usr/bin/env python3
"""Benchmark of the routed-expert hot path on one MI355X.

Metric: expert-FFN decode GB/s (% of HBM peak) + prefill grouped-GEMM TFLOP/s.

Workloads (synthetic, seeds of the benchmark configs; weights quantised on the GPU by the
library's own quantiser against the config-1 codebook the reference fitted; affinity_amd/
synthetic.py):
  value      C5: batch-1 decode of the config-2 MoE layer (256 experts x 2.875 bpw, top-6 softmax
             routes) through a stack of resident layers (43 by default: 92.9 GiB), one token per
             step, captured in a HIP graph. GB/s counts algorithmic bytes: 6 experts x 9,060,352 B
             per layer (codes + fields + row scales; activations excluded).
  c3         M = 8 speculative-decode tokens per layer, same stack; bytes = distinct experts x stride.
  prefill    C4: 4096 tokens x hidden 4096 (bf16), Zipf(1.1) routes, one layer; TFLOP/s counts
             2*(2*I*H + H*I) per (token, expert) slot = 1.2370e12 FLOP per layer.
  roofline   the dominant decode kernel (the persistent per-layer launch): its algorithmic bytes
             per launch (6 x 9,060,352 B) over its average duration, timed with HIP events on the
             launch stream (the C5 graph holds only these launches); traffic = HBM bytes per
             launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary.
  shared_expert  the FP8 shared expert that follows the routed experts (hidden 4096, inter 2048,
             one per layer, random E4M3 weights): batch-1 decode over the layers in a graph (GB/s
             of its 25 MB of weights) and one 4096-token bf16 chunk (TFLOP/s).
  producer   the config-1 codebook recipe (3 x 2^19 samples of the config-1 matrices, the joint
             fit, projection, packing) on the GPU, timed, and compared with the reference's packed
             codebook bit for bit.
  cpu_baseline  the reference's own CPU path (oracle/_ref/libaffref.so, else the oracle that
             restates it) on bounded samples of every config, on this host's cores; its outputs are
             also the checker of the GPU results reported under "parity".

    python bench.py [--steps K] [--warmup W] [--layers L] [--gpus 1]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

from affinity_amd import synthetic  # noqa: E402
from affinity_amd.synthetic import E, H, I, K, S_R, S_X  # noqa: E402

STRIDE = 9_060_352
HBM_PEAK = 8.0e12               # B/s, MI355X
BF16_PEAK = 2.5e15              # FLOP/s dense, MI355X
FLOP_PER_SLOT = 2 * (2 * I * H + H * I)
S_SHEXP = 17                    # seed of the synthetic shared-expert weights


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def rel_l2(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


class ClockSampler:
    """The GPU's shader clock while a timed region runs: a thread reads amdsmi's current gfx clock
    (the mean over the XCDs) every few milliseconds between start() and stop(). Records why when
    the reading is unavailable (no amdsmi, no permission); never raises."""

    def __init__(self, period_s: float = 0.002):
        self.period = period_s
        self.err = None
        self.handle = None
        try:
            import amdsmi
            amdsmi.amdsmi_init()
            self.smi = amdsmi
            self.handle = amdsmi.amdsmi_get_processor_handles()[0]
            self.read()
        except Exception as e:  # noqa: BLE001 - recorded in the result instead
            self.err = f"{type(e).__name__}: {e}"
            self.handle = None

    def read(self) -> float:
        m = self.smi.amdsmi_get_gpu_metrics_info(self.handle)
        per_xcd = [v for v in m.get("current_gfxclks", []) if isinstance(v, (int, float)) and v < 65535]
        if per_xcd:
            return float(sum(per_xcd)) / len(per_xcd)
        return float(self.smi.amdsmi_get_clock_info(self.handle, self.smi.AmdSmiClkType.GFX)["clk"])

    def start(self) -> None:
        import threading
        self.samples, self.stop_flag = [], False

        def run():
            while not self.stop_flag:
                try:
                    self.samples.append(self.read())
                except Exception as e:  # noqa: BLE001
                    self.err = f"{type(e).__name__}: {e}"
                    return
                time.sleep(self.period)
        if self.handle is not None:
            self.thread = threading.Thread(target=run, daemon=True)
            self.thread.start()

    def stop(self) -> dict:
        if self.handle is None:
            return {"mhz": None, "why": self.err}
        self.stop_flag = True
        self.thread.join()
        v = self.samples
        if not v:
            return {"mhz": None, "why": self.err or "no sample inside the timed region"}
        return {"mhz": round(sum(v) / len(v), 1), "min": min(v), "max": max(v), "samples": len(v)}


def time_graph(torch, fn, steps, warmup, clock=None, clock_key=None, clocks=None):
    """Captures fn into a HIP graph and times `steps` replays with events on the current stream
    (with `clock`, the shader clock over the timed replays goes to clocks[clock_key])."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if clock is not None:
        clock.start()
    start.record()
    for _ in range(steps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    if clock is not None:
        clocks[clock_key] = clock.stop()
    return start.elapsed_time(end) / steps, g, out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=43)
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["decode", "all"], default="all")
    ap.add_argument("--staged", action="store_true",
                    help="also time the three-launch (staged) decode for comparison")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run a plain 1 GiB device copy (the reference point for HBM counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: the routed-expert path is single-GPU in this build "
              "(the multi-GPU split is a design note, not built). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch
    import affinity_amd.experts as ax
    from affinity_amd._lib import lib, check

    ax.init()
    torch.cuda.set_device(0)
    cb_packed = synthetic.c1_codebook()
    clock = ClockSampler()
    clocks: dict = {}
    L = args.layers

    if args.calibrate:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration copy: 1 GiB read + 1 GiB written")
        del src, dst

    # ---- resident stack ----------------------------------------------------------------------
    cont = synthetic.build_layer_container(ax, torch, log=log)
    pools = [ax.ExpertPool.from_container(cont, cb_packed) for _ in range(L)]
    torch.cuda.synchronize()
    log(f"{L} layers resident: {L * E * STRIDE / 2**30:.2f} GiB")
    layers = [p.layer() for p in pools]

    # ---- decode inputs -------------------------------------------------------------------------
    x1 = ax.gen_normal(S_X, H, 1.0).view(1, H)
    x8 = ax.gen_normal(S_X, 8 * H, 1.0).view(8, H)
    routes1, routes8 = [], []
    for l in range(L):
        lg = ax.gen_normal(S_R + l, 8 * E, 1.0, bf16_round=False).view(8, E)
        routes1.append(synthetic.softmax_topk(lg[:1], K))
        routes8.append(synthetic.softmax_topk(lg, K))
    ws1 = ax.DecodeWorkspace(1, K)
    ws8 = ax.DecodeWorkspace(8, K)
    y1 = torch.zeros((L, H), device="cuda")
    y8 = torch.zeros((L, 8, H), device="cuda")

    def decode_step(x, routes, ws, y, M):
        s = torch.cuda.current_stream().cuda_stream
        for l in range(L):
            sel, w = routes[l]
            check(lib().affx_expert_ffn_decode(C.byref(layers[l]), x.data_ptr(), H, 1, M, sel.data_ptr(),
                                               w.data_ptr(), K, y[l].data_ptr(), H, 1, 0, ws.buf.data_ptr(),
                                               ws.bytes, s), "decode")
        return y

    # eager reference result, then the graph
    decode_step(x1, routes1, ws1, y1, 1)
    torch.cuda.synchronize()
    eager1 = y1.clone()
    ms1, g1, _ = time_graph(torch, lambda: decode_step(x1, routes1, ws1, y1, 1), args.steps, args.warmup,
                            clock, "c5_decode", clocks)
    torch.cuda.synchronize()
    assert torch.equal(y1, eager1), "graph replay differs from the eager decode"
    bytes_tok = L * K * STRIDE
    gbs = bytes_tok / (ms1 * 1e-3) / 1e9
    log(f"C5 decode: {ms1 * 1e3:.1f} us/token over {L} layers -> {gbs:.0f} GB/s "
        f"({100 * gbs * 1e9 / HBM_PEAK:.1f}% of HBM peak)")

    # ---- the dominant kernel: the persistent decode launch, one per layer ------------------------
    # the C5 graph holds nothing but the L launches of decode_fused_kernel on the stream that the
    # events above were recorded on, so its per-launch duration is the graph time over L
    fu_us = ms1 * 1e3 / L
    fu_bytes = K * STRIDE
    fu_achieved = fu_bytes / (fu_us * 1e-6) / 1e9
    log(f"decode_fused_kernel: {fu_us:.2f} us/launch avg, {fu_bytes} B -> {fu_achieved:.0f} GB/s")
    # HBM bytes per launch from the committed counter summary (FETCH_SIZE + WRITE_SIZE passes,
    # each scaled by what the counter reads for a plain copy of known size)
    traffic = None
    tpath = os.path.join(HERE, "profiles", "decode_fused_c5_traffic.txt")
    if os.path.exists(tpath):
        with open(tpath) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch:"):
                    traffic = int(line.split(":")[1])

    if args.staged:
        def staged_step():
            st = torch.cuda.current_stream().cuda_stream
            for l in range(L):
                sel, w = routes1[l]
                check(lib().affx_decode_staged(C.byref(layers[l]), x1.data_ptr(), H, 1, 1, sel.data_ptr(),
                                               w.data_ptr(), K, y1.data_ptr() + 4 * H * l, H, 1, 0,
                                               ws1.buf.data_ptr(), ws1.bytes, st), "staged")
            return y1
        mss, _, _ = time_graph(torch, staged_step, args.steps, args.warmup)
        assert torch.equal(y1, eager1), "staged decode differs from the fused decode"
        log(f"C5 staged (3 launches per layer): {mss * 1e3:.1f} us/token -> "
            f"{bytes_tok / (mss * 1e-3) / 1e9:.0f} GB/s")

    # ---- C3: M = 8 tokens ------------------------------------------------------------------------
    ms8, _, _ = time_graph(torch, lambda: decode_step(x8, routes8, ws8, y8, 8), args.steps, args.warmup,
                           clock, "c3_decode", clocks)
    distinct = sum(int(torch.unique(r[0]).numel()) for r in routes8)
    gbs8 = distinct * STRIDE / (ms8 * 1e-3) / 1e9
    log(f"C3 decode (M=8): {ms8 * 1e3:.1f} us/step, {distinct / L:.1f} experts/layer -> {gbs8:.0f} GB/s")

    # a launch whose workgroups gave up waiting for each other wrote invalid output: fail the run
    st1, st8 = ws1.status(), ws8.status()
    if st1 or st8:
        log(f"decode workspace status {st1}, {st8}: a launch gave up waiting; results invalid")
        return 3

    result = {
        "metric": "expert-FFN decode GB/s (% of HBM peak) + prefill grouped-GEMM TFLOP/s",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms1, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3 weights x 3-term e4m3 activations, fp32 accumulate",
        "data": "synthetic: seeded bf16(0.02 N(0,1)) experts quantised on the GPU at 2.875 bpw",
        "config": {"workload": f"C5: batch-1 decode, config-2 layer (256 experts, top-6) x {L} resident "
                               f"layers ({L * E * STRIDE / 2**30:.1f} GiB), HIP graph per token",
                   "hbm_fraction": round(gbs * 1e9 / HBM_PEAK, 4),
                   "tokens_per_s_expert_only": round(1e3 / ms1, 1),
                   "bytes_per_token": bytes_tok},
        "roofline": {"bound": "hbm", "achieved": round(fu_achieved, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(fu_achieved * 1e9 / HBM_PEAK, 4), "traffic": traffic,
                     "kernel": "decode_fused_kernel<1,8,1,true,true,1>", "bytes_per_launch": fu_bytes,
                     "us_per_launch": round(fu_us, 3)},
        "c3": {"gb_per_s": round(gbs8, 1), "us_per_step": round(ms8 * 1e3, 2),
               "us_per_layer": round(ms8 * 1e3 / L, 2), "hbm_fraction": round(gbs8 * 1e9 / HBM_PEAK, 4),
               "distinct_experts_per_layer": round(distinct / L, 2)},
        "decode_status": {"m1": st1, "m8": st8},
        "clock": {"source": "amdsmi current_gfxclks (mean over the XCDs), sampled every 2 ms in the timed "
                            "region; MHz", "regions": clocks},
    }

    # ---- C4 prefill ------------------------------------------------------------------------------
    prefill = None
    if args.only == "all":
        T = 4096
        sel_np, w_np = synthetic.zipf_routes(T, E, K)
        counts = np.bincount(sel_np.reshape(-1), minlength=E)
        xb = ax.gen_normal(S_X, T * H, 1.0).view(T, H).to(torch.bfloat16)
        sel_t = torch.from_numpy(sel_np).cuda()
        w_t = torch.from_numpy(w_np).cuda()
        gws = ax.GroupedWorkspace(T, K, E)
        yp = torch.zeros((T, H), device="cuda")
        for _ in range(2):
            ax.expert_ffn_grouped(pools[0], xb, sel_t, w_t, y=yp, workspace=gws)
        torch.cuda.synchronize()
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        clock.start()
        st.record()
        for _ in range(args.prefill_steps):
            ax.expert_ffn_grouped(pools[0], xb, sel_t, w_t, y=yp, workspace=gws)
        en.record()
        torch.cuda.synchronize()
        clocks["c4_prefill"] = clock.stop()
        msp = st.elapsed_time(en) / args.prefill_steps
        flops = T * K * FLOP_PER_SLOT
        tf = flops / (msp * 1e-3) / 1e12
        log(f"C4 prefill: {msp:.3f} ms/layer -> {tf:.1f} TFLOP/s ({100 * tf * 1e12 / BF16_PEAK:.1f}% of bf16 peak)")
        # the form the engine hook runs: an f32 activation as a bf16 pair (three terms for gate/up)
        # (its own output buffer: yp keeps the bf16 run's result for the parity check below)
        xf = ax.gen_normal(S_X + 1, T * H, 1.0, bf16_round=False).view(T, H)
        xh = xf.to(torch.bfloat16)
        xl = (xf - xh.float()).to(torch.bfloat16)
        del xf
        y3 = torch.zeros_like(yp)
        ax.expert_ffn_grouped(pools[0], xh, sel_t, w_t, y=y3, x_lo=xl, workspace=gws)
        torch.cuda.synchronize()
        clock.start()
        st.record()
        for _ in range(args.prefill_steps):
            ax.expert_ffn_grouped(pools[0], xh, sel_t, w_t, y=y3, x_lo=xl, workspace=gws)
        en.record()
        torch.cuda.synchronize()
        clocks["c4_prefill_hi_lo"] = clock.stop()
        msp3 = st.elapsed_time(en) / args.prefill_steps
        tf3 = flops / (msp3 * 1e-3) / 1e12
        del xh, xl, y3
        log(f"C4 prefill, hi/lo input (the engine hook's form): {msp3:.3f} ms/layer -> {tf3:.1f} TFLOP/s")
        result["prefill"] = {"tflop_per_s": round(tf, 1), "ms_per_layer": round(msp, 4),
                             "frac_of_bf16_peak": round(tf * 1e12 / BF16_PEAK, 4),
                             "tokens_per_s": round(T / (msp * 1e-3), 1), "flop_per_layer": flops,
                             "hi_lo_input": {"tflop_per_s": round(tf3, 1), "ms_per_layer": round(msp3, 4),
                                             "frac_of_bf16_peak": round(tf3 * 1e12 / BF16_PEAK, 4)},
                             "expert_counts": {"min": int(counts.min()), "median": float(np.median(counts)),
                                               "max": int(counts.max())}}
        prefill = (sel_np, w_np, xb, yp)

    # ---- the step after: the FP8 shared expert (V4-Flash: hidden 4096, inter 2048) ---------------
    # one expert per layer, L layers resident (1.1 GB: none is served from the 256 MB last-level
    # cache when the next token comes), batch-1 decode in a graph like C5, then one 4096-token chunk
    shared = None
    if args.only == "all":
        gen = torch.Generator(device="cuda")
        gen.manual_seed(S_SHEXP)

        def fp8(rows, cols):
            w = torch.randint(0, 256, (rows, cols), dtype=torch.uint8, device="cuda", generator=gen)
            w[(w & 0x7F) == 0x7F] ^= 1          # no NaN codes (the reference decodes them as NaN)
            s = torch.randint(116, 124, (rows // 128, cols // 128), dtype=torch.uint8, device="cuda",
                              generator=gen)
            return w, s

        sh_mats0 = None
        shexps = []
        for l in range(L):
            mats = [fp8(I, H), fp8(I, H), fp8(H, I)]
            if l == 0:
                sh_mats0 = [(w.cpu().numpy(), s.cpu().numpy()) for w, s in mats]
            shexps.append(ax.SharedExpert(*[a for m in mats for a in m]))
            del mats
        sh_bytes = 3 * I * H + 3 * (I // 128) * (H // 128)
        ys = torch.zeros((L, H), device="cuda")
        sws = torch.empty(int(lib().affx_shared_decode_workspace_size(1, H, I)), dtype=torch.uint8, device="cuda")

        def shared_step():
            s = torch.cuda.current_stream().cuda_stream
            for l in range(L):
                check(lib().affx_shared_expert_decode(C.byref(shexps[l].abi), x1.data_ptr(), H, 1, 1,
                                                      ys[l].data_ptr(), H, 1, 0, sws.data_ptr(), sws.numel(), s),
                      "shared_expert_decode")
            return ys

        ms_sh, _, _ = time_graph(torch, shared_step, args.steps, args.warmup, clock, "shared_decode", clocks)
        gbs_sh = L * sh_bytes / (ms_sh * 1e-3) / 1e9
        T = 4096
        xs_b = ax.gen_normal(S_X, T * H, 1.0).view(T, H).to(torch.bfloat16)
        yb = torch.zeros((T, H), device="cuda")
        shexps[0].batch(xs_b, yb, accumulate=False)
        torch.cuda.synchronize()
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.record()
        for l in range(args.prefill_steps):
            shexps[l % L].batch(xs_b, yb, accumulate=False)
        en.record()
        torch.cuda.synchronize()
        ms_shb = st.elapsed_time(en) / args.prefill_steps
        shexps[0].batch(xs_b, yb, accumulate=False)   # layer 0's result for the parity check
        torch.cuda.synchronize()
        tf_shb = T * 2 * 3 * I * H / (ms_shb * 1e-3) / 1e12
        log(f"shared expert: decode {ms_sh * 1e3 / L:.2f} us/layer -> {gbs_sh:.0f} GB/s "
            f"({100 * gbs_sh * 1e9 / HBM_PEAK:.1f}% of HBM peak); {T}-token chunk {ms_shb:.3f} ms -> "
            f"{tf_shb:.1f} TFLOP/s")
        result["shared_expert"] = {
            "workload": f"FP8 shared expert (hidden {H}, inter {I}, UE8M0 128x128 tile scales), one per layer "
                        f"x {L} layers; batch-1 decode in a graph, and one {T}-token bf16 chunk",
            "decode_us_per_layer": round(ms_sh * 1e3 / L, 3), "decode_gb_per_s": round(gbs_sh, 1),
            "decode_hbm_fraction": round(gbs_sh * 1e9 / HBM_PEAK, 4), "bytes_per_layer": sh_bytes,
            "batch_ms": round(ms_shb, 4), "batch_tflop_per_s": round(tf_shb, 1),
            "batch_frac_of_bf16_peak": round(tf_shb * 1e12 / BF16_PEAK, 4)}
        toks = np.array([0, 1, 1000, 2047, 4095])
        shared = (sh_mats0, x1.cpu().numpy()[0], ys[0].cpu().numpy(), xs_b.float().cpu().numpy()[toks],
                  yb.cpu().numpy()[toks])
        del shexps, xs_b, yb, ys, sws

    # ---- the codebook producer: the config-1 recipe fitted on the GPU ----------------------------
    producer_exact = None
    producer_sample = None
    if args.only == "all":
        import affinity_amd.codebook as cbk
        mats = [ax.gen_normal(1000, I * H, 0.02).view(I, H), ax.gen_normal(1001, I * H, 0.02).view(I, H),
                ax.gen_normal(1002, H * I, 0.02).view(H, I)]
        torch.cuda.synchronize()
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.record()
        samples = torch.cat([cbk.collect_normalized_samples(m, 1 << 19) for m in mats])
        en.record()
        torch.cuda.synchronize()
        ms_collect = st.elapsed_time(en)
        fitter = cbk.CodebookFit(samples.numel())
        st.record()
        cbf = fitter.fit(samples, 50, 1)
        packed = cbk.pack_codebook_e4m3_quads(cbk.project_codebook_e4m3(cbf))
        en.record()
        torch.cuda.synchronize()
        ms_fit = st.elapsed_time(en)
        seq_draws, passes = fitter.stats()
        producer_exact = bool(np.array_equal(packed.cpu().numpy().view(np.uint32), cb_packed))
        # a bounded sample of the same samples for the CPU comparison (the CPU baseline leg)
        sub = samples[: 1 << 16].contiguous()
        fit_sub = cbk.CodebookFit(sub.numel())
        fit_sub.fit(sub, 50, 1)
        torch.cuda.synchronize()
        st.record()
        cb_sub = fit_sub.fit(sub, 50, 1)
        en.record()
        torch.cuda.synchronize()
        producer_sample = (sub.cpu().numpy(), cb_sub.cpu().numpy().reshape(-1), st.elapsed_time(en))
        log(f"config-1 codebook on the GPU: collect {ms_collect:.1f} ms, fit + project + pack {ms_fit:.1f} ms, "
            f"{passes} Lloyd passes, {seq_draws} sequential draws, equal to the reference's: {producer_exact}")
        result["producer"] = {"workload": "config-1 codebook: 3 x 2^19 samples, fit_codebook(50, seed 1), "
                                          "projection and packing",
                              "collect_ms": round(ms_collect, 2), "fit_project_pack_ms": round(ms_fit, 2),
                              "lloyd_passes": passes, "sequential_draws": seq_draws,
                              "bit_exact_vs_reference": producer_exact}
        del mats, samples, fitter, cbf, packed, sub, fit_sub, cb_sub

    # ---- CPU baseline (and the checker of the GPU results) ----------------------------------------
    if not args.no_cpu_baseline:
        gpu = {"c1_dequant": [ax.dequant_matrix(pools[0], 0, m).cpu().numpy() for m in range(3)],
               "x1": x1.cpu().numpy()[0], "x8": x8.cpu().numpy(),
               "routes1": [(r[0].cpu().numpy(), r[1].cpu().numpy()) for r in routes1],
               "routes8": (routes8[0][0].cpu().numpy(), routes8[0][1].cpu().numpy()),
               "y1": y1.cpu().numpy(), "y8": y8[0].cpu().numpy()}
        if prefill is not None:
            sel_np, w_np, xb, yp = prefill
            toks, _, _ = synthetic.prefill_sample(sel_np, E)
            gpu["c4"] = (sel_np, w_np, xb.float().cpu().numpy()[toks], yp.cpu().numpy()[toks], toks)
        if producer_sample is not None:
            gpu["fit"] = producer_sample
        if shared is not None:
            gpu["shared"] = shared
        result["cpu_baseline"], result["parity"] = cpu_baseline(ax, cont, gpu, L)
        # every GPU result checked against the CPU path must be within the path's 1e-3 (the dequant
        # bit-exact): a number measured on a wrong result is not a measurement
        def failed(v) -> bool:
            return (not v) if isinstance(v, bool) else (isinstance(v, float) and not v <= 1e-3)
        if producer_exact is not None:
            result["parity"]["c1_codebook_fit_bit_exact"] = producer_exact
        bad = [k for k, v in result["parity"].items() if failed(v)]
        result["parity_ok"] = not bad
        if bad:
            log(f"PARITY FAILED: {bad}")
    print(json.dumps(result), flush=True)
    return 0 if result.get("parity_ok", True) else 1


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(ax, cont, gpu, L):
    """The reference's CPU path (else the oracle restating it) on bounded samples of every config
    timed on this host; returns (cpu_baseline, parity). The samples:
      C1  dequantize_matrix of the config-1 expert (1 thread); its FFN at 1 and all threads
      C2  one token through layer 0's 6 routed experts (1 and all threads): the reported value
      C5  the same for layer L-1; ms per token over L layers = L x the mean token-layer time
      C3  the 8-token layer 0 (48 routed expert FFNs)
      C4  64 sampled prefill tokens, extrapolated linearly to the 4096-token layer
    The same outputs are the checker of the GPU's (rel L2; dequant bit for bit)."""
    from oracle import load_oracle, load_ref, ref_available
    _, off, size = ax.expert_layout()
    cbf = ax.codebook_floats(synthetic.c1_codebook()).reshape(-1)
    kind = "reference" if ref_available() else "port"
    lib = load_ref() if kind == "reference" else load_oracle()
    if kind == "reference":
        n_all = lib.pool_threads()
    else:
        n_all = min(os.cpu_count() or 1, 16)
    cache = {}

    def expert(e):
        e = int(e)
        if e not in cache:
            cache[e] = synthetic.expert_bytes(cont, e, STRIDE)
        return cache[e]

    def planes(ex, m):
        return (np.ascontiguousarray(ex[off[3 * m]:off[3 * m] + size[3 * m]]),
                np.ascontiguousarray(ex[off[3 * m + 1]:off[3 * m + 1] + size[3 * m + 1]]),
                np.ascontiguousarray(ex[off[3 * m + 2]:off[3 * m + 2] + size[3 * m + 2]]).view(np.uint16))

    def ffn(ex, x, wt, y, mt):
        """y += wt * FFN(x): src/engine/model.cpp:1187-1198 over the reference's GEMV."""
        if kind == "reference":
            g = lib.gemv(*planes(ex, 0), I, H, cbf, x, 1.0, mt=mt)
            u = lib.gemv(*planes(ex, 1), I, H, cbf, x, 1.0, mt=mt)
            a = lib.swiglu(g, u, 10.0)
            lib.gemv(*planes(ex, 2), H, I, cbf, a, float(wt), y, mt=mt)
        else:
            lib.set_threads(n_all if mt else 1)
            lib.expert_ffn(ex, cbf, x, float(wt), 10.0, y)
        return y

    def token(x, sel, w, mt):
        y = np.zeros(H, np.float32)
        for e, wt in zip(sel, w):
            ffn(expert(e), x, wt, y, mt)
        return y

    def timed(fn, reps):
        fn()                                   # warm-up (and the result)
        t0 = time.perf_counter()
        for _ in range(reps):
            out = fn()
        return (time.perf_counter() - t0) / reps, out

    x1 = gpu["x1"]
    ex0 = expert(0)
    # C1: dequant (1 thread) and one expert FFN
    dims = ((I, H), (I, H), (H, I))
    if kind == "reference":
        t_deq, deq = timed(lambda: [lib.dequantize(*planes(ex0, m), *dims[m], cbf) for m in range(3)], 3)
    else:
        lib.set_threads(1)
        t_deq, deq = timed(lambda: [lib.dequantize(*planes(ex0, m), *dims[m], cbf) for m in range(3)], 3)
    deq_exact = all(np.array_equal(a.view(np.uint32), b.view(np.uint32)) for a, b in zip(deq, gpu["c1_dequant"]))
    t_c1_1, _ = timed(lambda: ffn(ex0, x1, 1.0, np.zeros(H, np.float32), False), 5)
    t_c1_n, _ = timed(lambda: ffn(ex0, x1, 1.0, np.zeros(H, np.float32), True), 5)
    # C2 (layer 0) at 1 and all threads, C5's last layer
    s0, w0 = gpu["routes1"][0][0][0], gpu["routes1"][0][1][0]
    t_c2_1, y_c2 = timed(lambda: token(x1, s0, w0, False), 3)
    t_c2_n, _ = timed(lambda: token(x1, s0, w0, True), 5)
    sl, wl = gpu["routes1"][L - 1][0][0], gpu["routes1"][L - 1][1][0]
    t_c5_n, y_c5 = timed(lambda: token(x1, sl, wl, True), 3)
    # C3: eight tokens of layer 0
    s8, w8 = gpu["routes8"]
    t_c3_n, y_c3 = timed(lambda: np.stack([token(gpu["x8"][t], s8[t], w8[t], True) for t in range(8)]), 2)
    out = {"kind": kind, "unit": "GB/s",
           "sample": "C2: 1 token x the 6 routed experts of layer 0 (one token-layer), all threads",
           "cores": n_all, "cpu_model": cpu_model(), "hardware_concurrency": os.cpu_count(),
           "value": round(6 * STRIDE / t_c2_n / 1e9, 3),
           "ms_per_token_layer": round(t_c2_n * 1e3, 2),
           "single_thread": {"value": round(6 * STRIDE / t_c2_1 / 1e9, 4), "cores": 1,
                             "ms_per_token_layer": round(t_c2_1 * 1e3, 1)},
           "c1": {"dequant_ms_1thread": round(t_deq * 1e3, 1),
                  "dequant_gb_per_s_1thread": round(STRIDE / t_deq / 1e9, 3),
                  "ffn_ms_1thread": round(t_c1_1 * 1e3, 2), "ffn_ms_all": round(t_c1_n * 1e3, 2),
                  "ffn_gb_per_s_all": round(STRIDE / t_c1_n / 1e9, 3)},
           "c3_ms_per_layer_all": round(t_c3_n * 1e3, 1),
           "c5_ms_per_token_all": round(L * (t_c2_n + t_c5_n) / 2 * 1e3, 1)}
    parity = {"c1_dequant_bit_exact": deq_exact,
              "c2_layer0_rel_l2": rel_l2(gpu["y1"][0], y_c2),
              f"c5_layer{L - 1}_rel_l2": rel_l2(gpu["y1"][L - 1], y_c5),
              "c3_layer0_rel_l2": rel_l2(gpu["y8"], y_c3)}
    msg = (f"CPU baseline ({kind}, {n_all} threads): C1 dequant {t_deq * 1e3:.0f} ms, C1 FFN "
           f"{t_c1_1 * 1e3:.1f} / {t_c1_n * 1e3:.1f} ms; C2 {t_c2_1 * 1e3:.0f} / {t_c2_n * 1e3:.1f} ms per "
           f"token-layer; C3 {t_c3_n * 1e3:.0f} ms per layer")
    if "c4" in gpu:
        sel_np, w_np, xs, yg, toks = gpu["c4"]
        t0 = time.perf_counter()
        yc = np.stack([token(xs[i], sel_np[t], w_np[t], True) for i, t in enumerate(toks)])
        t_c4 = time.perf_counter() - t0
        out["c4"] = {"tokens_timed": len(toks), "ms_sample": round(t_c4 * 1e3, 1),
                     "ms_per_layer_extrapolated": round(t_c4 * 4096 / len(toks) * 1e3, 0),
                     "note": "per-token GEMV path, 64 sampled tokens, extrapolated linearly to 4096"}
        parity["c4_sample_rel_l2"] = rel_l2(yg, yc)
        parity["c4_sample_worst_token_rel_l2"] = max(rel_l2(yg[i], yc[i]) for i in range(len(toks)))
        msg += f"; C4 {len(toks)} tokens {t_c4:.1f} s"
    if "fit" in gpu:
        # the codebook fit on 2^16 of the config-1 samples (50 iterations, seed 1), one run
        fs, cb_gpu, ms_gpu = gpu["fit"]
        t0 = time.perf_counter()
        cb_cpu = lib.fit_codebook(fs, 50, 1, project=False) if kind == "reference" else lib.fit_codebook(fs, 50, 1)
        t_fit = time.perf_counter() - t0
        out["producer"] = {"sample": f"fit_codebook on {fs.size} of the config-1 samples, 50 iterations, seed 1",
                           "cpu_s": round(t_fit, 2), "gpu_ms": round(ms_gpu, 2),
                           "cpu_threads": 1 if kind == "reference" else n_all}
        parity["fit_sample_bit_exact"] = bool(np.array_equal(cb_cpu.view(np.uint32), cb_gpu.view(np.uint32)))
        msg += f"; fit of {fs.size} samples {t_fit:.1f} s (GPU {ms_gpu:.1f} ms)"
    if "shared" in gpu:
        # the shared expert of layer 0: the host composition (src/engine/model.cpp:1214-1222) over
        # the reference's FP8 matvec, for the decode token and five tokens of the 4096-token chunk
        ((wg, sg), (wu, su), (wd, sd)), xd, yd, xb, yb = gpu["shared"]

        def shexp(x):
            g, u = lib.matvec_fp8(wg, sg, x), lib.matvec_fp8(wu, su, x)
            return lib.matvec_fp8(wd, sd, lib.swiglu(g, u, 10.0))

        t_sh, y_sh = timed(lambda: shexp(xd), 3)
        out["shared_expert"] = {"sample": "layer 0's shared expert on the decode token (three FP8 matvecs)",
                                "ms_per_token_layer": round(t_sh * 1e3, 2),
                                "gb_per_s": round(3 * I * H / t_sh / 1e9, 3)}
        parity["shared_expert_decode_rel_l2"] = rel_l2(yd, y_sh)
        parity["shared_expert_batch_sample_rel_l2"] = rel_l2(yb, np.stack([shexp(x) for x in xb]))
        msg += f"; shared expert {t_sh * 1e3:.1f} ms per token-layer"
    parity = {k: (round(v, 9) if isinstance(v, float) else v) for k, v in parity.items()}
    log(msg)
    log(f"parity vs the CPU path: {parity}")
    return out, parity


if __name__ == "__main__":
    sys.exit(main())
