#!/usr/bin/env python3
"""Headline benchmark of the Gated DeltaNet hot paths on one MI355X.

Metric (the brief's): prefill tokens/s at T=8192 + decode steps/s at B=256,
with the achieved MFMA / HBM roofline fractions.  Every one of the brief's
five configs gets a line in the same JSON object, each with its throughput,
its roofline fraction, the CPU oracle (a restatement of the reference's
PyTorch code, oracle/) timed on this host on the same inputs, and the
same-run parity of the GPU results against that oracle:

* primary line (``value``): chunked prefill, B=1, T=8192, H=16, dk=dv=128,
  chunk 64, zero initial state, seeded synthetic bf16 inputs already resident
  in HBM.  One step = one ``prefill.prefill`` call (all kernels).
  ``roofline``: the prefill's state phase (the GEMM phases: map, scan and
  output kernels, one ``gdn_prefill_state_hip`` call) against bf16 MFMA
  peak, with the algorithmic state-recurrence FLOPs; durations come from HIP
  events around per-phase launches on the stream the kernels run on.
* ``prefill_cfg2``: config 2, B=1, T=2048, H=16.
* ``prefill_batches``: the metric prefill at B=4 and B=8 (timing only).
* ``prefill_sweep``: the reference's prefill sweep (bench/bench_prefill.py:
  67-104), B in {1, 8, 32, 64} x T in {2048, 4096, 8192} at H=16,
  dk=dv=128 (timing only, inputs drawn on the GPU).
* ``prefill_varlen``: config 4, 8 packed sequences, lengths U[512, 8192]
  (seed 3), nonzero initial states.
* ``decode``: config 3, B=256, H=32, dk=dv=128, one 512 MiB fp32 state
  updated in place, 100 consecutive steps with fresh q/k/v/a/b per step.
* ``layer_e2e``: config 5, the whole layer (RMSNorm, fused projection + conv
  + SiLU, prefill, output projection) at B=4 x T=4096, then decode steps at
  B=4 continuing from the prefill state.
* ``layer_packed``: the layer forward over config 4's 8 packed sequences at
  config-5 dims (one packed in-projection launch, the packed prefill, W_o).
* ``layer_decode_batches``: the layer's decode step at config-5 dims for
  B = 1, 8, 32, 64, 128, 256 (the reference's serving sweep), HBM roofline
  per B, parity against the oracle layer at B=256.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]
                    [--no-extra] [--only prefill,cfg2,batches,sweep,varlen,decode,layer,packed,serve]
"""

import argparse
import json
import math
import os
import platform
import sys
import time

# ---- algorithmic work (per unit), kept next to the formulas they come from ----
C, K, V = 64, 128, 128
PREFILL_FLOP_PER_TOKEN_HEAD = 2 * (3 * C * K + 2 * C * V + 3 * K * V)       # 180,224: whole path
STATE_FLOP_PER_TOKEN_HEAD = 2 * (3 * K * V + 2 * C * V)                      # 131,072: state kernels
INTRA_FLOP_PER_TOKEN_HEAD = 2 * (2 * C * K)                                  # 32,768: intra kernel


def prefill_bytes(ntok, H, nseq, has_state=False):
    """Algorithmic HBM bytes of one prefill (bf16 q,k,v,o,a,b; fp32 mask, states)."""
    return ntok * H * (2 * (2 * K + V) + 2 * V + 4) + 4 * ntok + 4 * nseq * H * K * V * (1 + int(has_state))


def decode_bytes(B, H):
    """Algorithmic HBM bytes of one decode step: S read + write, q,k,v,a,b, o, A_log, dt_bias."""
    return B * H * (8 * K * V + 2 * (2 * K + V) + 4 * V + 4) + 8 * H


PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
LEGS = ("prefill", "cfg2", "batches", "sweep", "varlen", "decode", "layer", "packed", "serve")


def measured_traffic(kernel):
    """HBM bytes per dispatch of `kernel` from profiles/hbm_traffic.json (rocprofv3 --pmc runs), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)["kernels"][kernel]["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def time_events(fn, iters, torch):
    """Average ms per call of fn() over iters calls, HIP events on the current stream."""
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / iters


class DeviceSettle:
    """Unrelated GPU work run before each timed leg: bf16 8192 x 8192 x 8192
    GEMMs and 256 MiB copies for ``ms`` milliseconds, so that the device's
    power management is in its loaded state when the leg's own warm-up
    starts.  Measured on MI355X after 3 s idle: the B=1, T=8192 prefill's
    first 100 calls average 88.6 us and the calls after the first ~200 run
    81.8 us; B=8, T=8192 goes 0.45 -> 0.373 ms over its first ~60 calls; and
    300 ms of this load before 5 warm-up + 20 timed calls gives the settled
    figures (80 us, 0.37 ms) where no load gives 87 us and 0.45 ms.  None of
    it touches a leg's inputs, outputs or kernels."""

    def __init__(self, torch, dev, ms):
        self.torch, self.ms = torch, ms
        if ms > 0:
            self.a = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
            self.b = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
            self.src = torch.ones(64 << 20, device=dev)
            self.dst = torch.empty_like(self.src)

    def __call__(self):
        if self.ms <= 0:
            return
        t0 = time.perf_counter()
        while (time.perf_counter() - t0) * 1e3 < self.ms:
            for _ in range(4):
                self.torch.matmul(self.a, self.b)
                self.dst.copy_(self.src)
            self.torch.cuda.synchronize()

    def describe(self):
        return {"ms": self.ms, "load": "bf16 8192^3 GEMMs + 256 MiB copies (unrelated buffers), before each timed "
                                       "leg's warm-up"}


def time_cpu(fn, reps):
    """Seconds per call of fn() after one warm-up call, and the warm-up's result."""
    res = fn()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    return (time.perf_counter() - t0) / reps, res


def out_parity(out, ref, atol=2e-2, rtol=2e-2):
    """The brief's bf16 bar: max |diff|, whether allclose(atol, rtol) holds, and the
    error relative to the output's scale (max |diff| / max |ref|)."""
    o, r = out.float().cpu(), ref.float().cpu()
    d = (o - r).abs()
    return {"max_abs_err": d.max().item(), "within_2e-2": bool((d <= atol + rtol * r.abs()).all()),
            "max_err_over_max_ref": d.max().item() / max(r.abs().max().item(), 1e-30)}


def rel_fro(x, ref):
    x, ref = x.double().cpu(), ref.double().cpu()
    return ((x - ref).norm() / ref.norm()).item()


def roofline_fracs(flop, nbytes, ms):
    """Achieved MFMA and HBM fractions of a timed call from its algorithmic work."""
    tf = flop / (ms / 1e3) / 1e12
    gbs = nbytes / (ms / 1e3) / 1e9
    return {"tflops": tf, "mfma_frac": tf / PEAK_BF16_TFLOPS, "gbs": gbs, "hbm_frac": gbs / PEAK_HBM_GBS}


def packed_leg(exts, dev, cpu, nthr, torch, args, settle):
    """GDNLayerCustom.forward(x, cu_seqlens=...) on config 4's 8 packed lengths
    (U[512, 8192], seed 3) at config 5's dims: RMSNorm, one packed in-projection
    launch (+ conv + SiLU, per-sequence conv caches), the packed prefill and the
    W_o GEMM.  MFMA roofline on the layer's algorithmic FLOPs (projections and
    the prefill's per token-head count); parity: sequence 0 against the oracle
    layer run on it alone (fp32 projection)."""
    from gdn_18646_amd import synth
    from gdn_18646_amd.gdn_layer import GDNLayerCustom, make_weights
    LD, LH = 2048, 16
    lengths = synth.varlen_lengths(8, 512, 8192, seed=3)
    Tt = sum(lengths)
    gp = torch.Generator().manual_seed(7)
    w_cpu = make_weights(device="cpu", D=LD, H=LH, DK=128, DV=128, std=0.02, generator=gp)
    layer = GDNLayerCustom({k: v.to(dev) for k, v in w_cpu.items()}, exts)
    x_cpu = torch.randn(1, Tt, LD, generator=gp).bfloat16()
    x = x_cpu.to(dev)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    y = layer.forward(x, cu_seqlens=cu)
    settle()
    layer.forward(x, cu_seqlens=cu)
    ms = time_events(lambda: layer.forward(x, cu_seqlens=cu), max(3, args.steps // 4), torch)
    ncols = 2 * LH * 128 + LH * 128 + 2 * LH
    flop = 2 * Tt * LD * ncols + PREFILL_FLOP_PER_TOKEN_HEAD * Tt * LH + 2 * Tt * LH * 128 * LD
    nbytes = 2 * Tt * LD * 2 + 2 * ncols * LD + 2 * LD * LH * 128 + prefill_bytes(Tt, LH, len(lengths)) - 4 * Tt
    leg = {"config": f"config 4's lengths {lengths} packed ({Tt} tokens), config 5's layer dims (hidden 2048, H=16, "
                     "dk=dv=128, conv 4, weights N(0, 0.02)), zero initial state",
           "ms": ms, "tokens_per_s": Tt / (ms / 1e3), **roofline_fracs(flop, nbytes, ms), "flop": flop, "bytes": nbytes}
    log(f"layer packed forward ({Tt} tokens, 8 sequences): {ms:.3f} ms, {Tt / (ms / 1e3):.4g} tok/s, "
        f"{leg['mfma_frac'] * 100:.1f}% of MFMA peak")
    from oracle.layer_ref import GDNLayerBaseline
    y0 = y[:, :lengths[0]].cpu()
    y_ref = GDNLayerBaseline(w_cpu, chunk_size=C, fp32_proj=True).forward(x_cpu[:, :lengths[0]])
    leg["parity_seq0_vs_oracle_fp32_proj"] = {**out_parity(y0, y_ref), "rel_fro": rel_fro(y0, y_ref)}
    log(f"  packed layer parity {leg['parity_seq0_vs_oracle_fp32_proj']}")
    return leg


def serve_leg(exts, dev, cpu, nthr, torch, settle):
    """GDNLayerCustom.decode at B in {1, 8, 32, 64, 128, 256}, config-5 dims (the
    reference's layer decode sweep, bench_gdn.py:332-342): one step = RMSNorm,
    q/k/v/a/b projection + conv step, the recurrence (state in place), W_o.
    B <= 16 runs the fused step with the skinny projection kernels, larger B
    the fused step with the tiled projection kernels (RMSNorm, tiled
    in-projection + conv step, recurrence, tiled out-projection).  Roofline: HBM, algorithmic bytes per step = both
    weight matrices + the fp32 state read and written + x in and y out.
    Parity at B=256: two steps from the same state against the oracle layer's
    decode (fp32 projection), which is also the CPU baseline."""
    from gdn_18646_amd.gdn_layer import GDNLayerCustom, make_weights
    LD, LH = 2048, 16
    gs = torch.Generator().manual_seed(6)
    w_cpu = make_weights(device="cpu", D=LD, H=LH, DK=128, DV=128, std=0.02, generator=gs)
    layer = GDNLayerCustom({k: v.to(dev) for k, v in w_cpu.items()}, exts)
    ncols = 2 * LH * 128 + LH * 128 + 2 * LH
    wbytes = 2 * ncols * LD + 2 * LD * LH * 128

    def state_for(SB):
        st = {k: v.cpu() for k, v in layer.init_decode_state(SB).items()}
        st["recurrent"].normal_(0.0, 0.02, generator=gs)
        for key in ("conv_q", "conv_k", "conv_v", "xn"):
            st[key].copy_(torch.randn(st[key].shape, generator=gs) * 0.5)
        return st

    leg = {"config": "GDNLayerCustom.decode, hidden 2048, H=16, dk=dv=128, conv 4, weights N(0, 0.02), fp32 state "
                     "N(0, 0.02) updated in place, fresh x N(0, 1) each step",
           "bytes_per_step": "2 (W_qkvab + W_o) + B H 128 128 4 x 2 (state read + write) + 4 B D (x, y)"}
    for SB in (1, 8, 32, 64, 128, 256):
        st = {k: v.to(dev) for k, v in state_for(SB).items()}
        xs = [torch.randn(SB, 1, LD, generator=gs).bfloat16().to(dev) for _ in range(8)]
        it = iter(range(10 ** 9))

        def step():
            layer.decode(xs[next(it) % len(xs)], st, inplace=True)

        settle()
        for _ in range(3):
            step()
        ms = time_events(step, 100 if SB <= 64 else 50, torch)
        nbytes = wbytes + SB * LH * 128 * 128 * 4 * 2 + 4 * SB * LD
        leg[f"B{SB}"] = {"ms_per_step": ms, "steps_per_s": 1e3 / ms, "tokens_per_s": SB * 1e3 / ms,
                         "gbs": nbytes / (ms * 1e6), "hbm_frac": nbytes / (ms * 1e6) / PEAK_HBM_GBS,
                         "bytes": nbytes,
                         "path": ("fused step (skinny projections)" if SB <= 16 and layer.fused_decode else
                                  "fused step (tiled projections)" if SB > 16 and layer.tiled_decode else "unfused")}
        log(f"layer decode B={SB}: {ms * 1e3:.1f} us/step, {nbytes / (ms * 1e6):.0f} GB/s")
        del st, xs
    # parity and CPU baseline at B=256
    SB = 256
    st_cpu = state_for(SB)
    x2 = [torch.randn(SB, 1, LD, generator=gs).bfloat16() for _ in range(2)]
    st = {k: v.to(dev) for k, v in st_cpu.items()}
    ys = []
    for x in x2:
        y, st = layer.decode(x.to(dev), st)
        ys.append(y.cpu())
    torch.cuda.synchronize()
    from oracle.layer_ref import GDNLayerBaseline
    base = GDNLayerBaseline(w_cpu, fp32_proj=True)
    st_ref, ys_ref, secs = st_cpu, [], []
    for x in x2:
        t0 = time.perf_counter()
        y_ref, st_ref = base.decode(x, st_ref)
        secs.append(time.perf_counter() - t0)
        ys_ref.append(y_ref)
    y_g, y_r = torch.cat(ys, 1), torch.cat(ys_ref, 1)
    leg["parity_B256_2steps"] = {**out_parity(y_g, y_r), "rel_fro": rel_fro(y_g, y_r),
                                 "state_rel_fro": rel_fro(st["recurrent"], st_ref["recurrent"])}
    if cpu:
        leg["cpu_baseline"] = dict(value=1.0 / secs[-1], unit="steps/s", cores=nthr, kind="port",
                                   sample=f"oracle.layer_ref.GDNLayerBaseline.decode (fp32 projection) at B=256 on "
                                          f"the same state and inputs, second of two steps, {secs[-1] * 1e3:.0f} ms")
    log(f"  layer decode parity {leg['parity_B256_2steps']}")
    return leg


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--decode-steps", type=int, default=100)
    ap.add_argument("--T", type=int, default=8192)
    ap.add_argument("--B", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="only the metric prefill and the config-3 decode")
    ap.add_argument("--only", default="", help="comma list of legs to run: " + ",".join(LEGS))
    ap.add_argument("--settle-ms", type=int, default=300,
                    help="unrelated GPU load (ms) before each timed leg's warm-up; 0 disables")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run 5 device copies of exactly 256 MiB (scale reference for HBM byte counters)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: every box in this setup has a single MI355X and the "
              "GDN hot path needs no collective (heads and sequences shard with no exchange); "
              "run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    legs = set(LEGS)
    if args.no_extra:
        legs = {"prefill", "decode"}
    if args.only:
        legs = {x.strip() for x in args.only.split(",") if x.strip()}
        unknown = legs - set(LEGS)
        if unknown:
            ap.error(f"unknown legs {sorted(unknown)}")
    cpu = not args.no_cpu_baseline

    import torch
    from gdn_18646_amd import abi, compile_kernels, synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    exts = compile_kernels()
    if cpu:
        torch.set_num_threads(os.cpu_count() or 1)
    nthr = torch.get_num_threads()
    cpu_desc = f"{os.cpu_count()} logical CPUs ({cpu_model()})"
    if args.copy_calibration:
        src = torch.ones(64 << 20, device=dev)  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    H = 16
    settle = DeviceSettle(torch, dev, args.settle_ms)
    empty = torch.empty(0, device=dev, dtype=torch.float32)
    pf = exts["prefill"]
    result = {}

    def on_dev(d):
        return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in d.items()}

    def prefill_call(g, state=None):
        return pf.prefill(g["q"], g["k"], g["v"], g["A_log"], g["a"], 0.0, g["b_logits"], g["mask"],
                          empty if state is None else state, 0.0)

    def prefill_oracle(d, reps):
        from oracle.prefill_ref import ref_prefill
        dt_t = torch.tensor(0.0)
        return time_cpu(lambda: ref_prefill(d["q"], d["k"], d["v"], d["A_log"], d["a"], dt_t, d["b_logits"],
                                            d["mask"], state_in=None, scale=0.0, chunk_size=C), reps)

    # ------------------------------------------------------------------ prefill (metric)
    B, T = args.B, args.T
    tok_s = ms_prefill = None
    if "prefill" in legs:
        d = synth.prefill_inputs(B, T, H, K, V, seed=1)
        g = on_dev(d)
        # the same W + K calls first without the settle load (reported beside the value)
        for _ in range(args.warmup):
            prefill_call(g)
        torch.cuda.synchronize()
        ms_unsettled = time_events(lambda: prefill_call(g), args.steps, torch)
        settle()
        for _ in range(args.warmup):
            prefill_call(g)
        torch.cuda.synchronize()
        ms_prefill = time_events(lambda: prefill_call(g), args.steps, torch)
        result["device_settle"] = {**settle.describe(), "metric_ms_per_step_without": ms_unsettled}
        out_gpu, S_gpu = prefill_call(g)
        torch.cuda.synchronize()

        # per-phase kernel timing through the C ABI (same stream as torch's current one)
        ws_bytes = abi.load().gdn_prefill_workspace_bytes(B, H, T, K, V)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        out_ph = torch.empty_like(out_gpu)
        S_ph = torch.empty_like(S_gpu)
        stream = torch.cuda.current_stream().cuda_stream
        ptrs = (g["q"].data_ptr(), g["k"].data_ptr(), g["v"].data_ptr(), g["A_log"].data_ptr(), g["a"].data_ptr(),
                0.0, g["b_logits"].data_ptr(), g["mask"].data_ptr(), None, 0.0, out_ph.data_ptr(), S_ph.data_ptr(),
                B, H, T, K, V, ws.data_ptr(), ws_bytes, stream)
        abi.call("gdn_prefill_hip", *ptrs)
        settle()
        ms_intra = time_events(lambda: abi.call("gdn_prefill_intra_hip", *ptrs), args.steps, torch)
        settle()
        ms_state = time_events(lambda: abi.call("gdn_prefill_state_hip", *ptrs), args.steps, torch)
        del ws, out_ph, S_ph

        tokens = B * T
        tok_s = tokens / (ms_prefill / 1e3)
        state_tflops = STATE_FLOP_PER_TOKEN_HEAD * tokens * H / (ms_state / 1e3) / 1e12
        intra_tflops = INTRA_FLOP_PER_TOKEN_HEAD * tokens * H / (ms_intra / 1e3) / 1e12
        path = roofline_fracs(PREFILL_FLOP_PER_TOKEN_HEAD * tokens * H, prefill_bytes(tokens, H, B), ms_prefill)
        log(f"prefill B={B} T={T} H={H}: {ms_prefill:.4f} ms/step, {tok_s:.4g} tok/s; intra {ms_intra:.4f} ms "
            f"({intra_tflops:.1f} TF/s), state {ms_state:.4f} ms ({state_tflops:.1f} TF/s); "
            f"path {path['tflops']:.1f} TF/s, {path['gbs']:.0f} GB/s")
        result["roofline"] = {
            "bound": "mfma",
            "kernel": "gdn_prefill_state_hip (map + scan + output kernels)",
            "achieved": state_tflops, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": state_tflops / PEAK_BF16_TFLOPS,
            "traffic": measured_traffic("prefill_state") if (B, T) == (1, 8192) else None,
            "flop_per_launch": STATE_FLOP_PER_TOKEN_HEAD * tokens * H, "kernel_ms": ms_state,
        }
        result["prefill_phases"] = {
            "intra_ms": ms_intra, "intra_tflops": intra_tflops, "state_ms": ms_state, "state_tflops": state_tflops,
            "path_tflops": path["tflops"], "path_mfma_frac": path["mfma_frac"],
            "path_gbs": path["gbs"], "path_hbm_frac": path["hbm_frac"],
            "path_flop": PREFILL_FLOP_PER_TOKEN_HEAD * tokens * H, "path_bytes": prefill_bytes(tokens, H, B),
        }
        if cpu:
            sec, (o_ref, S_ref) = prefill_oracle(d, 3)
            result["cpu_baseline"] = dict(
                value=tokens / sec, unit="tokens/s", cores=nthr, kind="port",
                sample=f"oracle.prefill_ref.ref_prefill (float32 torch CPU) on the same B={B} T={T} H={H} inputs, "
                       f"1 warm-up + 3 timed calls, {sec * 1e3:.0f} ms/call; {cpu_desc}")
            par = out_parity(out_gpu, o_ref)
            result["parity"] = {"prefill_out_max_abs_err": par["max_abs_err"],
                                "prefill_out_within_2e-2": par["within_2e-2"],
                                "prefill_state_rel_fro": rel_fro(S_gpu, S_ref)}
            log(f"  cpu oracle {sec * 1e3:.0f} ms/call ({nthr} threads); parity {result['parity']}")
        del d, g, out_gpu, S_gpu

    # ------------------------------------------------------------------ config 2: B=1, T=2048
    if "cfg2" in legs:
        d2 = synth.prefill_inputs(1, 2048, H, K, V, seed=1)
        g2 = on_dev(d2)
        settle()
        for _ in range(3):
            prefill_call(g2)
        ms2 = time_events(lambda: prefill_call(g2), args.steps, torch)
        o2, S2 = prefill_call(g2)
        torch.cuda.synchronize()
        leg = {"config": "config 2: B=1, T=2048, H=16, dk=dv=128, seed 1, zero initial state",
               "ms": ms2, "tokens_per_s": 2048 / (ms2 / 1e3),
               **roofline_fracs(PREFILL_FLOP_PER_TOKEN_HEAD * 2048 * H, prefill_bytes(2048, H, 1), ms2)}
        if cpu:
            sec, (o_ref, S_ref) = prefill_oracle(d2, 3)
            leg["cpu_baseline"] = dict(value=2048 / sec, unit="tokens/s", cores=nthr, kind="port",
                                       sample=f"oracle.prefill_ref.ref_prefill on the same inputs, 1 warm-up + 3 "
                                              f"timed calls, {sec * 1e3:.0f} ms/call")
            leg["parity"] = {**out_parity(o2, o_ref), "state_rel_fro": rel_fro(S2, S_ref)}
        result["prefill_cfg2"] = leg
        log(f"prefill cfg2 B=1 T=2048: {ms2:.4f} ms/step, {2048 / (ms2 / 1e3):.4g} tok/s, "
            f"parity {leg.get('parity')}")
        del d2, g2, o2, S2

    # ------------------------------------------------------------ prefill, B = 4 and 8
    if "batches" in legs:
        batches = {}
        for Bx in (4, 8):
            gx = on_dev(synth.prefill_inputs(Bx, T, H, K, V, seed=1))
            settle()
            for _ in range(2):
                prefill_call(gx)
            msx = time_events(lambda: prefill_call(gx), max(3, args.steps // 2), torch)
            batches[f"B{Bx}"] = {"ms": msx, "tokens_per_s": Bx * T / (msx / 1e3),
                                 **roofline_fracs(PREFILL_FLOP_PER_TOKEN_HEAD * Bx * T * H,
                                                  prefill_bytes(Bx * T, H, Bx), msx)}
            log(f"prefill B={Bx} T={T} H={H}: {msx:.4f} ms/step, {Bx * T / (msx / 1e3):.4g} tok/s")
            del gx
        result["prefill_batches"] = batches

    # ----------------------- the reference's prefill sweep, B x T, timing only
    if "sweep" in legs:
        # bench/bench_prefill.py:67-104 (and bench_gdn.py:315-329): B in
        # {1, 8, 32, 64} x T in {2048, 4096, 8192}, here at the metric's
        # H=16, dk=dv=128 with zero initial state; inputs drawn on the GPU.
        sweep = {}
        for Bx in (1, 8, 32, 64):
            for Tx in (2048, 4096, 8192):
                gx = synth.prefill_inputs_on_device(Bx, Tx, H, K, V, seed=5, device=dev)
                settle()
                for _ in range(2):
                    prefill_call(gx)
                msx = time_events(lambda: prefill_call(gx), max(3, min(args.steps, 10)), torch)
                sweep[f"B{Bx}_T{Tx}"] = {"ms": msx, "tokens_per_s": Bx * Tx / (msx / 1e3),
                                         **roofline_fracs(PREFILL_FLOP_PER_TOKEN_HEAD * Bx * Tx * H,
                                                          prefill_bytes(Bx * Tx, H, Bx), msx)}
                log(f"prefill sweep B={Bx} T={Tx}: {msx:.4f} ms, {Bx * Tx / (msx / 1e3):.4g} tok/s, "
                    f"{100 * sweep[f'B{Bx}_T{Tx}']['mfma_frac']:.1f}% MFMA")
                del gx
        sweep["config"] = ("reference sweep bench/bench_prefill.py:67-104 at H=16, dk=dv=128, zero state; "
                           "q,k unit rows, v,a,b N(0,1) bf16, drawn on the GPU (seed 5)")
        result["prefill_sweep"] = sweep

    # ------------------------------------- packed variable-length prefill (config 4)
    if "varlen" in legs:
        lengths = synth.varlen_lengths(8, 512, 8192, seed=3)
        dl = synth.varlen_inputs(lengths, H, K, V, seed=3)
        gl_ = on_dev(dl)

        def step_vl():  # offsets from the host, as a serving loop has them
            return pf.prefill_varlen(gl_["q"], gl_["k"], gl_["v"], gl_["A_log"], gl_["a"], 0.0, gl_["b_logits"],
                                     dl["cu_seqlens"], gl_["state_in"], 0.0)

        settle()
        for _ in range(2):
            step_vl()
        msv = time_events(step_vl, max(3, args.steps // 2), torch)
        ov, Sv = step_vl()
        torch.cuda.synchronize()
        ntok = int(sum(lengths))
        leg = {"config": "config 4: 8 packed sequences, lengths U[512, 8192] (seed 3): " + ",".join(map(str, lengths))
                         + f"; H={H}, dk=dv={K}, nonzero initial states",
               "tokens": ntok, "ms": msv, "tokens_per_s": ntok / (msv / 1e3),
               **roofline_fracs(PREFILL_FLOP_PER_TOKEN_HEAD * ntok * H, prefill_bytes(ntok, H, 8, True), msv)}
        if cpu:
            from oracle.prefill_ref import ref_prefill_varlen
            sec, (o_ref, S_ref) = time_cpu(
                lambda: ref_prefill_varlen(dl["q"], dl["k"], dl["v"], dl["A_log"], dl["a"], 0.0, dl["b_logits"],
                                           dl["cu_seqlens"], state_in=dl["state_in"], chunk_size=C), 1)
            leg["cpu_baseline"] = dict(value=ntok / sec, unit="tokens/s", cores=nthr, kind="port",
                                       sample=f"oracle.prefill_ref.ref_prefill_varlen on the same packed inputs, "
                                              f"1 warm-up + 1 timed call, {sec * 1e3:.0f} ms/call")
            leg["parity"] = {**out_parity(ov, o_ref),
                             "state_rel_fro_max": max(rel_fro(Sv[i], S_ref[i]) for i in range(len(lengths)))}
        result["prefill_varlen"] = leg
        log(f"prefill varlen ({ntok} tokens in 8 sequences): {msv:.4f} ms/call, {ntok / (msv / 1e3):.4g} tok/s, "
            f"parity {leg.get('parity')}")
        del dl, gl_, ov, Sv

    # ------------------------------------------------------------------ decode (config 1)
    if "decode" in legs:
        d1 = synth.decode_inputs(1, 4, K, V, seed=0)
        g1 = {k: v.to(dev) for k, v in d1.items()}
        S1 = g1["S"].clone()
        o1 = torch.empty(1, 4, V, device=dev)
        dec1 = exts["decode"]
        scale1 = K ** -0.5

        def step1():  # the same single step from S0 each time (out of place)
            dec1.forward(g1["q"], g1["k"], g1["v"], g1["a"], g1["b"], g1["A_log"], g1["dt_bias"], g1["S"], scale1,
                         o1, S1)

        settle()
        for _ in range(5):
            step1()
        ms1 = time_events(step1, 200, torch)
        gbs1 = decode_bytes(1, 4) / (ms1 / 1e3) / 1e9
        leg1 = {"config": "config 1: one GDN decode step, B=1 H=4 dk=dv=128, seed 0, S0 ~ N(0, 0.02)",
                "us_per_step": ms1 * 1e3, "steps_per_s": 1e3 / ms1,
                "roofline": {"bound": "hbm", "achieved": gbs1, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                             "frac": gbs1 / PEAK_HBM_GBS, "bytes_per_launch": decode_bytes(1, 4)}}
        if cpu:
            from oracle.decode_ref import ref_decode

            def cpu1():
                return ref_decode(d1["q"].reshape(1, 1, 4, K), d1["k"].reshape(1, 1, 4, K),
                                  d1["v"].reshape(1, 1, 4, V), d1["S"], d1["A_log"], d1["a"].reshape(1, 1, 4),
                                  d1["dt_bias"], d1["b"].reshape(1, 1, 4), scale1)

            sec1, (o1_ref, S1_ref) = time_cpu(cpu1, 200)
            leg1["cpu_baseline"] = dict(value=1 / sec1, unit="steps/s", cores=nthr, kind="port",
                                        sample=f"oracle.decode_ref.ref_decode on the same inputs, 1 warm-up + 200 "
                                               f"timed steps, {sec1 * 1e6:.0f} us/step")
            leg1["parity"] = {"out_max_abs_err": (o1.cpu().reshape(-1) - o1_ref.reshape(-1)).abs().max().item(),
                              "state_rel_fro": rel_fro(S1.cpu(), S1_ref)}
        result["decode_cfg1"] = leg1
        log(f"decode config 1 (B=1 H=4): {ms1 * 1e3:.1f} us/step, parity {leg1.get('parity')}")
        del d1, g1, S1, o1

    # ------------------------------------------------------------------ decode (config 3)
    if "decode" in legs:
        DB, DH = 256, 32
        dd = synth.decode_inputs(DB, DH, K, V, seed=2)
        stream_in = synth.decode_step_stream(args.decode_steps, DB, DH, K, V, seed=2)
        gsteps = [{k: v.to(dev) for k, v in st.items()} for st in stream_in]
        A_log_d, dtb_d = dd["A_log"].to(dev), dd["dt_bias"].to(dev)
        S_dev = dd["S"].to(dev)
        o_dev = torch.empty(DB, DH, V, device=dev)
        dec = exts["decode"]
        scale = K ** -0.5

        # parity leg: 3 steps from S0 on a copy, checked against the oracle below
        S_chk = S_dev.clone()
        o_chk = []
        for st in gsteps[:3]:
            dec.forward(st["q"], st["k"], st["v"], st["a"], st["b"], A_log_d, dtb_d, S_chk, scale, o_dev, S_chk)
            o_chk.append(o_dev.cpu())
        S_chk = S_chk.cpu()

        settle()
        for i in range(max(args.warmup, 1)):
            st = gsteps[i % len(gsteps)]
            dec.forward(st["q"], st["k"], st["v"], st["a"], st["b"], A_log_d, dtb_d, S_dev, scale, o_dev, S_dev)
        it = iter(range(10 ** 9))

        def decode_step():
            st = gsteps[next(it) % len(gsteps)]
            dec.forward(st["q"], st["k"], st["v"], st["a"], st["b"], A_log_d, dtb_d, S_dev, scale, o_dev, S_dev)

        ms_decode = time_events(decode_step, args.decode_steps, torch)
        dec_gbs = decode_bytes(DB, DH) / (ms_decode / 1e3) / 1e9
        log(f"decode B={DB} H={DH}: {ms_decode * 1e3:.1f} us/step, {1e3 / ms_decode:.1f} steps/s, {dec_gbs:.0f} GB/s")
        leg = {
            "value": 1e3 / ms_decode, "unit": "steps/s", "ms_per_step": ms_decode, "steps": args.decode_steps,
            "config": {"workload": "config 3: GDN decode B=256 H=32 dk=dv=128, fp32 state in place, fresh q/k/v "
                                   "each step", "B": DB, "H": DH, "dk": K, "dv": V},
            "dtype": "fp32",
            "roofline": {"bound": "hbm", "kernel": "gdn_decode_kernel", "achieved": dec_gbs, "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": dec_gbs / PEAK_HBM_GBS, "traffic": measured_traffic("decode"),
                         "bytes_per_launch": decode_bytes(DB, DH), "kernel_ms": ms_decode},
            "cpu_baseline": None,
        }
        if cpu:
            from oracle.decode_ref import ref_decode
            S_cpu = dd["S"]
            o_refs = []

            def cpu_dec(st, S):
                return ref_decode(st["q"].reshape(DB, 1, DH, K), st["k"].reshape(DB, 1, DH, K),
                                  st["v"].reshape(DB, 1, DH, V), S, dd["A_log"], st["a"].reshape(DB, 1, DH),
                                  dd["dt_bias"], st["b"].reshape(DB, 1, DH), scale)

            t0 = None
            nd = 5
            for i in range(nd + 1):  # step 0 is the warm-up
                if i == 1:
                    t0 = time.perf_counter()
                o_r, S_cpu = cpu_dec(stream_in[i % len(stream_in)], S_cpu)
                if i < 3:
                    o_refs.append(o_r)
                if i == 2:
                    S_ref3 = S_cpu.clone()
            cpu_dms = (time.perf_counter() - t0) / nd * 1e3
            leg["cpu_baseline"] = dict(value=1e3 / cpu_dms, unit="steps/s", cores=nthr, kind="port",
                                       sample=f"oracle.decode_ref.ref_decode on the same B={DB} H={DH} state and "
                                              f"inputs, 1 warm-up + {nd} timed steps, {cpu_dms:.0f} ms/step")
            leg["parity"] = {"out_max_abs_err": max((a - b).abs().max().item() for a, b in zip(o_chk, o_refs)),
                             "state_rel_fro_3steps": rel_fro(S_chk, S_ref3)}
            result.setdefault("parity", {}).update(
                {"decode_out_max_abs_err": leg["parity"]["out_max_abs_err"],
                 "decode_state_rel_fro_3steps": leg["parity"]["state_rel_fro_3steps"]})
        result["decode"] = leg
        del gsteps, S_dev, S_chk

    # ------------------------------------------------- end-to-end layer (config 5)
    if "layer" in legs:
        from gdn_18646_amd.gdn_layer import GDNLayerCustom, make_weights

        LD, LH, LB, LT = 2048, 16, 4, 4096
        gl = torch.Generator().manual_seed(5)
        w_cpu = make_weights(device="cpu", D=LD, H=LH, DK=128, DV=128, std=0.02, generator=gl)
        wl = on_dev(w_cpu)
        layer = GDNLayerCustom(wl, exts)
        x_cpu = torch.randn(LB, LT, LD, generator=gl).bfloat16()
        xl = x_cpu.to(dev)
        xd = [torch.randn(LB, 1, LD, generator=gl).bfloat16().to(dev) for _ in range(8)]
        y_l, st_l = layer.forward(xl, return_state=True)
        settle()
        layer.forward(xl)
        ms_lf = time_events(lambda: layer.forward(xl), max(3, args.steps // 4), torch)
        it_l = iter(range(10 ** 9))

        def layer_dec():
            layer.decode(xd[next(it_l) % len(xd)], st_l, inplace=True)

        settle()
        for _ in range(3):
            layer_dec()
        ms_ld = time_events(layer_dec, 128, torch)
        ncols = 2 * LH * 128 + LH * 128 + 2 * LH
        lflop = (2 * LB * LT * LD * ncols + PREFILL_FLOP_PER_TOKEN_HEAD * LB * LT * LH + 2 * LB * LT * LH * 128 * LD)
        lbytes = (2 * LB * LT * LD * 2 + 2 * ncols * LD + 2 * LD * LH * 128 +
                  prefill_bytes(LB * LT, LH, LB) - 4 * LB * LT)  # x in, y out, weights, prefill (no mask)
        dbytes = 2 * ncols * LD + 2 * LD * LH * 128 + LB * LH * 8 * 128 * 128 + 4 * LB * LD
        leg = {"config": "config 5: hidden 2048, H=16, dk=dv=128, conv 4, weights N(0, 0.02); prefill B=4 x "
                         "T=4096, then decode steps at B=4 continuing from the prefill state",
               "prefill_ms": ms_lf, "prefill_tokens_per_s": LB * LT / (ms_lf / 1e3),
               "prefill_roofline": {**roofline_fracs(lflop, lbytes, ms_lf), "flop": lflop, "bytes": lbytes},
               "decode_ms_per_step": ms_ld, "decode_steps_per_s": 1e3 / ms_ld,
               "decode_roofline": {**roofline_fracs(0, dbytes, ms_ld), "bytes": dbytes}}
        log(f"layer (config 5): prefill B={LB} T={LT} {ms_lf:.3f} ms ({LB * LT / (ms_lf / 1e3):.4g} tok/s), "
            f"decode B={LB} {ms_ld * 1e3:.1f} us/step")
        # decode == prefill at config 5: 32 decode steps from the prefill state of the
        # first 4064 tokens against the forward over all 4096 (GPU against GPU)
        _, st_full = layer.forward(xl, return_state=True)  # st_l was advanced by the timed decode steps
        _, st_p = layer.forward(xl[:, :LT - 32], return_state=True)
        ys = [layer.decode(xl[:, t:t + 1], st_p, inplace=True)[0] for t in range(LT - 32, LT)]
        torch.cuda.synchronize()
        yd = torch.cat(ys, 1)
        leg["parity"] = {"decode32_vs_prefill": out_parity(yd, y_l[:, LT - 32:]),
                         "decode32_state_rel_fro": rel_fro(st_p["recurrent"], st_full["recurrent"])}
        if cpu:
            from oracle.layer_ref import GDNLayerBaseline
            y0 = y_l[:1].cpu()
            t0 = time.perf_counter()
            GDNLayerBaseline(w_cpu, chunk_size=C).forward(x_cpu[:1])
            sec = time.perf_counter() - t0
            y_ref = GDNLayerBaseline(w_cpu, chunk_size=C, fp32_proj=True).forward(x_cpu[:1])
            leg["cpu_baseline"] = dict(value=LT / sec, unit="tokens/s", cores=nthr, kind="port",
                                       sample="oracle.layer_ref.GDNLayerBaseline.forward (ref_rmsnorm, "
                                              "ref_proj_conv_silu, ref_prefill, W_o) on sequence 0 of the same "
                                              f"input (1 x 4096 tokens), one call, {sec:.2f} s")
            leg["parity"]["forward_seq0_vs_oracle_fp32_proj"] = {**out_parity(y0, y_ref),
                                                                 "rel_fro": rel_fro(y0, y_ref)}
        result["layer_e2e"] = leg
        log(f"  layer parity {leg['parity']}")
        del layer, wl, xl, st_l

    # ------------------------------- packed layer forward (config-4 lengths, config-5 dims)
    if "packed" in legs:
        result["layer_packed"] = packed_leg(exts, dev, cpu, nthr, torch, args, settle)

    # ------------------------------- layer decode at serving batch sizes (config-5 dims)
    if "serve" in legs:
        result["layer_decode_batches"] = serve_leg(exts, dev, cpu, nthr, torch, settle)

    line = {
        "metric": "prefill tokens/s (T=8192) + decode steps/s (B=256); % of MFMA / HBM roofline",
        "value": tok_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_prefill,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded: q,k unit-norm N(0,1), v,a,b N(0,1), A_log=ln0.5, dt_bias=0)",
        "config": {"workload": f"GDN chunked prefill B={B} T={T} H={H} dk=dv=128 chunk=64, zero initial state",
                   "B": B, "T": T, "H": H, "dk": K, "dv": V, "chunk": C},
    }
    line.update(result)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
