#!/usr/bin/env python3
"""Headline benchmark of the Gated DeltaNet hot paths on one MI355X.

Metric (the brief's): prefill tokens/s at T=8192 + decode steps/s at B=256,
with the achieved MFMA / HBM roofline fractions.

* Primary line (``value``): chunked prefill, B=1, T=8192, H=16, dk=dv=128,
  chunk 64, zero initial state, seeded synthetic bf16 inputs already resident
  in HBM.  One step = one ``prefill.prefill`` call (both kernels).
* ``decode``: B=256, H=32, dk=dv=128, one 512 MiB fp32 state updated in place,
  100 consecutive steps with fresh q/k/v/a/b per step (inputs pre-staged).
* ``roofline``: the prefill state phase (the GEMM phase: map, scan and output
  kernels, one ``gdn_prefill_state_hip`` call) against bf16 MFMA peak, with
  the algorithmic state-recurrence FLOPs; ``decode.roofline``: the decode
  kernel against HBM peak.  Durations come from HIP events around per-phase
  launches on the stream the kernels run on.
* ``cpu_baseline``: the CPU oracle (oracle/, a restatement of the reference's
  PyTorch code) timed on this host on the same inputs, and the same-run parity
  of the GPU results against it.
* ``prefill_batches``: the same prefill at B=4 and B=8; ``prefill_varlen``:
  config 3 (8 packed sequences, lengths U[512, 8192], nonzero initial
  states); ``layer_e2e``: the end-to-end layer of config 5 (RMSNorm, fused
  projection + conv + SiLU, prefill, output projection at B=4 x T=4096, then
  decode steps at B=4).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline] [--no-extra]
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
STATE_FLOP_PER_TOKEN_HEAD = 2 * (3 * K * V + 2 * C * V)                      # 131,072: state kernel
INTRA_FLOP_PER_TOKEN_HEAD = 2 * (2 * C * K)                                  # 32,768: intra kernel


def prefill_bytes(B, T, H, has_state=False):
    """Algorithmic HBM bytes of one prefill (bf16 q,k,v,o,a,b; fp32 mask, states)."""
    return B * T * H * (2 * (2 * K + V) + 2 * V + 4) + 4 * B * T + 4 * B * H * K * V * (1 + int(has_state))


def decode_bytes(B, H):
    """Algorithmic HBM bytes of one decode step: S read + write, q,k,v,a,b, o, A_log, dt_bias."""
    return B * H * (8 * K * V + 2 * (2 * K + V) + 4 * V + 4) + 8 * H


PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


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


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--decode-steps", type=int, default=100)
    ap.add_argument("--T", type=int, default=8192)
    ap.add_argument("--B", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the B=4/8 prefill lines, the packed varlen prefill (config 3) and the "
                         "end-to-end layer (config 5) timing")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run 5 device copies of exactly 256 MiB (scale reference for HBM byte counters)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: every box in this setup has a single MI355X and the "
              "GDN hot path needs no collective (heads and sequences shard with no exchange); "
              "run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    from gdn_18646_amd import abi, compile_kernels, synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    exts = compile_kernels()
    if args.copy_calibration:
        src = torch.ones(64 << 20, device=dev)  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    B, T, H = args.B, args.T, 16

    # ------------------------------------------------------------------ prefill
    d = synth.prefill_inputs(B, T, H, K, V, seed=1)
    g = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in d.items()}
    empty = torch.empty(0, device=dev, dtype=torch.float32)
    pf = exts["prefill"]

    def prefill_step():
        return pf.prefill(g["q"], g["k"], g["v"], g["A_log"], g["a"], 0.0, g["b_logits"], g["mask"], empty, 0.0)

    for _ in range(args.warmup):
        prefill_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms_prefill = time_events(prefill_step, args.steps, torch)
    wall_prefill = (time.perf_counter() - t0) / args.steps * 1e3
    out_gpu, S_gpu = prefill_step()
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
    ms_intra = time_events(lambda: abi.call("gdn_prefill_intra_hip", *ptrs), args.steps, torch)
    ms_state = time_events(lambda: abi.call("gdn_prefill_state_hip", *ptrs), args.steps, torch)

    tokens = B * T
    tok_s = tokens / (ms_prefill / 1e3)
    state_tflops = STATE_FLOP_PER_TOKEN_HEAD * tokens * H / (ms_state / 1e3) / 1e12
    intra_tflops = INTRA_FLOP_PER_TOKEN_HEAD * tokens * H / (ms_intra / 1e3) / 1e12
    path_tflops = PREFILL_FLOP_PER_TOKEN_HEAD * tokens * H / (ms_prefill / 1e3) / 1e12
    path_gbs = prefill_bytes(B, T, H) / (ms_prefill / 1e3) / 1e9
    log(f"prefill B={B} T={T} H={H}: {ms_prefill:.4f} ms/step ({wall_prefill:.4f} ms wall), {tok_s:.4g} tok/s; "
        f"intra {ms_intra:.4f} ms ({intra_tflops:.1f} TF/s), state {ms_state:.4f} ms ({state_tflops:.1f} TF/s); "
        f"path {path_tflops:.1f} TF/s, {path_gbs:.0f} GB/s")

    # ------------------------------------------------------------ prefill, B = 4 and 8
    batches = {}
    if not args.no_extra:
        for Bx in (4, 8):
            dx = synth.prefill_inputs(Bx, T, H, K, V, seed=1)
            gx = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in dx.items()}

            def step_x():
                return pf.prefill(gx["q"], gx["k"], gx["v"], gx["A_log"], gx["a"], 0.0, gx["b_logits"], gx["mask"],
                                  empty, 0.0)

            for _ in range(2):
                step_x()
            msx = time_events(step_x, max(3, args.steps // 2), torch)
            batches[f"B{Bx}"] = {"ms": msx, "tokens_per_s": Bx * T / (msx / 1e3),
                                 "path_tflops": PREFILL_FLOP_PER_TOKEN_HEAD * Bx * T * H / (msx / 1e3) / 1e12}
            log(f"prefill B={Bx} T={T} H={H}: {msx:.4f} ms/step, {Bx * T / (msx / 1e3):.4g} tok/s")
            del dx, gx

    # ------------------------------------- packed variable-length prefill (config 3)
    varlen = None
    if not args.no_extra:
        lengths = synth.varlen_lengths(8, 512, 8192, seed=3)
        dl = synth.varlen_inputs(lengths, H, K, V, seed=3)
        gl_ = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in dl.items()}

        def step_vl():  # offsets from the host, as a serving loop has them
            return pf.prefill_varlen(gl_["q"], gl_["k"], gl_["v"], gl_["A_log"], gl_["a"], 0.0, gl_["b_logits"],
                                     dl["cu_seqlens"], gl_["state_in"], 0.0)

        for _ in range(2):
            step_vl()
        msv = time_events(step_vl, max(3, args.steps // 2), torch)
        ntok = int(sum(lengths))
        varlen = {"config": "8 packed sequences, lengths U[512, 8192] (seed 3): " + ",".join(map(str, lengths)) +
                            f"; H={H}, dk=dv={K}, nonzero initial states",
                  "tokens": ntok, "ms": msv, "tokens_per_s": ntok / (msv / 1e3),
                  "path_tflops": PREFILL_FLOP_PER_TOKEN_HEAD * ntok * H / (msv / 1e3) / 1e12}
        log(f"prefill varlen ({ntok} tokens in 8 sequences): {msv:.4f} ms/call, {ntok / (msv / 1e3):.4g} tok/s")
        del dl, gl_

    # ------------------------------------------------------------------ decode
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

    # ------------------------------------------------- end-to-end layer (config 5)
    layer_e2e = None
    if not args.no_extra:
        from gdn_18646_amd.gdn_layer import GDNLayerCustom, make_weights

        gl = torch.Generator().manual_seed(5)
        wl = {k: v.to(dev) for k, v in make_weights(device="cpu", D=2048, H=16, DK=128, DV=128, std=0.02,
                                                     generator=gl).items()}
        layer = GDNLayerCustom(wl, exts)
        LB, LT = 4, 4096
        xl = torch.randn(LB, LT, 2048, generator=gl).bfloat16().to(dev)
        xd = [torch.randn(LB, 1, 2048, generator=gl).bfloat16().to(dev) for _ in range(8)]
        _, st_l = layer.forward(xl, return_state=True)
        ms_lf = time_events(lambda: layer.forward(xl), max(3, args.steps // 4), torch)
        it_l = iter(range(10 ** 9))

        def layer_dec():
            layer.decode(xd[next(it_l) % len(xd)], st_l, inplace=True)

        for _ in range(3):
            layer_dec()
        ms_ld = time_events(layer_dec, 128, torch)
        step_g = layer.capture_decode(st_l)
        it_g = iter(range(10 ** 9))

        def layer_dec_graph():
            step_g(xd[next(it_g) % len(xd)])

        for _ in range(3):
            layer_dec_graph()
        ms_ldg = time_events(layer_dec_graph, 128, torch)
        layer_e2e = {"config": "hidden 2048, H=16, dk=dv=128, conv 4, weights N(0, 0.02); prefill B=4 x T=4096, "
                               "then decode steps at B=4 continuing from the prefill state",
                     "prefill_ms": ms_lf, "prefill_tokens_per_s": LB * LT / (ms_lf / 1e3),
                     "decode_ms_per_step": ms_ld, "decode_steps_per_s": 1e3 / ms_ld,
                     "decode_graph_ms_per_step": ms_ldg, "decode_graph_steps_per_s": 1e3 / ms_ldg}
        log(f"layer (config 5): prefill B={LB} T={LT} {ms_lf:.3f} ms ({LB * LT / (ms_lf / 1e3):.4g} tok/s), "
            f"decode B={LB} {ms_ld * 1e3:.1f} us/step eager, {ms_ldg * 1e3:.1f} us/step as a HIP graph")
        del layer, wl, xl, st_l, step_g

    # ------------------------------------------------------------------ CPU oracle
    cpu_prefill = cpu_decode = None
    parity = {}
    if not args.no_cpu_baseline:
        from oracle.decode_ref import ref_decode
        from oracle.prefill_ref import ref_prefill

        torch.set_num_threads(os.cpu_count() or 1)
        nthr = torch.get_num_threads()
        dt_t = torch.tensor(0.0)

        def cpu_pf():
            return ref_prefill(d["q"], d["k"], d["v"], d["A_log"], d["a"], dt_t, d["b_logits"], d["mask"],
                               state_in=None, scale=0.0, chunk_size=C)

        o_ref, S_ref = cpu_pf()  # warm-up, also the parity reference
        reps = 3
        t0 = time.perf_counter()
        for _ in range(reps):
            cpu_pf()
        cpu_ms = (time.perf_counter() - t0) / reps * 1e3
        cpu_prefill = dict(value=tokens / (cpu_ms / 1e3), unit="tokens/s", cores=nthr, kind="port",
                           sample=f"oracle.prefill_ref.ref_prefill (float32 torch CPU) on the same B={B} T={T} "
                                  f"H={H} inputs, 1 warm-up + {reps} timed calls, {cpu_ms:.0f} ms/call; "
                                  f"{os.cpu_count()} logical CPUs ({cpu_model()})")
        od = (out_gpu.float().cpu() - o_ref).abs()
        parity["prefill_out_max_abs_err"] = od.max().item()
        parity["prefill_out_within_2e-2"] = bool((od <= 2e-2 + 2e-2 * o_ref.abs()).all())
        parity["prefill_state_rel_fro"] = ((S_gpu.cpu() - S_ref).norm() / S_ref.norm()).item()

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
        cpu_decode = dict(value=1e3 / cpu_dms, unit="steps/s", cores=nthr, kind="port",
                          sample=f"oracle.decode_ref.ref_decode on the same B={DB} H={DH} state and inputs, "
                                 f"1 warm-up + {nd} timed steps, {cpu_dms:.0f} ms/step")
        parity["decode_out_max_abs_err"] = max((a - b).abs().max().item() for a, b in zip(o_chk, o_refs))
        parity["decode_state_rel_fro_3steps"] = ((S_chk - S_ref3).norm() / S_ref3.norm()).item()
        log(f"cpu oracle: prefill {cpu_ms:.0f} ms/call, decode {cpu_dms:.0f} ms/step, {nthr} threads; parity {parity}")

    result = {
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
        "roofline": {
            "bound": "mfma",
            "kernel": "gdn_prefill_state_hip (map + scan + output kernels)",
            "achieved": state_tflops,
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": state_tflops / PEAK_BF16_TFLOPS,
            "traffic": measured_traffic("prefill_state") if (B, T) == (1, 8192) else None,
            "flop_per_launch": STATE_FLOP_PER_TOKEN_HEAD * tokens * H,
            "kernel_ms": ms_state,
        },
        "prefill_phases": {
            "intra_ms": ms_intra, "intra_tflops": intra_tflops,
            "state_ms": ms_state, "state_tflops": state_tflops,
            "path_tflops": path_tflops, "path_mfma_frac": path_tflops / PEAK_BF16_TFLOPS,
            "path_gbs": path_gbs, "path_hbm_frac": path_gbs / PEAK_HBM_GBS,
            "path_flop": PREFILL_FLOP_PER_TOKEN_HEAD * tokens * H, "path_bytes": prefill_bytes(B, T, H),
        },
        "prefill_batches": batches or None,
        "prefill_varlen": varlen,
        "layer_e2e": layer_e2e,
        "decode": {
            "value": 1e3 / ms_decode, "unit": "steps/s", "ms_per_step": ms_decode, "steps": args.decode_steps,
            "config": {"workload": "GDN decode B=256 H=32 dk=dv=128, fp32 state in place, fresh q/k/v each step",
                       "B": DB, "H": DH, "dk": K, "dv": V},
            "dtype": "fp32",
            "roofline": {"bound": "hbm", "kernel": "gdn_decode_kernel", "achieved": dec_gbs, "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": dec_gbs / PEAK_HBM_GBS,
                         "traffic": measured_traffic("decode"),
                         "bytes_per_launch": decode_bytes(DB, DH), "kernel_ms": ms_decode},
            "cpu_baseline": cpu_decode,
        },
        "cpu_baseline": cpu_prefill,
        "parity": parity or None,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
