#!/usr/bin/env python3
"""bench.py — Mamba-2-2.7B-shaped int4 (group 64, fp16 scales) / bf16 inference on one MI355X.

Workload: 64 layers, d_model 2560, d_inner 5120, 80 heads x 64,
d_state 128, 1 group, conv 4, vocab 50280, random-init weights resident in HBM.
  * value     = greedy decode tokens/s at batch 1 (one step = one token through all
                64 layers + lm_head + argmax, replayed as one HIP graph);
  * prefill   = 4 x 4096 token prefill, tokens/s and MFMA utilisation;
  * decode at batch 4 / 16 is reported alongside;
  * roofline  = the dominant decode kernel (RMSNorm + in_proj GEMV + conv update
                + SSD step in one launch), algorithmic bytes per launch / its
                average launch time measured here with HIP events on the
                library's stream;
  * cpu_baseline = the CPU oracle (a C restatement of the reference kernels; the
                reference itself has no CPU path) on a bounded sample.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def ssd_flops_per_token_head(Q=64, N=128, P=64):
    # intra-chunk C.B^T, (M o decay).X, chunk state, C.S (dense count, per token per head)
    return 2 * Q * N + 2 * Q * P + 4 * N * P


def fused_buffers(sh):
    """Per-launch buffers of the dominant decode kernel (batch 1): hidden, conv
    state, SSD state, gated SSD output, the projection's tagged words."""
    import torch
    return (torch.randn(1, sh.d_model, device="cuda").to(torch.bfloat16),
            torch.zeros(sh.xbc, sh.d_conv, dtype=torch.bfloat16, device="cuda"),
            torch.zeros(sh.n_heads, sh.d_head, sh.d_state, dtype=torch.float32, device="cuda"),
            torch.empty(sh.d_inner, dtype=torch.bfloat16, device="cuda"),
            torch.zeros(sh.proj, dtype=torch.int64, device="cuda"))


def fused_launcher(L, ctx, m, sh, bufs):
    """All layers' lssm_inproj_ssd_decode launches (the engine's batch-1 decode
    kernel: RMSNorm + in_proj GEMV + conv update + SiLU + SSD step + SiLU(z)
    gate), one per layer; every call takes a new tag."""
    hid, cst, sst, y, xfer = bufs
    fn = L.lib.lssm_inproj_ssd_decode
    pre = [(hid.data_ptr(), Lw["norm_w"].data_ptr(), Lw["in_proj_w"].data_ptr(), Lw["in_proj_s"].data_ptr(),
            cst.data_ptr(), Lw["conv1d_w"].data_ptr(), Lw["conv1d_b"].data_ptr(), Lw["dt_bias"].data_ptr(),
            Lw["A_log"].data_ptr(), Lw["D"].data_ptr(), sst.data_ptr(), y.data_ptr(), xfer.data_ptr())
           for Lw in m.layers]
    post = (sh.d_model, sh.d_inner, sh.d_state, sh.n_groups, sh.n_heads, sh.d_head, sh.d_conv, 1e-5,
            L.W_Q4_G64, L.BF16)
    tag = [0]

    def run():
        bad = 0
        for a in pre:
            tag[0] += 1
            bad |= fn(ctx.h, *a, tag[0], *post)
        L.check(bad)
    return run


def fused_bytes(m, sh):
    """Algorithmic bytes of one launch: int4 weights + fp16 scales, hidden and
    norm weight, conv state read + write, conv weight + bias, SSD state read +
    write, A_log / dt_bias / D, the gated output (the tagged words that carry
    the projection between workgroups are not counted)."""
    Lw0 = m.layers[0]
    return (Lw0["in_proj_w"].numel() + Lw0["in_proj_s"].numel() * 2 +
            (sh.d_model * 2) * 2 +
            sh.xbc * sh.d_conv * 2 * 2 + sh.xbc * (sh.d_conv + 1) * 2 +
            2 * sh.n_heads * sh.d_head * sh.d_state * 4 +
            3 * sh.n_heads * 2 +
            sh.d_inner * 2)


def profile_kernel(L, ctx, m, sh, stream):
    """Workload of the rocprofv3 --pmc runs: the dominant decode kernel over all
    64 layers' weights, 10 times, then a 256 MiB device-to-device copy 10 times
    (the known-size reference that scales the FETCH_SIZE / WRITE_SIZE counters)."""
    import torch
    run = fused_launcher(L, ctx, m, sh, fused_buffers(sh))
    ctx.begin_batch()
    for _ in range(10):
        run()
    ctx.commit_and_wait()
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"profile_kernel": "inproj_ssd_decode", "launches": 10 * sh.n_layer,
                      "copy_bytes": src.numel(), "copies": 10}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--model", default="mamba2-2.7b")
    ap.add_argument("--prefill-batch", type=int, default=4)
    ap.add_argument("--prefill-len", type=int, default=4096)
    ap.add_argument("--prefill-reps", type=int, default=3)
    ap.add_argument("--batches", default="4,16", help="extra decode batch sizes to report")
    ap.add_argument("--cpu-steps", type=int, default=3)
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-kernel", action="store_true",
                    help="only run the dominant decode kernel over all layers plus a 256 MiB "
                         "device copy (the calibration reference for rocprofv3 --pmc runs)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(every box has one MI355X; multi-GPU sharding is design-only).", file=sys.stderr)
        sys.exit(2)

    import ctypes as C

    import torch

    import lite_ssm_amd as L
    from lite_ssm_amd.model import DeviceModel, Engine, shape

    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ctx = L.Ctx(stream=stream.cuda_stream)
    sh = shape(args.model)
    t0 = time.time()
    m = DeviceModel(sh, act=L.BF16, wfmt=L.W_Q4_G64, seed=0)
    torch.cuda.synchronize()
    print(f"[bench] model {args.model} built in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    PB, PL = args.prefill_batch, args.prefill_len
    batches = [int(b) for b in args.batches.split(",") if b]
    if args.profile_kernel:
        profile_kernel(L, ctx, m, sh, stream)
        return
    eng = Engine(ctx, m, max_batch=max([PB, 1] + batches), max_seq=PL)

    def timed(fn, reps=1):
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        ev0.record(stream)
        for _ in range(reps):
            fn()
        ev1.record(stream)
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) / 1e3

    g = torch.Generator().manual_seed(0)
    # ---------------- prefill 4 x 4096 ----------------
    ids = torch.randint(0, sh.vocab_size, (PB, PL), generator=g, dtype=torch.int32).cuda()
    nxt = torch.zeros(max([PB, 1] + batches), dtype=torch.int32, device="cuda")
    eng.reset()
    eng.prefill(ids, nxt)                                   # warm-up
    pt = []
    for _ in range(args.prefill_reps):
        eng.reset()
        pt.append(timed(lambda: eng.prefill(ids, nxt)))
    t_pre = min(pt)
    ptoks = PB * PL
    pre_flops = 2.0 * sh.linear_params() * sh.n_layer * ptoks + \
        ssd_flops_per_token_head() * sh.n_heads * sh.n_layer * ptoks + \
        2.0 * sh.d_model * sh.vocab_size * PB
    print(f"[bench] prefill {PB}x{PL}: {t_pre * 1e3:.1f} ms", file=sys.stderr, flush=True)

    # ---------------- decode bs=1 (headline) ----------------
    eng.reset()
    ids1 = ids[:1, :256].contiguous()
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    eng.prefill(ids1, tok)
    eng.decode_graph(tok, tok, args.warmup)                 # capture + warm-up
    torch.cuda.synchronize()
    t_dec = timed(lambda: eng.decode_graph(tok, tok, args.steps))
    tok_s = args.steps / t_dec
    print(f"[bench] decode bs=1: {t_dec / args.steps * 1e3:.3f} ms/token", file=sys.stderr, flush=True)

    # algorithmic bytes per decode token (weights once + per-sequence state r/w)
    wbytes = m.weight_bytes()
    state_bytes = sh.n_layer * (sh.n_heads * sh.d_head * sh.d_state * 4 + sh.xbc * sh.d_conv * 2)
    extra = {}
    for b in batches:
        eng.reset()
        tb = torch.zeros(b, dtype=torch.int32, device="cuda")
        eng.prefill(ids[:b, :128].contiguous() if b <= PB else
                    torch.randint(0, sh.vocab_size, (b, 128), generator=g, dtype=torch.int32).cuda(), tb)
        eng.decode_graph(tb, tb, 4)
        n = max(16, args.steps // 8)
        tbt = timed(lambda: eng.decode_graph(tb, tb, n))
        extra[f"decode_bs{b}_tok_s"] = round(b * n / tbt, 1)
        extra[f"decode_bs{b}_hbm_frac"] = round((wbytes + 2 * b * state_bytes) / (tbt / n) / 1e9 / HBM_PEAK_GBS, 4)
        print(f"[bench] decode bs={b}: {tbt / n * 1e3:.3f} ms/step", file=sys.stderr, flush=True)

    # ---------------- dominant kernel, live (HIP events on the library's stream) ----------------
    # (shapes the fused launch does not take, e.g. 8B with more workgroups than
    # CUs, decode through separate launches: roofline is then null)
    roof = None
    run = fused_launcher(L, ctx, m, sh, fused_buffers(sh))
    ctx.begin_batch()
    try:
        run()
        reps = 10
        t_k = timed(run, reps)
    except L.LssmError as err:
        t_k = None
        print(f"[bench] inproj_ssd_decode not measured: {err}", file=sys.stderr, flush=True)
    finally:
        ctx.commit_and_wait()
    if t_k is not None:
        k_us = t_k / (reps * sh.n_layer) * 1e6
        k_bytes = fused_bytes(m, sh)
        achieved = k_bytes / (k_us * 1e-6) / 1e9
        print(f"[bench] inproj_ssd_decode: {k_us:.2f} us/launch, {achieved:.0f} GB/s", file=sys.stderr, flush=True)

    # ---------------- CPU baseline (oracle, bounded sample) ----------------
    cpu = None
    if not args.no_cpu_baseline:
        import numpy as np

        import oracle as O
        nthr = max(1, min(args.cpu_threads, os.cpu_count() or 1))
        O.set_num_threads(nthr)
        host = m.to_host()
        om = O.Model(host, vars(sh), L.BF16, L.W_Q4_G64)
        conv, ssd = om.new_state(1)
        tk = np.array([1], np.int32)
        om.decode(conv, ssd, tk)                             # warm-up (page-in)
        c0 = time.time()
        for _ in range(args.cpu_steps):
            lg = om.decode(conv, ssd, tk)
            tk = O.argmax(lg, L.BF16)
        ct = time.time() - c0
        cpu = {"value": round(args.cpu_steps / ct, 3), "unit": "tok/s", "cores": nthr, "kind": "port",
               "sample": f"{args.cpu_steps} greedy decode steps at batch 1 through all {sh.n_layer} "
                         f"layers + lm_head of the same int4-g64/bf16 weights, CPU oracle "
                         f"(C, OpenMP {nthr} threads)"}
        print(f"[bench] cpu oracle: {ct / args.cpu_steps:.2f} s/token", file=sys.stderr, flush=True)

    if t_k is not None:
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "inproj_ssd_decode (RMSNorm + in_proj int4-g64 GEMV + conv update + SiLU "
                          "+ SSD step + SiLU(z) gate, one launch per layer)",
                "bytes_per_launch": int(k_bytes), "avg_launch_us": round(k_us, 3)}

    # HBM bytes per launch of the same kernel from the two rocprofv3 --pmc passes
    # (FETCH_SIZE, WRITE_SIZE, calibrated on a 256 MiB copy), recorded in profiles/
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "inproj_ssd_decode_traffic.json")
    if args.model == "mamba2-2.7b" and os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("traffic_bytes")
    if roof is not None:
        roof["traffic"] = traffic

    out = {
        "metric": "decode tok/s (bs=1) + prefill tok/s, Mamba-2-2.7B int4; % HBM/MFMA roofline",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_dec / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"{args.model}-shaped int4-g64 (fp16 scales) bf16, greedy decode "
                               f"batch 1 (BASELINE config 4), random-init weights in HBM",
                   "layers": sh.n_layer, "d_model": sh.d_model, "vocab": sh.vocab_size,
                   "batch": 1, "prefill": f"{PB}x{PL}"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "step_hbm_frac": round((wbytes + 2 * state_bytes) / (t_dec / args.steps) / 1e9 / HBM_PEAK_GBS, 4),
        "step_bytes": int(wbytes + 2 * state_bytes),
        "prefill_tok_s": round(ptoks / t_pre, 1),
        "prefill_ms": round(t_pre * 1e3, 2),
        "prefill_tflops": round(pre_flops / t_pre / 1e12, 2),
        "prefill_mfma_frac": round(pre_flops / t_pre / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
    }
    out.update(extra)
    eng.close()
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
