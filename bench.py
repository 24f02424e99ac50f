#!/usr/bin/env python3
"""bench.py — Mamba-2 inference on one MI355X: the BASELINE configs.

Headline: Mamba-2-2.7B shape (64 layers, d_model 2560,
d_inner 5120, 80 heads x 64, d_state 128, 1 group, conv 4, vocab 50280),
int4 group-64 weights with fp16 scales, bf16 activations, random-init weights
resident in HBM.
  * value     = greedy decode tokens/s at batch 1 (one step = one token through
                all 64 layers + lm_head + argmax, replayed as one HIP graph);
  * prefill   = 4 x 4096 tokens: tokens/s and the fraction of the bf16 MFMA peak;
  * decode at batch 4 / 16 alongside;
  * roofline  = the dominant decode kernel (RMSNorm + in_proj GEMV + conv
                update + SSD step in one launch), timed with HIP events on the
                library's stream over all 64 layers' weights and the engine's
                own per-layer conv / SSD state slabs (each launch reads state
                last touched 63 launches earlier, beyond the 256 MB last-level
                cache), algorithmic bytes per launch / its average launch time;
  * cpu_baseline = the CPU oracle (a C restatement of the reference kernels; the
                reference has no CPU path) on a bounded sample, with all the
                host threads this process may use and with one.
Other BASELINE rows (key "configs"): 1 = the fp32 SSD op at the 130M layer
shape; 2 = the 130M int8-g32 linears as GEMV (M = 1, rotated over > 512 MB of
weight copies so every launch reads HBM) and GEMM (M = 2048); 3 = the 130M
model (prefill 2048, greedy decode); 5 = the 8B model (prefill 8192, decode at
batch 32).

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--skip 1,2,3,ref,5,cpu]
"""
import argparse
import hashlib
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0           # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 / fp16
MFMA_FP32_PEAK_TFLOPS = 157.3   # MI355X dense fp32 matrix
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "inproj_ssd_decode_traffic.json")
# the sources the dominant decode kernel is built from: a recorded traffic
# figure is used only while they are unchanged
KERNEL_SOURCES = ["lite_ssm_amd/csrc/gemv.hip", "lite_ssm_amd/csrc/gemv_core.hpp",
                  "lite_ssm_amd/csrc/common.hpp"]


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def sources_sha():
    h = hashlib.sha256()
    for p in KERNEL_SOURCES:
        with open(os.path.join(ROOT, p), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def ssd_flops_per_token_head(Q=64, N=128, P=64):
    # intra-chunk C.B^T, (M o decay).X, chunk state, C.S (dense count, per token per head)
    return 2 * Q * N + 2 * Q * P + 4 * N * P


class Timer:
    """HIP events on the library's stream (torch's Event records on the stream given)."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream

    def __call__(self, fn, reps=1):
        t = self.torch
        ev0, ev1 = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        t.cuda.synchronize()
        ev0.record(self.stream)
        for _ in range(reps):
            fn()
        ev1.record(self.stream)
        t.cuda.synchronize()
        return ev0.elapsed_time(ev1) / 1e3


# ----------------------------------------------------------------------------- roofline kernel
def fused_setup(L, torch, eng, m, sh):
    """The dominant decode kernel's per-launch arguments for every layer, on the
    engine's own per-layer conv / SSD state slabs (lssm_engine_state) and a
    word buffer per layer."""
    import ctypes as C
    cp, sp = C.c_void_p(), C.c_void_p()
    L.check(L.lib.lssm_engine_state(eng.h, C.byref(cp), C.byref(sp)))
    es = 2
    conv_slab = eng.max_batch * sh.xbc * sh.d_conv * es
    ssd_slab = eng.max_batch * sh.n_heads * sh.d_head * sh.d_state * 4
    hid = (torch.randn(1, sh.d_model, device="cuda") * 0.5).to(torch.bfloat16)
    y = torch.empty(sh.n_layer, sh.d_inner, dtype=torch.bfloat16, device="cuda")
    xfer = torch.zeros(sh.n_layer, sh.proj, dtype=torch.int64, device="cuda")
    args = []
    for li, Lw in enumerate(m.layers):
        args.append((hid.data_ptr(), Lw["norm_w"].data_ptr(), Lw["in_proj_w"].data_ptr(),
                     Lw["in_proj_s"].data_ptr(), cp.value + li * conv_slab, Lw["conv1d_w"].data_ptr(),
                     Lw["conv1d_b"].data_ptr(), Lw["dt_bias"].data_ptr(), Lw["A_log"].data_ptr(),
                     Lw["D"].data_ptr(), sp.value + li * ssd_slab, y[li].data_ptr(), xfer[li].data_ptr()))
    return args, (hid, y, xfer)


def fused_launcher(L, ctx, sh, args):
    """All layers' lssm_inproj_ssd_decode launches, one per layer; every call takes a new tag."""
    fn = L.lib.lssm_inproj_ssd_decode
    post = (sh.d_model, sh.d_inner, sh.d_state, sh.n_groups, sh.n_heads, sh.d_head, sh.d_conv, 1e-5,
            L.W_Q4_G64, L.BF16)
    tag = [1 << 20]

    def run():
        bad = 0
        for a in args:
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


def recorded_traffic():
    """HBM bytes per launch from the committed rocprofv3 --pmc passes, if they
    were measured on the kernel sources as they are now."""
    if not os.path.exists(TRAFFIC_JSON):
        return None, "no recorded counter passes"
    rec = json.load(open(TRAFFIC_JSON))
    if rec.get("kernel_sources_sha") != sources_sha():
        return None, "recorded counter passes are of other kernel sources"
    return rec.get("traffic_bytes"), "profiles/inproj_ssd_decode_traffic.json"


# ----------------------------------------------------------------------------- BASELINE rows
def bench_ssd_op(L, torch, ctx, timer):
    """Config 1: the SSD chunked scan alone, fp32, Mamba-2-130M layer shape."""
    Lq, H, P, N, G, ck = 512, 24, 64, 128, 1, 64
    g = torch.Generator(device="cuda").manual_seed(1)
    f = dict(device="cuda", dtype=torch.float32)
    x = torch.randn(Lq, H * P, generator=g, **f)
    dt = torch.randn(Lq, H, generator=g, **f) * 0.5 - 2.0      # softplus applied in the kernel
    dtb = torch.zeros(H, **f)
    alog = torch.rand(H, generator=g, **f) * float(torch.log(torch.tensor(16.0)))
    B = torch.randn(Lq, G * N, generator=g, **f) / N ** 0.5
    Cm = torch.randn(Lq, G * N, generator=g, **f) / N ** 0.5
    D = torch.randn(H, generator=g, **f)
    y = torch.empty(Lq, H * P, **f)
    st = torch.zeros(H, P, N, **f)
    dims = L.SSDDims(Lq, H, P, N, G, ck, 1e-6, 1e6, 1)

    def run():
        L.check(L.lib.lssm_ssd_chunked(ctx.h, x.data_ptr(), B.data_ptr(), Cm.data_ptr(), dt.data_ptr(),
                                       dtb.data_ptr(), alog.data_ptr(), D.data_ptr(), y.data_ptr(),
                                       st.data_ptr(), 1, dims, L.F32))
    ctx.begin_batch()
    try:
        run()
        reps = 50
        t = timer(run, reps) / reps
    finally:
        ctx.commit_and_wait()
    flops = ssd_flops_per_token_head() * Lq * H
    byts = 4 * (2 * Lq * H * P + 2 * Lq * G * N + Lq * H + 3 * H + 2 * H * P * N)
    return {"workload": "SSD chunked scan fp32, L 512, H 24, P 64, N 128, G 1, chunk 64",
            "us": round(t * 1e6, 2), "gflops": round(flops / t / 1e9, 1),
            "gbs": round(byts / t / 1e9, 1), "flops": flops, "bytes": byts,
            "fp32_mfma_frac": round(flops / t / 1e12 / MFMA_FP32_PEAK_TFLOPS, 4)}


def bench_linears_130m(L, torch, ctx, timer):
    """Config 2: the 130M in_proj / out_proj as int8-g32 linears (fp16 act)."""
    from lite_ssm_amd.model import quantize
    out = {}
    g = torch.Generator(device="cuda").manual_seed(2)
    for name, (N, K) in (("in_proj", (3352, 768)), ("out_proj", (768, 1536))):
        w = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.float16).float()
        p, s = quantize(w, L.W_Q8_G32)
        wbytes = p.numel() + s.numel() * 2
        copies = (512 << 20) // wbytes + 1                      # > 512 MB: every launch reads HBM
        ps = [p.clone() for _ in range(copies)]
        ss = [s.clone() for _ in range(copies)]
        x1 = torch.randn(1, K, generator=g, device="cuda").to(torch.float16)
        y1 = torch.empty(1, N, dtype=torch.float16, device="cuda")

        def gemv():
            bad = 0
            for pi, si in zip(ps, ss):
                bad |= L.lib.lssm_linear(ctx.h, x1.data_ptr(), 0, pi.data_ptr(), si.data_ptr(), y1.data_ptr(),
                                         0, None, 1, N, K, L.W_Q8_G32, L.F16, L.EPI_NONE)
            L.check(bad)
        ctx.begin_batch()
        try:
            gemv()
            t1 = timer(gemv) / copies
        finally:
            ctx.commit_and_wait()
        del ps, ss
        M = 2048
        xm = torch.randn(M, K, generator=g, device="cuda").to(torch.float16)
        ym = torch.empty(M, N, dtype=torch.float16, device="cuda")

        def gemm():
            L.check(L.lib.lssm_linear(ctx.h, xm.data_ptr(), 0, p.data_ptr(), s.data_ptr(), ym.data_ptr(), 0,
                                      None, M, N, K, L.W_Q8_G32, L.F16, L.EPI_NONE))
        ctx.begin_batch()
        try:
            gemm()
            reps = 20
            tm = timer(gemm, reps) / reps
        finally:
            ctx.commit_and_wait()
        gb = wbytes + 2 * K + 2 * N
        fl = 2.0 * M * N * K
        out[name] = {"N": N, "K": K, "gemv_us": round(t1 * 1e6, 3), "gemv_bytes": gb,
                     "gemv_gbs": round(gb / t1 / 1e9, 1), "gemv_hbm_frac": round(gb / t1 / 1e9 / HBM_PEAK_GBS, 4),
                     "weight_copies": copies,
                     "gemm_m": M, "gemm_us": round(tm * 1e6, 2), "gemm_tflops": round(fl / tm / 1e12, 2),
                     "gemm_mfma_frac": round(fl / tm / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)}
    out["workload"] = "130M in_proj 3352x768 / out_proj 768x1536, int8 group 32, fp16 scales, fp16 act"
    return out


def bench_ref_api(L, torch, ctx, timer, n_new=33, prompt_len=64):
    """The drop-in path: the reference's own host code (SSMFile, Mamba2Model,
    generate(); tests/cpp/_bin/ref_model_run, built from the reference sources
    against include/lite_ssm/*.hpp) on this backend, greedy decode of a
    130M-shaped int4-b32 / fp16 file, the reference's formats.  Its activations
    and state live in DeviceBuffers in HBM whose host views are synchronised at
    op boundaries; every op is its own launch (and, outside the model's
    batches, a host round trip).  Beside it, the engine on
    the same file (HBM-resident, one graph launch per four steps).  None when the
    harness was not built (it needs the reference checkout at build time)."""
    import subprocess
    import tempfile
    from lite_ssm_amd import ssm as S
    from lite_ssm_amd.model import Engine, shape
    exe = os.path.join(ROOT, "tests", "cpp", "_bin", "ref_model_run")
    if not os.path.exists(exe):
        return None
    sh = shape("mamba2-130m")
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "m.ssm")
        S.write_random(path, sh, L.F16, L.W_Q4_B32, seed=1)
        ids = [(7 * i + 3) % sh.vocab_size for i in range(prompt_len)]
        r = subprocess.run([exe, path, str(n_new), os.path.join(d, "l.bin"), ",".join(map(str, ids))],
                           capture_output=True, text=True, timeout=600)
        if r.returncode != 0:
            log(f"ref_model_run failed ({r.returncode}): {r.stderr.strip()[-200:]}")
            return None
        rec = json.loads(r.stdout.strip().splitlines()[-1])
        with S.SSMFile(path) as f:
            fm = f.model(ctx)
            eng = Engine(ctx, fm, 1, max(prompt_len, sh.chunk_size))
            try:
                tb = torch.tensor([ids], dtype=torch.int32, device="cuda")
                nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
                t_pre = timer(lambda: eng.prefill(tb, nxt))
                eng.decode_graph(nxt, nxt, 4)
                t_dec = timer(lambda: eng.decode_graph(nxt, nxt, n_new - 1)) / (n_new - 1)
            finally:
                eng.close()
    return {"workload": "mamba2-130m-shaped, int4-b32 weights, fp16 act, random init; "
                        f"{prompt_len}-token prompt, {n_new - 1} greedy decode steps at batch 1",
            "ref_api_prefill_ms": round(rec["first_ms"], 3),
            "ref_api_decode_tok_s": round((n_new - 1) * 1000.0 / rec["decode_ms"], 1),
            "engine_prefill_ms": round(t_pre * 1e3, 3),
            "engine_decode_tok_s": round(1.0 / t_dec, 1)}


def bench_model(L, torch, ctx, timer, name, act, wfmt, prefill_batch, prefill_len, decode_batch, steps,
                seed):
    """A whole random-init model: prefill tokens/s and greedy decode tokens/s."""
    from lite_ssm_amd.model import DeviceModel, Engine, shape
    sh = shape(name)
    t0 = time.time()
    m = DeviceModel(sh, act=act, wfmt=wfmt, seed=seed)
    torch.cuda.synchronize()
    log(f"{name} built in {time.time() - t0:.1f}s")
    eng = Engine(ctx, m, max(prefill_batch, decode_batch), prefill_len)
    try:
        g = torch.Generator().manual_seed(seed)
        ids = torch.randint(0, sh.vocab_size, (prefill_batch, prefill_len), generator=g, dtype=torch.int32).cuda()
        nxt = torch.zeros(max(prefill_batch, decode_batch), dtype=torch.int32, device="cuda")
        eng.prefill(ids, nxt)
        pt = []
        for _ in range(3):
            eng.reset()
            pt.append(timer(lambda: eng.prefill(ids, nxt)))
        t_pre = statistics.median(pt)
        ptoks = prefill_batch * prefill_len
        pflops = 2.0 * sh.linear_params() * sh.n_layer * ptoks + \
            ssd_flops_per_token_head(P=sh.d_head, N=sh.d_state) * sh.n_heads * sh.n_layer * ptoks + \
            2.0 * sh.d_model * sh.vocab_size * prefill_batch
        eng.reset()
        tb = torch.zeros(decode_batch, dtype=torch.int32, device="cuda")
        eng.prefill(torch.randint(0, sh.vocab_size, (decode_batch, 64), generator=g, dtype=torch.int32).cuda(), tb)
        eng.decode_graph(tb, tb, 4)
        t_dec = timer(lambda: eng.decode_graph(tb, tb, steps)) / steps
        wbytes = m.weight_bytes()
        state_bytes = sh.n_layer * (sh.n_heads * sh.d_head * sh.d_state * 4 + sh.xbc * sh.d_conv * (4 if act == L.F32 else 2))
        step_bytes = wbytes + 2 * decode_batch * state_bytes
        return {"workload": f"{name}-shaped, {'int8-g32' if wfmt == L.W_Q8_G32 else 'int4-g64'} weights, "
                           f"{'fp16' if act == L.F16 else 'bf16'} act, random init",
                "prefill": f"{prefill_batch}x{prefill_len}", "prefill_ms": round(t_pre * 1e3, 2),
                "prefill_tok_s": round(ptoks / t_pre, 1),
                "prefill_mfma_frac": round(pflops / t_pre / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                "decode_batch": decode_batch, "decode_steps": steps,
                "decode_ms_per_step": round(t_dec * 1e3, 4),
                "decode_tok_s": round(decode_batch / t_dec, 1),
                "decode_step_bytes": int(step_bytes),
                "decode_hbm_frac": round(step_bytes / t_dec / 1e9 / HBM_PEAK_GBS, 4)}
    finally:
        eng.close()
        del m
        torch.cuda.empty_cache()


def host_threads():
    """Threads this process may use: the CPU affinity, capped by OMP_NUM_THREADS
    where the environment sets it (the GPU box's share of its host)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return n


def cpu_model_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(O, L, m, sh, decode_steps, prefill_len):
    """The C oracle (the reference kernels restated; the reference itself has no
    CPU path) on a bounded sample of the same workload: greedy decode steps at
    batch 1 through all layers + lm_head (median and min over the steps), and
    one prefill of `prefill_len` tokens; with all host threads and with one."""
    import numpy as np
    host = m.to_host()
    om = O.Model(host, vars(sh), L.BF16, L.W_Q4_G64)
    nthr = host_threads()
    res = {}
    for thr in (nthr, 1):
        O.set_num_threads(thr)
        conv, ssd = om.new_state(1)
        tk = np.array([1], np.int32)
        om.decode(conv, ssd, tk)                                 # warm-up (page-in)
        ts = []
        for _ in range(decode_steps if thr == nthr else 2):
            c0 = time.time()
            lg = om.decode(conv, ssd, tk)
            ts.append(time.time() - c0)
            tk = O.argmax(lg, L.BF16)
        res[thr] = ts
    O.set_num_threads(nthr)
    conv, ssd = om.new_state(1)
    ids = np.random.default_rng(0).integers(0, sh.vocab_size, (1, prefill_len)).astype(np.int32)
    c0 = time.time()
    om.prefill(conv, ssd, ids)
    tp = time.time() - c0
    med = statistics.median(res[nthr])
    return {"value": round(1.0 / med, 3), "unit": "tok/s", "cores": nthr, "kind": "port",
            "sample": f"{len(res[nthr])} greedy decode steps at batch 1 through all {sh.n_layer} layers + "
                      f"lm_head of the same int4-g64/bf16 weights (median step; min "
                      f"{min(res[nthr]) * 1e3:.0f} ms), C oracle with OpenMP, {nthr} threads",
            "cpu_model": cpu_model_name(),
            "decode_tok_s_1thread": round(1.0 / statistics.median(res[1]), 4),
            "prefill_tok_s": round(prefill_len / tp, 1),
            "prefill_sample": f"1 x {prefill_len} tokens, {nthr} threads"}


# ----------------------------------------------------------------------------- main
def profile_kernel(L, torch, ctx, eng, m, sh):
    """Workload of the rocprofv3 --pmc runs: the dominant decode kernel over all
    64 layers' weights and the engine's state slabs, 10 times, the batch-1
    out_proj launch over all layers 10 times, then a 256 MiB device-to-device
    copy 10 times (the known-size reference that scales the FETCH_SIZE /
    WRITE_SIZE counters)."""
    args, keep = fused_setup(L, torch, eng, m, sh)
    run = fused_launcher(L, ctx, sh, args)
    ctx.begin_batch()
    for _ in range(10):
        run()
    ctx.commit_and_wait()
    # then the batch-1 out_proj launch (RMSNorm + int4 GEMV + residual, the
    # engine's second launch per layer) over every layer, 10 times, on the
    # fused launches' gated outputs
    hid, y, _ = keep
    ctx.begin_batch()
    for _ in range(10):
        bad = 0
        for li, Lw in enumerate(m.layers):
            bad |= L.lib.lssm_norm_linear_decode(ctx.h, y[li].data_ptr(), Lw["mixer_norm_w"].data_ptr(), 1e-5,
                                                 Lw["out_proj_w"].data_ptr(), Lw["out_proj_s"].data_ptr(),
                                                 hid.data_ptr(), hid.data_ptr(), 1, sh.d_model, sh.d_inner,
                                                 L.W_Q4_G64, L.BF16, L.EPI_ADD)
        L.check(bad)
    ctx.commit_and_wait()
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"profile_kernel": "inproj_ssd_decode", "launches": 10 * sh.n_layer,
                      "copy_bytes": src.numel(), "copies": 10, "kernel_sources_sha": sources_sha()}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--prefill-batch", type=int, default=4)
    ap.add_argument("--prefill-len", type=int, default=4096)
    ap.add_argument("--prefill-reps", type=int, default=3)
    ap.add_argument("--batches", default="4,16", help="extra decode batch sizes to report")
    ap.add_argument("--cpu-steps", type=int, default=8)
    ap.add_argument("--skip", default="", help="comma list of sections to skip: 1,2,3,ref,5,cpu")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-kernel", action="store_true",
                    help="only run the dominant decode kernel over all layers plus a 256 MiB "
                         "device copy (the calibration reference for rocprofv3 --pmc runs)")
    args = ap.parse_args()
    skip = set(s for s in args.skip.split(",") if s)
    if args.no_cpu_baseline:
        skip.add("cpu")

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(every box has one MI355X; multi-GPU sharding is design-only).", file=sys.stderr)
        sys.exit(2)

    import torch

    import lite_ssm_amd as L
    from lite_ssm_amd.model import DeviceModel, Engine, shape

    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ctx = L.Ctx(stream=stream.cuda_stream)
    timer = Timer(torch, stream)
    sh = shape("mamba2-2.7b")
    t0 = time.time()
    m = DeviceModel(sh, act=L.BF16, wfmt=L.W_Q4_G64, seed=0)
    torch.cuda.synchronize()
    log(f"model mamba2-2.7b built in {time.time() - t0:.1f}s")
    PB, PL = args.prefill_batch, args.prefill_len
    batches = [int(b) for b in args.batches.split(",") if b]
    eng = Engine(ctx, m, max_batch=max([PB, 1] + batches), max_seq=PL)
    if args.profile_kernel:
        profile_kernel(L, torch, ctx, eng, m, sh)
        return

    g = torch.Generator().manual_seed(0)
    # ---------------- prefill 4 x 4096 ----------------
    ids = torch.randint(0, sh.vocab_size, (PB, PL), generator=g, dtype=torch.int32).cuda()
    nxt = torch.zeros(max([PB, 1] + batches), dtype=torch.int32, device="cuda")
    eng.reset()
    eng.prefill(ids, nxt)                                   # warm-up
    pt = []
    for _ in range(args.prefill_reps):
        eng.reset()
        pt.append(timer(lambda: eng.prefill(ids, nxt)))
    t_pre = statistics.median(pt)
    ptoks = PB * PL
    pre_flops = 2.0 * sh.linear_params() * sh.n_layer * ptoks + \
        ssd_flops_per_token_head() * sh.n_heads * sh.n_layer * ptoks + \
        2.0 * sh.d_model * sh.vocab_size * PB
    log(f"prefill {PB}x{PL}: {t_pre * 1e3:.1f} ms (median of {len(pt)}, min {min(pt) * 1e3:.1f})")

    # ---------------- decode bs=1 (headline) ----------------
    eng.reset()
    ids1 = ids[:1, :256].contiguous()
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    eng.prefill(ids1, tok)
    eng.decode_graph(tok, tok, args.warmup)                 # capture + warm-up
    torch.cuda.synchronize()
    t_dec = timer(lambda: eng.decode_graph(tok, tok, args.steps))
    tok_s = args.steps / t_dec
    log(f"decode bs=1: {t_dec / args.steps * 1e3:.3f} ms/token")

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
        tbt = timer(lambda: eng.decode_graph(tb, tb, n))
        extra[f"decode_bs{b}_tok_s"] = round(b * n / tbt, 1)
        extra[f"decode_bs{b}_hbm_frac"] = round((wbytes + 2 * b * state_bytes) / (tbt / n) / 1e9 / HBM_PEAK_GBS, 4)
        log(f"decode bs={b}: {tbt / n * 1e3:.3f} ms/step")

    # ---------------- dominant kernel, live, on the engine's buffers ----------------
    roof = None
    fargs, keep = fused_setup(L, torch, eng, m, sh)
    run = fused_launcher(L, ctx, sh, fargs)
    ctx.begin_batch()
    try:
        run()
        reps = 10
        t_k = timer(run, reps)
    except L.LssmError as err:
        t_k = None
        log(f"inproj_ssd_decode not measured: {err}")
    finally:
        ctx.commit_and_wait()
    if t_k is not None:
        k_us = t_k / (reps * sh.n_layer) * 1e6
        k_bytes = fused_bytes(m, sh)
        achieved = k_bytes / (k_us * 1e-6) / 1e9
        traffic, tsrc = recorded_traffic()
        log(f"inproj_ssd_decode: {k_us:.2f} us/launch, {achieved:.0f} GB/s; traffic: {tsrc}")
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "inproj_ssd_decode (RMSNorm + in_proj int4-g64 GEMV + conv update + SiLU "
                          "+ SSD step + SiLU(z) gate, one launch per layer)",
                "bytes_per_launch": int(k_bytes), "avg_launch_us": round(k_us, 3),
                "kernel_sources_sha": sources_sha()}
    del keep

    # ---------------- CPU baseline (oracle, bounded sample) ----------------
    cpu = None
    if "cpu" not in skip:
        import oracle as O
        cpu = cpu_baseline(O, L, m, sh, args.cpu_steps, 64)
        log(f"cpu oracle: {cpu['value']} tok/s on {cpu['cores']} threads ({cpu['cpu_model']})")
    eng.close()
    del m
    torch.cuda.empty_cache()

    # ---------------- the other BASELINE rows ----------------
    configs = {}
    if "1" not in skip:
        configs["1_ssd_op_fp32"] = bench_ssd_op(L, torch, ctx, timer)
        log(f"config 1: {configs['1_ssd_op_fp32']['us']} us")
    if "2" not in skip:
        configs["2_linears_130m_q8"] = bench_linears_130m(L, torch, ctx, timer)
        log("config 2 done")
    if "3" not in skip:
        configs["3_130m_q8_f16"] = bench_model(L, torch, ctx, timer, "mamba2-130m", L.F16, L.W_Q8_G32,
                                               1, 2048, 1, 256, 3)
        log(f"config 3: {configs['3_130m_q8_f16']['decode_tok_s']} tok/s decode")
    if "ref" not in skip:
        rec = bench_ref_api(L, torch, ctx, timer)
        if rec is not None:
            configs["ref_api_130m_q4b32_f16"] = rec
            log(f"reference API path: {rec['ref_api_decode_tok_s']} tok/s decode "
                f"(engine {rec['engine_decode_tok_s']})")
    if "5" not in skip:
        configs["5_8b_q4_bf16"] = bench_model(L, torch, ctx, timer, "mamba2-8b", L.BF16, L.W_Q4_G64,
                                              1, 8192, 32, 64, 5)
        log(f"config 5: {configs['5_8b_q4_bf16']['decode_tok_s']} tok/s decode at batch 32")

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
        "config": {"workload": "mamba2-2.7b-shaped int4-g64 (fp16 scales) bf16, greedy decode "
                               "batch 1 (BASELINE config 4), random-init weights in HBM",
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
    out["configs"] = configs
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
