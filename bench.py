"""Benchmark of the headline workload: fwd+bwd(+AdamW) tokens/s of a LoRA fine-tune of a
Qwen3-0.6B-shaped decoder with a frozen Q8_0 base, batch 4 x 1024, on one MI355X.

    python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--config lora_q8|lora_q4k|full_bf16|tiny]

Prints ONE JSON line.  The timed region is K full training steps (forward,
backward, global-norm clip, AdamW) of the resident engine, bracketed by
torch.cuda.synchronize().  Inputs (synthetic uniform token ids, next-token
labels) are already in HBM.  The step runs as a replayed HIP graph (bit-identical
to eager launches).  The dominant kernel's roofline comes from HIP events the library
records for each MFMA GEMM launch on its own stream (timestamped by the dispatch, via
hipExtLaunchKernelGGL) during a separate pass of eager steps after the timed region
(smhip_profile_begin/end).  cpu_baseline times a restatement of the reference's
AVX2/FMA CPU tiers (oracle/cpu_twin.c) on a bounded sample of the same workload (see
cpu_baseline()).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "fwd+bwd tokens/sec/GPU (LoRA, Q8_0 base); bwd MFMA util % & HBM GB/s"
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3      # MI355X fp32 matrix
PEAK_HBM_GBS = 8000.0


def make_config(name):
    from sharpmind_amd import model as M
    if name == "lora_q8":
        return M.qwen3_0_6b(batch=4, seq=1024, qtype=M.QTYPE_Q8_0, rank=16, alpha=32.0), "Qwen3-0.6B LoRA r16 a32 Q8_0 base, 4x1024"
    if name == "lora_q4k":
        return M.qwen3_1_7b(batch=2, seq=2048, qtype=M.QTYPE_Q4_K, rank=32, alpha=64.0), "Qwen3-1.7B LoRA r32 a64 Q4_K base, 2x2048"
    if name == "full_bf16":
        return M.qwen3_0_6b(batch=8, seq=512, qtype=M.QTYPE_F32, rank=0, alpha=0.0), "Qwen3-0.6B full-parameter bf16 (fp32 masters), 8x512"
    if name == "tiny":
        return M.tiny_llama(), "tiny Llama 2x256 fp32, 4x128"
    raise SystemExit(f"unknown config {name}")


def elementwise_hbm(L, dev, reps=20):
    """Config 2: the fused elementwise backward kernels at the configured shapes, timed with
    events on the launch stream.  GB/s = algorithmic bytes (each input read once, each output
    written once) / kernel time; frac against the 8 TB/s HBM peak."""
    import torch
    from sharpmind_amd import check
    s = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    out = {}

    def timed(name, fn, nbytes):
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        sec = e0.elapsed_time(e1) / reps * 1e-3
        out[name] = {"us": round(sec * 1e6, 1), "bytes": nbytes, "gbs": round(nbytes / sec / 1e9, 1),
                     "frac": round(nbytes / sec / 1e9 / PEAK_HBM_GBS, 4)}

    T, D = 8192, 1024  # RMSNorm backward: dY, x_hat read; dX written (gamma / rmsInv are 40 KB)
    dy = torch.randn(T, D, device=dev, generator=g)
    xn = torch.randn(T, D, device=dev, generator=g)
    rinv = torch.rand(T, device=dev, generator=g) + 0.5
    gam = 1 + 0.1 * torch.randn(D, device=dev, generator=g)
    dgam = torch.zeros(D, device=dev)
    dx = torch.empty_like(dy)
    timed("rmsnorm_bwd_8192x1024", lambda: check(L.smhip_grad_rmsnorm(dy.data_ptr(), xn.data_ptr(), rinv.data_ptr(),
          gam.data_ptr(), dgam.data_ptr(), dx.data_ptr(), T, D, s)), 3 * T * D * 4)
    del dy, xn, dx
    T, F = 8192, 3072  # SwiGLU backward: dAct, gate, up read; [dg | du] written
    da = torch.randn(T, F, device=dev, generator=g)
    ga = torch.randn(T, F, device=dev, generator=g)
    up = torch.randn(T, F, device=dev, generator=g)
    dgu = torch.empty(T, 2 * F, device=dev)
    timed("swiglu_bwd_8192x3072", lambda: check(L.smhip_grad_swiglu(da.data_ptr(), ga.data_ptr(), up.data_ptr(),
          dgu.data_ptr(), T, F, s)), 5 * T * F * 4)
    del da, ga, up, dgu
    T, V = 8192, 32000  # cross-entropy backward: logits read once, dLogits written once
    z = 2 * torch.randn(T, V, device=dev, generator=g)
    lab = torch.randint(0, V, (T,), device=dev, dtype=torch.int32, generator=g)
    dz = torch.empty_like(z)
    loss = torch.zeros(1, device=dev)
    timed("ce_bwd_8192x32000", lambda: check(L.smhip_ce_softmax_grad(z.data_ptr(), lab.data_ptr(), dz.data_ptr(),
          loss.data_ptr(), T, V, -100, 0.0, s)), 2 * T * V * 4)
    del z, dz
    n = 100_000_000  # AdamW: param, grad, m, v read; param, m, v written
    p = 0.02 * torch.randn(n, device=dev, generator=g)
    gr = 0.02 * torch.randn(n, device=dev, generator=g)
    m = 0.02 * torch.randn(n, device=dev, generator=g)
    v = (0.02 * torch.randn(n, device=dev, generator=g)).abs_()
    timed("adamw_100M", lambda: check(L.smhip_adamw_update(p.data_ptr(), gr.data_ptr(), m.data_ptr(), v.data_ptr(), n,
          0.9, 0.95, 0.1, 0.05, 1e-4, 1e-8, 0.1, s)), 7 * n * 4)
    return out


def gemm_dx_traffic():
    """HBM bytes per launch of the backward dX GEMMs (kernel instantiations with TAG 1), measured
    offline with rocprofv3 --pmc
    (FETCH_SIZE and WRITE_SIZE runs, scaled by a device-copy calibration); the summary with
    the commands is profiles/gemm_dx_traffic_lora_q8_qwen3_0.6b_4x1024.md.  None if absent."""
    path = os.path.join(ROOT, "profiles", "gemm_dx_traffic_lora_q8_qwen3_0.6b_4x1024.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1].strip())
    except OSError:
        pass
    return None


def _host_cpu():
    """(logical CPUs, model name) of this host, from os and /proc/cpuinfo."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return os.cpu_count(), model


def cpu_baseline(cfg):
    """The reference's AVX2/FMA CPU tiers, restated in oracle/cpu_twin.c (-O3 -mavx2 -mfma, OpenMP over
    the loops the reference runs in Parallel.For, on this host's cores), timed on a bounded sample:
    one decoder block's forward + backward + AdamW at the configuration's full batch x sequence,
    and the head (final norm, LM head through the Q8_0 table, cross-entropy, head dX) on 128
    tokens.  Step time = n_layers x block + head x (tokens / 128); value = tokens / step time."""
    import oracle
    head_tokens = 128
    full = 0 if cfg.lora_rank else 1
    blk, head, threads = oracle.twin_time_step(cfg.d_model, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.ffn_dim,
                                               cfg.vocab, cfg.batch, cfg.seq, cfg.lora_rank, head_tokens, full)
    step = cfg.n_layers * blk + head * (cfg.tokens / head_tokens)
    ncpu, model = _host_cpu()
    return {"value": round(cfg.tokens / step, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "host_cpus": ncpu, "cpu_model": model,
            "sample": f"oracle/cpu_twin.c: restatement of the reference AVX2/FMA tiers (QuantizedMatMulQ8_0 FMA, "
                      f"Linear_FMA, Attention_Scalar per batch row, AdamWUpdate_AVX2), {threads} OpenMP threads; "
                      f"one block fwd+bwd at {cfg.batch}x{cfg.seq} tokens = {blk:.2f} s (x{cfg.n_layers} layers), "
                      f"head + CE on {head_tokens} tokens = {head:.2f} s (x{cfg.tokens // head_tokens}); "
                      f"extrapolated step {step:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="lora_q8")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true", help="launch kernels one by one instead of replaying a graph")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 64 MiB device copy (byte reference for the HBM traffic counters)")
    args = ap.parse_args()
    if args.calibrate_copy:
        # reference for the rocprofv3 FETCH_SIZE / WRITE_SIZE counters: a device copy of 64 MiB
        import torch
        src = torch.empty(64 << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "device copy", "bytes_read": 64 << 20, "bytes_written": 64 << 20}))
        return
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported in this build "
              "(the data-parallel design is described in DESIGN.md; no multi-GPU figure is produced)",
              file=sys.stderr)
        sys.exit(2)

    import ctypes
    import torch
    import sharpmind_amd
    from sharpmind_amd import check
    from sharpmind_amd.engine import Engine, next_token_labels
    from sharpmind_amd.model import PREC_BF16, QTYPE_Q8_0

    cfg, desc = make_config(args.config)
    dev = torch.device("cuda:0")
    L = sharpmind_amd.lib()
    eng = Engine(cfg, lr=1e-3, beta1=0.9, beta2=0.95, adam_eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    eng.init_synthetic(seed=0)
    T = cfg.tokens
    ids = torch.empty(T, dtype=torch.int32, device=dev)
    check(L.smhip_fill_token_ids(ids.data_ptr(), T, 1234, cfg.vocab, torch.cuda.current_stream().cuda_stream))
    labels = next_token_labels(ids, cfg.seq)
    loss = torch.zeros(1, device=dev)
    if not args.eager:
        eng.use_graph(True)
    for _ in range(max(args.warmup, 1)):
        eng.step(ids, labels, loss)
    torch.cuda.synchronize()
    loss_first = float(loss.cpu()[0])

    t0 = time.perf_counter()
    for _ in range(args.steps):
        eng.step(ids, labels, loss)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    loss_last = float(loss.cpu()[0])

    # roofline pass: eager steps with live HIP-event timing of the GEMM / flash kernels
    psteps = max(1, min(args.steps, 3))
    check(L.smhip_profile_begin(200000))
    for _ in range(psteps):
        eng.step(ids, labels, loss)
    prof = (ctypes.c_double * 12)()
    check(L.smhip_profile_end(prof, 4))

    ms_per_step = dt * 1e3 / args.steps
    tokens_per_s = T / (dt / args.steps)
    peak = PEAK_BF16_TFLOPS if cfg.precision == PREC_BF16 else PEAK_FP32_TFLOPS
    cat = lambda c: (prof[3 * c], prof[3 * c + 1], prof[3 * c + 2])  # (ms, launches, flops)
    g_ms, g_n, g_fl = cat(0)
    dx_ms, dx_n, dx_fl = cat(3)
    all_ms, all_n, all_fl = g_ms + dx_ms, g_n + dx_n, g_fl + dx_fl
    tf = lambda fl, ms: round(fl / (ms * 1e-3) / 1e12, 2) if ms else None
    if dx_n:  # dominant kernel: the backward dX GEMMs through the frozen quantised base
        k_ms, k_n, k_fl = dx_ms, dx_n, dx_fl
        if os.environ.get("SMHIP_BASE_WS") == "1":
            kname = ("gemm_kernel<..., TAG 1>: backward dX = dY W through the frozen base (bf16 copy decoded "
                     "each step), bf16 MFMA")
        elif cfg.base_qtype == QTYPE_Q8_0:
            kname = ("gemm_q8f_kernel<128, 128, 2, 4, 4, 2, true, ..., TAG 1, ...>: backward dX = dY W through "
                     "the frozen Q8_0 base, int8 codes and fp16 scales copied to LDS and decoded there "
                     "(never expanded in HBM), bf16 MFMA")
        else:
            kname = ("gemm_q8f_kernel<128, 128, 2, 4, 4, 2, true, ..., TAG 1, ..., Q4 true>: backward dX = dY W "
                     "through the frozen Q4_K base, 4-bit codes and fp32 scale/min pairs copied to LDS and "
                     "decoded there (never expanded in HBM), bf16 MFMA")
    else:
        k_ms, k_n, k_fl = all_ms, all_n, all_fl
        kname = "gemm_kernel (all linears, fwd+bwd)"
    achieved = tf(k_fl, k_ms) or 0.0
    sustained = None
    if cfg.precision == PREC_BF16:  # what the matrix cores sustain on this device (register operands)
        v = ctypes.c_double()
        check(L.smhip_probe_mfma_bf16(ctypes.byref(v)))
        sustained = round(v.value, 1)
    roofline = {"bound": "mfma", "achieved": achieved, "peak": peak, "unit": "TFLOP/s",
                "frac": round(achieved / peak, 4), "traffic": gemm_dx_traffic() if dx_n else None,
                "mfma_sustained_tflops": sustained,
                "frac_of_sustained": round(achieved / sustained, 4) if sustained else None,
                "kernel": kname,
                "launches_per_step": k_n / psteps, "avg_launch_us": round(k_ms / k_n * 1e3, 2) if k_n else None,
                "algorithmic_flops_per_launch": round(k_fl / k_n) if k_n else None,
                "all_gemm": {"ms_per_step": round(all_ms / psteps, 3), "launches_per_step": all_n / psteps,
                             "tflops": tf(all_fl, all_ms)},
                "flash_fwd_ms_per_step": round(prof[3] / psteps, 3),
                "flash_fwd_tflops": tf(prof[5], prof[3]),
                "flash_bwd_ms_per_step": round(prof[6] / psteps, 3),
                "flash_bwd_tflops": tf(prof[8], prof[6])}
    out = {
        "metric": METRIC, "value": round(tokens_per_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16" if cfg.precision == PREC_BF16 else "fp32",
        "data": "synthetic: uniform random token ids, random-init weights (base quantised on device)",
        "config": {"workload": desc, "global_batch": cfg.batch, "seq_len": cfg.seq, "parallelism": "single GPU",
                   "launch": "eager" if args.eager else "hip_graph",
                   "layers": cfg.n_layers, "vocab": cfg.vocab, "loss_first": round(loss_first, 4),
                   "loss_last": round(loss_last, 4)},
        "roofline": roofline,
    }
    del eng
    torch.cuda.empty_cache()
    out["elementwise_hbm"] = elementwise_hbm(L, dev)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(cfg)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
