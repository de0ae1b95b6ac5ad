#!/usr/bin/env python3
"""Benchmark: one MMDiT block step of Qwen-Image-2.1 at 1024x1024 output with
Q4_K_M weights on one MI355X, through the C ABI of libqimm.so.

Workload (the configuration the headline metric is quoted on): hidden 4096,
32 heads x 128, MLP 12288; 4096 image tokens (64x64 latent grid) attending over
a cached 256-token text prefix; q/k/v/out/gate_up in Q4_K, the MLP down
projection in Q6_K; adaLN modulation row; bf16 MFMA with f32 accumulation and
an f32 residual stream; every quantized-matmul input rounded to int8 as the
reference CPU path rounds it (the block's default QIMM_ACT_CANDLE mode: Q8_K
per 256 values, the operands bf16(d * q)). A step is one block forward; the timed loop cycles over
several distinct blocks' weights (more bytes than the 256 MB last-level cache)
and over the 32 layers of the prefix cache, as the 32-block x 20-step denoising
loop does. Inputs are resident in HBM before timing starts.

After the timed loop, a profiled pass records HIP events on the launch stream
between the stages of each step (qimm_block_profile), giving each in-step
kernel's duration, TFLOP/s and roofline fraction; the CPU oracle is timed on a
bounded sample of the same block on the host cores.

Beside the headline number: the same step with bf16 activations
(QIMM_ACT_BF16), and the whole configuration as the reference runs it: 32
distinct blocks x 20 denoising steps with true CFG, each prompt's 256-token text
prefix filled once through the 32 blocks into its own cache (denoise_loop).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "qwen3-image21_amd")
sys.path.insert(0, PKG)

METRIC = "ms per MMDiT block step + attention TFLOP/s at 1024² Q4_K_M (1 GPU)"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBPS = 8000.0

HID, HEADS, HD, MLP = 4096, 32, 128, 12288
S_IMG, P_TXT, GRID = 4096, 256, 64
LAYERS = 32


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--blocks", type=int, default=4, help="distinct block weight sets cycled in the loop")
    ap.add_argument("--profile-steps", type=int, default=16, help="steps timed stage by stage after the loop")
    ap.add_argument("--cpu-rows", type=int, default=4096, help="token rows in the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-weight-streaming", action="store_true",
                    help="skip the short-token weight-streaming measurements")
    ap.add_argument("--no-denoise-loop", action="store_true",
                    help="skip the 32-block x 20-step denoising loop with CFG")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the Q8_0 dequant-GEMM sets, the multi-reference attention, the MLP-16384 block, "
                         "the 8448-token prefix fill, the config-1 block and the torch SDPA bar")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="first run one plain device copy of this many MiB, the known-size kernel that "
                         "scales the FETCH_SIZE / WRITE_SIZE counters of a rocprofv3 --pmc pass")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the block step is not sharded across GPUs "
              "(see the sharding notes); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import qimm
    import synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    ctx = qimm.Context(0)
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib * (1 << 18)
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        log(f"bench: calibration copy of {args.copy_calibration_mib} MiB done")

    # ---- weights: distinct blocks, Q4_K with a Q6_K down projection ----
    t0 = time.time()
    blocks, host_w0 = [], None
    wbytes = 0
    for i in range(args.blocks):
        rng = np.random.default_rng(1000 + i)
        w = {
            "to_q": synth.random_blocks(rng, synth.Q4_K, HID, HID),
            "to_k": synth.random_blocks(rng, synth.Q4_K, HID, HID),
            "to_v": synth.random_blocks(rng, synth.Q4_K, HID, HID),
            "to_out": synth.random_blocks(rng, synth.Q4_K, HID, HID),
            "gate_up": synth.random_blocks(rng, synth.Q4_K, 2 * MLP, HID),
            "down": synth.random_blocks(rng, synth.Q6_K, HID, MLP),
        }
        shapes = {"to_q": (synth.Q4_K, HID, HID), "to_k": (synth.Q4_K, HID, HID), "to_v": (synth.Q4_K, HID, HID),
                  "to_out": (synth.Q4_K, HID, HID), "gate_up": (synth.Q4_K, 2 * MLP, HID),
                  "down": (synth.Q6_K, HID, MLP)}
        keep = []
        T = qimm.BlockTensors()
        for name, field in (("to_q", "to_q"), ("to_k", "to_k"), ("to_v", "to_v"), ("to_out", "to_out"),
                            ("gate_up", "gate_up"), ("down", "mlp_out")):
            t, r, c = shapes[name]
            setattr(T, field, qimm.make_tensor(t, r, c, w[name].tobytes(), keep))
        nq = (1 + 0.02 * rng.standard_normal(HD)).astype(np.float32)
        nk = (1 + 0.02 * rng.standard_normal(HD)).astype(np.float32)
        T.norm_q = qimm.make_tensor(synth.F32, HD, 1, nq.tobytes(), keep)
        T.norm_k = qimm.make_tensor(synth.F32, HD, 1, nk.tobytes(), keep)
        blocks.append(ctx.block_create(qimm.BlockConfig(HID, HEADS, HD, MLP), T))
        if i == 0:
            wbytes = sum(v.size for v in w.values())
            host_w0 = (w, shapes, nq, nk)
        del keep
    log(f"bench: {args.blocks} blocks uploaded ({wbytes / 1e6:.1f} MB GGUF each) in {time.time() - t0:.1f}s")

    # ---- prefix cache (32 layers), activations, modulation, RoPE rows ----
    g = torch.Generator(device="cuda").manual_seed(0)
    kv = ctx.kv_create(LAYERS, 1, HEADS, P_TXT)
    for layer in range(LAYERS):
        k = torch.randn((1, HEADS, P_TXT, HD), generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn((1, HEADS, P_TXT, HD), generator=g, device="cuda").to(torch.bfloat16)
        kv.store(layer, k.data_ptr(), v.data_ptr(), sh)
    x = torch.randn((1, S_IMG, HID), generator=g, device="cuda")
    x_out = torch.empty_like(x)
    mod = 0.5 * torch.randn((1, 1, 4 * HID), generator=g, device="cuda")
    mask = [0] * P_TXT + [1] * S_IMG
    pe_host = qimm.rope_table([(1, GRID, GRID)], mask)[P_TXT:]
    pe = torch.from_numpy(np.ascontiguousarray(pe_host)).cuda()

    def step(i):
        blocks[i % len(blocks)].forward(x.data_ptr(), x_out.data_ptr(), 1, S_IMG, mod.data_ptr(), pe.data_ptr(),
                                        kv, i % LAYERS, None, None, sh)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    log("bench: warmup done")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = e0.elapsed_time(e1) / args.steps
    assert torch.isfinite(x_out).all().item(), "non-finite block output"
    log(f"bench: block step {ms_step:.3f} ms (wall {wall * 1e3 / args.steps:.3f} ms)")


    # ---- per-stage device times inside the step (HIP events on the launch stream) ----
    att_flop = 4.0 * HEADS * S_IMG * (S_IMG + P_TXT) * HD
    kernels = roofline = None
    stages = stage_profile(blocks, step, args.profile_steps)
    if stages is None:
        log("bench: no profiled steps, stage report skipped")
    else:
        log(f"bench: stage medians sum to {sum(stages.values()):.3f} ms (timed step {ms_step:.3f} ms)")
        kernels, roofline = stage_report(stages, att_flop, synth)

    block_flop = att_flop + 2.0 * S_IMG * HID * (3 * HID + HID + 2 * MLP) + 2.0 * S_IMG * MLP * HID

    # ---- the same step with bf16 activations (no int8 rounding, no f32 staging) ----
    for blk in blocks:
        blk.set_act_mode(qimm.ACT_BF16)
    ms_bf16 = timed(torch, stream, lambda it=iter(range(1 << 30)): step(next(it)), max(8, args.steps // 2), warmup=2)
    stages_bf16 = stage_profile(blocks, step, args.profile_steps)
    for blk in blocks:
        blk.set_act_mode(qimm.ACT_CANDLE)
    log(f"bench: block step with bf16 activations {ms_bf16:.3f} ms")

    # ---- weight streaming at short token counts (the HBM-bound regime) ----
    streaming = None if args.no_weight_streaming else weight_streaming(ctx, torch, np, qimm, synth, stream, host_w0)

    # ---- the configuration as the reference runs it: 32 blocks x 20 steps with CFG ----
    denoise = None
    if not args.no_denoise_loop:
        for blk in blocks:
            blk.free()
        blocks = []
        denoise = denoise_loop(ctx, torch, np, qimm, synth, stream)

    # ---- the other measured configurations: Q8_0 dequant-GEMM sets, multi-reference attention ----
    q8 = mref = mlp16k = pfill = cfg1 = sdpa = gemm_bar = None
    if not args.no_other_configs:
        q8 = q8_gemm_sets(ctx, torch, np, qimm, synth, stream)
        mref = multi_ref_attention(ctx, torch, qimm, stream)
        mlp16k = block_mlp16384(ctx, torch, np, qimm, synth, stream, kv, x, x_out, mod, pe)
        pfill = prefix_fill_8448(ctx, torch, np, qimm, synth, stream)
        cfg1 = config1_block(ctx, torch, np, qimm, synth, stream, cpu=not args.no_cpu_baseline)
        sdpa = torch_sdpa_bar(torch, stream)
        gemm_bar = torch_gemm_bar(torch, stream)

    # ---- CPU baseline: the oracle in candle mode on a bounded sample ----
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args.cpu_rows, host_w0)

    for blk in blocks:
        blk.free()
    kv.free()

    out = {
        "metric": METRIC,
        "value": round(ms_step, 4),
        "unit": "ms/block-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "MMDiT block step, 1024x1024 T2I, Q4_K_M (Q4_K + Q6_K down), cached prefix",
                   "hidden": HID, "heads": HEADS, "head_dim": HD, "mlp": MLP, "batch": 1,
                   "image_tokens": S_IMG, "prefix_tokens": P_TXT, "distinct_blocks": args.blocks,
                   "weights_mb_per_block": round(wbytes / 1e6, 1),
                   "activations": "int8 rounding of every quantized-matmul input as the reference CPU path "
                                  "(QIMM_ACT_CANDLE: Q8_K per 256 values), bf16 MFMA operands bf16(d*q)"},
        "block_step_bf16_activations_ms": round(ms_bf16, 4),
        "attention_tflops": round(kernels["attention"]["tflops"], 2) if kernels else None,
        "attention_frac_bf16_peak": round(kernels["attention"]["frac_bf16_peak"], 4) if kernels else None,
        "block_tflops": round(block_flop / ms_step / 1e9, 2),
        "block_frac_bf16_peak": round(block_flop / ms_step / 1e9 / PEAK_BF16_TFLOPS, 4),
        "stages_ms": {k: round(v, 4) for k, v in stages.items()} if stages else None,
        "stages_bf16_activations_ms": {k: round(v, 4) for k, v in stages_bf16.items()} if stages_bf16 else None,
        "kernels": {k: {kk: round(vv, 4) for kk, vv in v.items()} for k, v in kernels.items()} if kernels else None,
        "roofline": roofline,
        "denoise_loop": denoise,
        "weight_streaming": streaming,
        "dequant_gemm_q8_0": q8,
        "multi_ref_attention": mref,
        "block_mlp16384": mlp16k,
        "prefix_fill_8448": pfill,
        "config1_block": cfg1,
        "attention_torch_sdpa": sdpa,
        "gemm_torch_bf16": gemm_bar,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def denoise_loop(ctx, torch, np, qimm, synth, stream, layers=LAYERS, steps=20, cfg_scale=4.0, host_sets=4):
    """The headline configuration as the reference runs it: text-to-image at
    1024x1024 with true CFG, QwenImageTransformerQuantized over 32 blocks
    (src/quantized_transformer.rs:460-551) driven by the sampling loop
    (src/pipeline.rs:154-197). Each of the two prompts' 256-token text prefixes
    runs once through txt_in and the 32 blocks under the t = 0 modulation and the
    block-causal mask into its own bf16 cache (prefix_kv, :359-392); then each of
    the 20 steps embeds the timestep, runs the cached forward of the 4096 image
    tokens for both prompts (img_in, modulation, the 32 blocks, norm_out,
    proj_out), combines them (neg + s (cond - neg)) and takes the Euler step, all
    on the device. 32 distinct Q4_K_M blocks (device copies of `host_sets`
    random weight sets; 4.3 GB), Q8_0 global linears, joint_dim 4096.
    Reported: the denoise time (both prefix fills and the 20 steps) from HIP
    events, and ms per block-step over the 2 x 20 x 32 block forwards. The
    reference publishes 30.0 s for this loop on an NVIDIA L20 (README.md:133-139):
    other hardware, context only."""
    t0 = time.time()
    sets = [random_block(np, synth, 5000 + i, HID, MLP, synth.Q4_K, synth.Q6_K) for i in range(host_sets)]
    blocks = [upload_block(ctx, qimm, synth, dict(hidden=HID, heads=HEADS, mlp=MLP), *sets[i % host_sets])
              for i in range(layers)]
    del sets
    rng = np.random.default_rng(6000)
    CH, JD = 64, 4096

    def q8(rows, cols):
        return (synth.Q8_0, synth.random_blocks(rng, synth.Q8_0, rows, cols), rows, cols)

    def f32(rows, cols, std):
        return (synth.F32, (rng.standard_normal((rows, cols)) * std).astype(np.float32), rows, cols)

    g = {"img_in": f32(HID, CH, 0.1), "t_linear_1": q8(HID, 256), "t_linear_2": q8(HID, HID),
         "modulation": q8(4 * HID, HID), "norm_out": q8(HID, HID), "proj_out": f32(CH, HID, 0.02),
         "txt_norm": f32(1, JD, 0.1), "txt_in": q8(HID, JD), "txt_out": q8(HID, HID)}
    keep = []
    T = qimm.ModelTensors()
    for name, (t, data, rows, cols) in g.items():
        setattr(T, name, qimm.make_tensor(t, rows, cols, data.tobytes(), keep))
    model = ctx.model_create(qimm.ModelConfig(CH, JD, HID, layers), T, blocks)
    del keep, g
    log(f"bench: denoise loop: {layers} blocks and the global layers uploaded in {time.time() - t0:.1f}s")

    sh = stream.cuda_stream
    gen = torch.Generator(device="cuda").manual_seed(21)
    txt = [torch.randn((1, P_TXT, JD), generator=gen, device="cuda") for _ in range(2)]
    lat0 = torch.randn((1, S_IMG, CH), generator=gen, device="cuda")
    lat = torch.empty_like(lat0)
    ids, plen, tlen = qimm.joint_layout(P_TXT, None, (), (GRID, GRID))
    pe_full = qimm.rope_table([(1, GRID, GRID)], [1 if i >= 0 else 0 for i in ids])
    pe_pre = torch.from_numpy(np.ascontiguousarray(pe_full[:plen])).cuda()
    pe_tgt = torch.from_numpy(np.ascontiguousarray(pe_full[plen:])).cuda()
    ids_d = torch.from_numpy(np.array(ids[:plen], np.int32)).cuda()
    pieces = qimm.joint_layout_pieces(P_TXT)
    sig = qimm.flow_match_sigmas(steps, S_IMG)
    tsin = torch.empty((steps, 256), dtype=torch.float32, device="cuda")
    for i in range(steps):
        ctx.timestep_embedding([sig[i]], tsin[i].data_ptr(), sh)
    caches = [ctx.kv_create(layers, 1, HEADS, plen) for _ in range(2)]
    pc, pn = torch.empty_like(lat0), torch.empty_like(lat0)
    n = S_IMG * CH

    def run(nsteps):
        lat.copy_(lat0)
        for j in range(2):
            model.prefix_fill(txt[j].data_ptr(), P_TXT, None, 0, 1, pieces, ids_d.data_ptr(), None,
                              pe_pre.data_ptr(), caches[j], sh)
        for i in range(nsteps):
            model.forward(lat.data_ptr(), 1, S_IMG, tsin[i].data_ptr(), pe_tgt.data_ptr(), caches[0], pc.data_ptr(),
                          None, sh)
            model.forward(lat.data_ptr(), 1, S_IMG, tsin[i].data_ptr(), pe_tgt.data_ptr(), caches[1], pn.data_ptr(),
                          None, sh)
            ctx.cfg_combine(pc.data_ptr(), pn.data_ptr(), n, cfg_scale, pc.data_ptr(), sh)
            dt = (sig[i + 1] - sig[i]) if i + 1 < steps else -sig[i]
            ctx.euler_step(lat.data_ptr(), pc.data_ptr(), n, dt, sh)

    with torch.cuda.stream(stream):
        run(1)  # warm-up: one step
        torch.cuda.synchronize()
        e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        wall0 = time.perf_counter()
        e0.record(stream)
        lat.copy_(lat0)
        for j in range(2):
            model.prefix_fill(txt[j].data_ptr(), P_TXT, None, 0, 1, pieces, ids_d.data_ptr(), None,
                              pe_pre.data_ptr(), caches[j], sh)
        e1.record(stream)
        for i in range(steps):
            model.forward(lat.data_ptr(), 1, S_IMG, tsin[i].data_ptr(), pe_tgt.data_ptr(), caches[0], pc.data_ptr(),
                          None, sh)
            model.forward(lat.data_ptr(), 1, S_IMG, tsin[i].data_ptr(), pe_tgt.data_ptr(), caches[1], pn.data_ptr(),
                          None, sh)
            ctx.cfg_combine(pc.data_ptr(), pn.data_ptr(), n, cfg_scale, pc.data_ptr(), sh)
            dt = (sig[i + 1] - sig[i]) if i + 1 < steps else -sig[i]
            ctx.euler_step(lat.data_ptr(), pc.data_ptr(), n, dt, sh)
        e2.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - wall0
    fill_ms, loop_ms = e0.elapsed_time(e1), e1.elapsed_time(e2)
    assert torch.isfinite(lat).all().item(), "non-finite latents"
    for kv in caches:
        kv.free()
    model.free()
    for b in blocks:
        b.free()
    total_s = (fill_ms + loop_ms) / 1e3
    per_block = loop_ms / (2 * steps * layers)
    log(f"bench: denoise loop 1024x1024 Q4_K_M, {layers} blocks x {steps} steps, CFG: {total_s:.3f} s "
        f"(prefix fills {fill_ms:.1f} ms, steps {loop_ms:.1f} ms, {per_block:.3f} ms per block-step incl. the "
        f"global layers; wall {wall:.3f} s)")
    return {"denoise_s": round(total_s, 4), "prefix_fill_ms": round(fill_ms, 2), "steps_ms": round(loop_ms, 2),
            "ms_per_block_step_in_loop": round(per_block, 4), "wall_s": round(wall, 4), "blocks": layers,
            "steps": steps, "cfg": "true CFG, 2 prompts x 256 text tokens, sequential batch-1 forwards",
            "reference_published_s": {"value": 30.0, "hardware": "NVIDIA L20", "source": "README.md:133-139",
                                      "note": "context only: other hardware"}}


def stage_profile(blocks, step, nsteps, warm=8):
    """Median ms per stage over `nsteps` block steps timed stage by stage (HIP
    events between the stages, read back after each step), after `warm`
    profiled steps that are not counted: the first steps after a long timed
    loop run up to 20% slow while the clock settles, the median keeps one
    such step from moving a stage."""
    if nsteps <= 0:
        return None
    per = {}
    for blk in blocks:
        blk.profile(True)
    for i in range(warm + nsteps):
        step(i)
        if i >= warm:
            for k, v in blocks[i % len(blocks)].stage_times().items():
                per.setdefault(k, []).append(v)
    for blk in blocks:
        blk.profile(False)
    return {k: sorted(v)[len(v) // 2] if len(v) % 2 else 0.5 * sum(sorted(v)[len(v) // 2 - 1:len(v) // 2 + 1])
            for k, v in per.items()}


def stage_report(stages, att_flop, synth):
    """Per-kernel ms, TFLOP/s and roofline fraction from the stage times of the
    block step; the dominant kernel's roofline with its measured HBM traffic."""
    log("bench: stages " + ", ".join(f"{k} {v:.3f}" for k, v in stages.items()) + " ms")
    gemm = {"qkv": (3 * HID, HID), "out_proj": (HID, HID), "gate_up": (2 * MLP, HID), "down": (HID, MLP)}
    kernels = {"attention": {"ms": stages["attention"], "gflop": att_flop / 1e9}}
    for name, (n, k) in gemm.items():
        kernels[name] = {"ms": stages[name], "gflop": 2.0 * S_IMG * n * k / 1e9}
    qk4 = synth.row_bytes(synth.Q4_K, HID)
    kernels["qkv"]["weight_bytes"] = 3 * HID * qk4
    kernels["out_proj"]["weight_bytes"] = HID * qk4
    kernels["gate_up"]["weight_bytes"] = 2 * MLP * qk4
    kernels["down"]["weight_bytes"] = HID * synth.row_bytes(synth.Q6_K, MLP)
    for kname, kd in kernels.items():
        kd["tflops"] = kd["gflop"] / kd["ms"]
        kd["frac_bf16_peak"] = kd["tflops"] / PEAK_BF16_TFLOPS
        if "weight_bytes" in kd:
            kd["weight_gbps"] = kd["weight_bytes"] / kd["ms"] / 1e6
        log(f"bench: {kname}: {kd['ms']:.3f} ms, {kd['tflops']:.1f} TFLOP/s")
    dom_name = max(kernels, key=lambda n: kernels[n]["ms"])
    dom = kernels[dom_name]
    traffic = measured_traffic(dom_name)
    roofline = {"kernel": dom_name, "bound": "mfma", "achieved": round(dom["tflops"], 2),
                "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(dom["tflops"] / PEAK_BF16_TFLOPS, 4),
                "traffic": traffic["bytes"] if traffic else None, "flop_per_launch": dom["gflop"] * 1e9}
    if traffic:
        roofline["traffic_source"] = traffic["source"]
    return kernels, roofline


def weight_streaming(ctx, torch, np, qimm, synth, stream, host_w, token_counts=(16, 64), iters=50):
    """The block's Q4_K gate_up projection (24576 x 4096, 56.6 MB) and Q6_K
    down projection (4096 x 12288, 41.3 MB) at short token counts, where the
    time is the weight bytes over HBM bandwidth: device time per call (both
    kernels of the split-K path) from HIP events on the launch stream."""
    w, shapes, _, _ = host_w
    out = {}
    sh = stream.cuda_stream
    for name in ("gate_up", "down"):
        t, n, k = shapes[name]
        wbytes = synth.row_bytes(t, k) * n
        # enough copies that one pass over them exceeds the 256 MB last-level
        # cache: every call streams its weights from HBM
        copies = [ctx.upload(t, n, k, w[name].tobytes()) for _ in range(int(300e6 // wbytes) + 1)]
        for m in token_counts:
            x = torch.randn((m, k), device="cuda").to(torch.bfloat16)
            y = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
            for W in copies:
                ctx.qmatmul(W, x.data_ptr(), m, k, y.data_ptr(), synth.BF16, sh)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(stream)
            for i in range(iters):
                ctx.qmatmul(copies[i % len(copies)], x.data_ptr(), m, k, y.data_ptr(), synth.BF16, sh)
            e1.record(stream)
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / iters * 1e3
            gbps = wbytes / us / 1e3
            out[f"{name}_m{m}"] = {"us": round(us, 2), "weight_mb": round(wbytes / 1e6, 1), "gbps": round(gbps, 1),
                                   "frac_hbm": round(gbps / PEAK_HBM_GBPS, 4)}
            log(f"bench: {name} at {m} tokens: {us:.1f} us, {gbps:.0f} GB/s of weights "
                f"({gbps / PEAK_HBM_GBPS:.2f} of HBM peak)")
        for W in copies:
            W.free()
    return out


def q8_gemm_sets(ctx, torch, np, qimm, synth, stream, token_counts=(4352, 256, 64, 16), iters=10):
    """Dequant-GEMM with Q8_0 weights on the fused QKV [12288 x 4096], output
    [4096 x 4096], MLP up [16384 x 4096] and down [4096 x 16384] sets, bf16
    activations ~ N(0, 1) of 4352 tokens (the image + prefix rows of a joint
    pass) and of 256, 64 and 16 tokens (the weight-bandwidth regime), bf16
    output. Every call reads its weights from
    HBM (rotating copies past the last-level cache). Device time per call from
    HIP events on the launch stream."""
    sets = {"qkv": (3 * HID, HID), "out": (HID, HID), "up": (16384, HID), "down": (HID, 16384)}
    out = {}
    sh = stream.cuda_stream
    for name, (n, k) in sets.items():
        rng = np.random.default_rng(77)
        data = synth.random_blocks(rng, synth.Q8_0, n, k).tobytes()
        wbytes = len(data)
        copies = [ctx.upload(synth.Q8_0, n, k, data) for _ in range(int(300e6 // wbytes) + 1)]
        for m in token_counts:
            x = torch.randn((m, k), device="cuda").to(torch.bfloat16)
            y = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
            for W in copies:
                ctx.qmatmul(W, x.data_ptr(), m, k, y.data_ptr(), synth.BF16, sh)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(stream)
            for i in range(iters):
                ctx.qmatmul(copies[i % len(copies)], x.data_ptr(), m, k, y.data_ptr(), synth.BF16, sh)
            e1.record(stream)
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / iters
            tflops = 2.0 * m * n * k / ms / 1e9
            gbps = wbytes / ms / 1e6
            out[f"{name}_m{m}"] = {"ms": round(ms, 4), "tflops": round(tflops, 1),
                                   "frac_bf16_peak": round(tflops / PEAK_BF16_TFLOPS, 4),
                                   "weight_gbps": round(gbps, 1), "frac_hbm": round(gbps / PEAK_HBM_GBPS, 4)}
            log(f"bench: Q8_0 {name} {n}x{k} at {m} tokens: {ms:.3f} ms, {tflops:.0f} TFLOP/s, {gbps:.0f} GB/s")
        for W in copies:
            W.free()
    return out


def multi_ref_attention(ctx, torch, qimm, stream, iters=10):
    """Joint attention of the image-conditioned multi-reference step with true
    CFG: batch 2 (the two prompts), 32 heads x 128, 4096 image-token queries
    over a cached 8448-token prefix (256 text + 2 x 4096 condition-image
    tokens, one prefix per prompt) plus the 4096 own keys: 12544 keys,
    4 B H Sq (P + S) D = 1683.6 GFLOP per call."""
    B, P, S = 2, 8448, S_IMG
    g = torch.Generator(device="cuda").manual_seed(5)
    kv = ctx.kv_create(1, B, HEADS, P)
    k = torch.randn((B, HEADS, P, HD), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((B, HEADS, P, HD), generator=g, device="cuda").to(torch.bfloat16)
    kv.store(0, k.data_ptr(), v.data_ptr(), stream.cuda_stream)
    del k, v
    q = torch.randn((B, HEADS, S, HD), generator=g, device="cuda").to(torch.bfloat16)
    ko = torch.randn((B, HEADS, S, HD), generator=g, device="cuda").to(torch.bfloat16)
    vto = torch.randn((B, HEADS, HD, S), generator=g, device="cuda").to(torch.bfloat16)
    o = torch.empty((B, S, HEADS * HD), device="cuda", dtype=torch.bfloat16)
    scale = HD ** -0.5

    def call():
        ctx.attention(q.data_ptr(), B, HEADS, S, kv, 0, ko.data_ptr(), vto.data_ptr(), S, scale, o.data_ptr(),
                      stream.cuda_stream)

    for _ in range(3):
        call()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(iters):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / iters
    assert torch.isfinite(o.float()).all().item(), "non-finite attention output"
    kv.free()
    flop = 4.0 * B * HEADS * S * (P + S) * HD
    tflops = flop / ms / 1e9
    log(f"bench: multi-reference attention (B=2, 12544 keys): {ms:.3f} ms, {tflops:.0f} TFLOP/s")
    return {"ms": round(ms, 4), "gflop": round(flop / 1e9, 1), "tflops": round(tflops, 1),
            "frac_bf16_peak": round(tflops / PEAK_BF16_TFLOPS, 4), "batch": B, "prefix_tokens": P,
            "own_tokens": S, "keys": P + S}


def cpu_model():
    """The host CPU as lscpu names it (vendor, model name, sockets x cores x
    threads, AVX-512 / VNNI flags), else /proc/cpuinfo's model name."""
    import subprocess
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        kv = {}
        for line in txt.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                kv.setdefault(k.strip(), v.strip())
        flags = kv.get("Flags", "").split()
        simd = [f for f in ("avx2", "avx512f", "avx512bw", "avx512_vnni", "avx_vnni", "amx_int8") if f in flags]
        name = kv.get("Model name")
        if name:
            return (f"{kv.get('Vendor ID', '')} {name}; {kv.get('Socket(s)', '?')} socket(s) x "
                    f"{kv.get('Core(s) per socket', '?')} cores x {kv.get('Thread(s) per core', '?')} threads, "
                    f"{kv.get('CPU(s)', '?')} CPUs; {' '.join(simd)}").strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_counts():
    """Online CPUs (os.cpu_count, nproc's --all view) and the ones this process may run on (nproc)."""
    try:
        usable = len(os.sched_getaffinity(0))
    except OSError:
        usable = None
    return {"online_cpus": os.cpu_count(), "nproc": usable}


def upload_block(ctx, qimm, synth, cfg, w, types):
    """Block from host GGUF bytes: w[name] = bytes, types[name] = (ggml type, rows, cols)."""
    keep = []
    T = qimm.BlockTensors()
    for name, field in (("to_q", "to_q"), ("to_k", "to_k"), ("to_v", "to_v"), ("to_out", "to_out"),
                        ("gate_up", "gate_up"), ("down", "mlp_out")):
        t, r, c = types[name]
        setattr(T, field, qimm.make_tensor(t, r, c, w[name].tobytes(), keep))
    for name in ("norm_q", "norm_k"):
        setattr(T, name, qimm.make_tensor(synth.F32, HD, 1, w[name].tobytes(), keep))
    return ctx.block_create(qimm.BlockConfig(cfg["hidden"], cfg["heads"], HD, cfg["mlp"]), T)


def random_block(np, synth, seed, hidden, mlp, attn_type, down_type):
    rng = np.random.default_rng(seed)
    types = {"to_q": (attn_type, hidden, hidden), "to_k": (attn_type, hidden, hidden),
             "to_v": (attn_type, hidden, hidden), "to_out": (attn_type, hidden, hidden),
             "gate_up": (attn_type, 2 * mlp, hidden), "down": (down_type, hidden, mlp)}
    w = {n: synth.random_blocks(rng, t, r, c) for n, (t, r, c) in types.items()}
    w["norm_q"] = (1 + 0.02 * rng.standard_normal(HD)).astype(np.float32)
    w["norm_k"] = (1 + 0.02 * rng.standard_normal(HD)).astype(np.float32)
    return w, types


def timed(torch, stream, fn, iters, warmup=2):
    for _ in range(warmup):
        fn()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(iters):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def block_mlp16384(ctx, torch, np, qimm, synth, stream, kv, x, x_out, mod, pe, nblocks=2, iters=16):
    """The block step at 1024x1024 with an MLP of 16384 (the MLP width the headline
    configuration states; the reference's own blocks use 3 x hidden = 12288): the same
    4096 tokens over the 256-token prefix, Q4_K with a Q6_K down projection, two distinct
    blocks cycled (more bytes than the last-level cache). 2491.1 GFLOP per step."""
    mlp = 16384
    blocks = []
    for i in range(nblocks):
        w, types = random_block(np, synth, 3000 + i, HID, mlp, synth.Q4_K, synth.Q6_K)
        blocks.append(upload_block(ctx, qimm, synth, dict(hidden=HID, heads=HEADS, mlp=mlp), w, types))
        del w
    sh = stream.cuda_stream
    it = [0]

    def step():
        i = it[0]
        it[0] += 1
        blocks[i % nblocks].forward(x.data_ptr(), x_out.data_ptr(), 1, S_IMG, mod.data_ptr(), pe.data_ptr(), kv,
                                    i % LAYERS, None, None, sh)

    ms = timed(torch, stream, step, iters, warmup=4)
    assert torch.isfinite(x_out).all().item(), "non-finite block output"
    for b in blocks:
        b.free()
    flop = 4.0 * HEADS * S_IMG * (S_IMG + P_TXT) * HD + 2.0 * S_IMG * HID * (4 * HID + 3 * mlp)
    log(f"bench: block step with MLP 16384: {ms:.3f} ms, {flop / ms / 1e9:.0f} TFLOP/s")
    return {"ms": round(ms, 4), "gflop": round(flop / 1e9, 1), "tflops": round(flop / ms / 1e9, 1),
            "frac_bf16_peak": round(flop / ms / 1e9 / PEAK_BF16_TFLOPS, 4), "mlp": mlp}


def prefix_fill_8448(ctx, torch, np, qimm, synth, stream, iters=4):
    """The prefix pass of the multi-reference step (prefix_kv): one Q8_0 block over the
    8448 prefix tokens of one prompt (256 text + 2 condition images of 64 x 64 latents),
    block-causal mask from the image ids, the t = 0 modulation row, the layer's K/V
    written out as the cache entry. Attention work counts the allowed (query, key)
    pairs only: 4 x 32 heads x 128 x pairs."""
    P, T = 8448, 256
    w, types = random_block(np, synth, 4000, HID, MLP, synth.Q8_0, synth.Q8_0)
    blk = upload_block(ctx, qimm, synth, dict(hidden=HID, heads=HEADS, mlp=MLP), w, types)
    del w
    ids = np.array([-1] * T + [0] * 4096 + [1] * 4096, dtype=np.int32)
    pe_h = qimm.rope_table([(1, 64, 64), (1, 64, 64)], [0] * T + [1] * 8192)
    g = torch.Generator(device="cuda").manual_seed(9)
    xp = torch.randn((1, P, HID), generator=g, device="cuda")
    xo = torch.empty_like(xp)
    mod0 = 0.5 * torch.randn((1, 1, 4 * HID), generator=g, device="cuda")
    ids_d = torch.from_numpy(ids).cuda()
    pe_d = torch.from_numpy(np.ascontiguousarray(pe_h)).cuda()
    k_o = torch.empty((1, HEADS, P, HD), dtype=torch.bfloat16, device="cuda")
    v_o = torch.empty_like(k_o)
    sh = stream.cuda_stream

    def call():
        blk.forward_masked(xp.data_ptr(), xo.data_ptr(), 1, P, mod0.data_ptr(), 1, pe_d.data_ptr(),
                           image_ids=ids_d.data_ptr(), k_out=k_o.data_ptr(), v_out=v_o.data_ptr(), stream=sh)

    ms = timed(torch, stream, call, iters)
    st = stage_profile([blk], lambda i: call(), 3, warm=2)
    assert torch.isfinite(xo).all().item(), "non-finite prefix output"
    blk.free()
    text_pairs = T * (T + 1) // 2
    pairs = text_pairs + 4096 * (T + 4096) + 4096 * P
    att_flop = 4.0 * HEADS * HD * pairs
    gemm_flop = 2.0 * P * HID * (4 * HID + 3 * MLP)
    log(f"bench: prefix fill P=8448 (Q8_0 block, block-causal mask): {ms:.3f} ms per block per prompt, "
        f"attention {st['attention']:.3f} ms ({att_flop / st['attention'] / 1e9:.0f} TFLOP/s on allowed pairs)")
    return {"ms": round(ms, 4), "attention_ms": round(st["attention"], 4),
            "attention_gflop_allowed_pairs": round(att_flop / 1e9, 1),
            "attention_tflops": round(att_flop / st["attention"] / 1e9, 1),
            "gemm_gflop": round(gemm_flop / 1e9, 1), "stages_ms": {k: round(v, 4) for k, v in st.items()},
            "prefix_tokens": P, "weights": "Q8_0"}


def config1_block(ctx, torch, np, qimm, synth, stream, cpu=True, iters=50):
    """The reference CPU-path configuration, timed in full on the GPU and on the host
    cores: hidden 3072, 24 heads x 128, MLP 9216, 256 image tokens (16 x 16 grid) over a
    64-token bf16 prefix, N(0, 0.02) weights quantized to Q8_0, 63.8 GFLOP per block.
    The CPU leg is the oracle in candle mode (int8 activations) on the same inputs."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    O.use_native_build()
    cfg = dict(hidden=3072, heads=24, head_dim=HD, mlp=9216)
    b, s, p = 1, 256, 64
    w = synth.block_weights(11, cfg["hidden"], cfg["heads"], cfg["mlp"], synth.Q8_0)
    types = {"to_q": (synth.Q8_0, 3072, 3072), "to_k": (synth.Q8_0, 3072, 3072), "to_v": (synth.Q8_0, 3072, 3072),
             "to_out": (synth.Q8_0, 3072, 3072), "gate_up": (synth.Q8_0, 2 * 9216, 3072),
             "down": (synth.Q8_0, 3072, 9216)}
    wb = {n: (w[n][1] if isinstance(w[n], tuple) else w[n]) for n in w}
    blk = upload_block(ctx, qimm, synth, cfg, wb, types)
    rng = np.random.default_rng(12)
    x = rng.standard_normal((b, s, cfg["hidden"])).astype(np.float32)
    mod = (rng.standard_normal((b, 1, 4 * cfg["hidden"])) * 0.5).astype(np.float32)
    pe_h = qimm.rope_table([(1, 16, 16)], [0] * p + [1] * s)[p:]
    kpre = rng.standard_normal((b, cfg["heads"], p, HD)).astype(np.float32)
    vpre = rng.standard_normal((b, cfg["heads"], p, HD)).astype(np.float32)
    kb = torch.from_numpy(kpre).to(torch.bfloat16)
    vb = torch.from_numpy(vpre).to(torch.bfloat16)
    kv = ctx.kv_create(1, b, cfg["heads"], p)
    kd, vd = kb.cuda(), vb.cuda()
    sh = stream.cuda_stream
    kv.store(0, kd.data_ptr(), vd.data_ptr(), sh)
    xd = torch.from_numpy(x).cuda()
    xo = torch.empty_like(xd)
    md = torch.from_numpy(mod).cuda()
    ped = torch.from_numpy(np.ascontiguousarray(pe_h)).cuda()

    def call():
        blk.forward(xd.data_ptr(), xo.data_ptr(), b, s, md.data_ptr(), ped.data_ptr(), kv, 0, None, None, sh)

    ms = timed(torch, stream, call, iters, warmup=5)
    got = xo.cpu().numpy()
    blk.free()
    kv.free()
    flop = 2.0 * s * cfg["hidden"] * (4 * cfg["hidden"] + 3 * cfg["mlp"]) + 4.0 * cfg["heads"] * s * (s + p) * HD
    out = {"gpu_ms": round(ms, 4), "gflop": round(flop / 1e9, 2), "gpu_tflops": round(flop / ms / 1e9, 1),
           "weights": "Q8_0", "hidden": 3072, "heads": 24, "mlp": 9216, "tokens": s, "prefix_tokens": p}
    log(f"bench: config-1 block (hidden 3072, 256 tokens over 64): GPU {ms:.4f} ms")
    if cpu:
        kp16 = O.f32_to_bf16(kpre)
        vp16 = O.f32_to_bf16(vpre)
        O.lib()
        t0 = O.now()
        ref, _, _ = O.block_forward(cfg, w, x, mod, pe_h, kp16, vp16, mode=O.CANDLE)
        cpu_ms = (O.now() - t0) * 1e3
        cos = float((got.ravel().astype(np.float64) @ ref.ravel()) /
                    np.sqrt((got.ravel().astype(np.float64) ** 2).sum() * (ref.ravel().astype(np.float64) ** 2).sum()))
        out.update({"cpu_ms": round(cpu_ms, 1), "cpu_cores": O.num_threads(), "cpu_model": cpu_model(),
                    "cpu_isa": O.isa(), **cpu_counts(),
                    "cpu_kind": "port (oracle, candle mode: int8 activations, integer vec-dots)",
                    "gpu_vs_cpu_cosine": round(cos, 7)})
        log(f"bench: config-1 block on the CPU oracle: {cpu_ms:.1f} ms on {O.num_threads()} threads, "
            f"GPU/CPU output cosine {cos:.7f}")
    return out


def torch_sdpa_bar(torch, stream, iters=20):
    """torch's fused attention (flash or memory-efficient backend; the math backend is
    excluded) at the cached step's attention shape: B1, 32 heads, 4096 queries over
    4352 keys, bf16, as a practical bar for the joint-attention kernel on this GPU."""
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        import torch.nn.functional as F
        g = torch.Generator(device="cuda").manual_seed(3)
        q = torch.randn((1, HEADS, S_IMG, HD), generator=g, device="cuda").to(torch.bfloat16)
        k = torch.randn((1, HEADS, S_IMG + P_TXT, HD), generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn((1, HEADS, S_IMG + P_TXT, HD), generator=g, device="cuda").to(torch.bfloat16)
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            ms = timed(torch, stream, lambda: F.scaled_dot_product_attention(q, k, v), iters)
        flop = 4.0 * HEADS * S_IMG * (S_IMG + P_TXT) * HD
        log(f"bench: torch SDPA at the attention shape: {ms:.3f} ms, {flop / ms / 1e9:.0f} TFLOP/s")
        return {"ms": round(ms, 4), "tflops": round(flop / ms / 1e9, 1),
                "frac_bf16_peak": round(flop / ms / 1e9 / PEAK_BF16_TFLOPS, 4)}
    except Exception as e:  # no fused backend: report why, measure nothing
        log(f"bench: torch SDPA bar unavailable: {e}")
        return {"error": str(e)[:200]}


def torch_gemm_bar(torch, stream, iters=10):
    """torch's plain bf16 GEMM (hipBLASLt) at the block's four projection shapes
    with 4096 token rows, y = x W^T with W already bf16 (no dequantization, no
    fused epilogue): the practical bar for the dequant-GEMMs on this GPU."""
    out = {}
    g = torch.Generator(device="cuda").manual_seed(4)
    for name, (n, k) in (("qkv", (3 * HID, HID)), ("out", (HID, HID)), ("gate_up", (2 * MLP, HID)),
                         ("down", (HID, MLP))):
        x = torch.randn((S_IMG, k), generator=g, device="cuda").to(torch.bfloat16)
        w = torch.randn((n, k), generator=g, device="cuda").to(torch.bfloat16)
        with torch.cuda.stream(stream):
            ms = timed(torch, stream, lambda: torch.mm(x, w.t()), iters)
        tflops = 2.0 * S_IMG * n * k / ms / 1e9
        out[name] = {"ms": round(ms, 4), "tflops": round(tflops, 1), "frac_bf16_peak": round(tflops / PEAK_BF16_TFLOPS, 4)}
        log(f"bench: torch bf16 GEMM {S_IMG}x{n}x{k}: {ms:.3f} ms, {tflops:.0f} TFLOP/s")
    return out


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_block_q4km_1024.json")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE and WRITE_SIZE passes, each scaled by what the counter
    reads for a plain copy of known size), or None when it holds no figure."""
    try:
        with open(TRAFFIC_FILE) as f:
            data = json.load(f)
        k = data["kernels"][kernel]
        return {"bytes": int(k["traffic_bytes"]), "source": os.path.relpath(TRAFFIC_FILE, ROOT)}
    except (OSError, KeyError, ValueError):
        return None


def cpu_baseline(rows, host_w):
    """Oracle (candle mode: int8 activations, integer vec-dots, f32 attention)
    on `rows` token rows of the same block: the row work (LayerNorm and
    modulation, q/k RMSNorm and RoPE, SwiGLU, residuals), the six quantized
    matmuls and the attention of `rows` queries over all 4352 keys, scaled to
    the 4096-token step."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    O.use_native_build()
    w, shapes, _, _ = host_w
    rng = np.random.default_rng(3)
    x = rng.standard_normal((rows, HID)).astype(np.float32)
    h = rng.standard_normal((rows, MLP)).astype(np.float32)
    scale = (rng.standard_normal((1, HID)) * 0.1).astype(np.float32)
    gate = (rng.standard_normal((1, HID)) * 0.1).astype(np.float32)
    gu = rng.standard_normal((rows, 2 * MLP)).astype(np.float32)
    qk = rng.standard_normal((2, HEADS, rows, HD)).astype(np.float32)
    nw = np.ones(HD, dtype=np.float32)
    pe = O.rope_table([(1, GRID, GRID)], [1] * S_IMG)[:rows]
    O.lib()
    # the row work around the matmuls: two LayerNorm x (1 + scale), the q/k
    # RMSNorm and RoPE, SwiGLU and the two gated residual adds
    t0 = O.now()
    for _ in range(2):
        O.layernorm_mod(x, scale)
    for i in range(2):
        O.apply_rope(O.rmsnorm(qk[i], nw), pe)
    g = gu[:, :MLP]
    _ = g / (1.0 + np.exp(-g)) * gu[:, MLP:]
    for _ in range(2):
        _ = x + gate * x
    t_rows = O.now() - t0
    log(f"cpu baseline: row ops {t_rows:.2f}s")
    t_gemm = 0.0
    for name in ("to_q", "to_k", "to_v", "to_out", "gate_up", "down"):
        t, n, k = shapes[name]
        a = h if name == "down" else x
        t0 = O.now()
        O.qmatmul(t, w[name], n, k, a, O.CANDLE)
        t_gemm += O.now() - t0
        log(f"cpu baseline: {name} {O.now() - t0:.2f}s")
    q = rng.standard_normal((1, HEADS, rows, HD)).astype(np.float32)
    ko = rng.standard_normal((1, HEADS, S_IMG, HD)).astype(np.float32)
    vo = rng.standard_normal((1, HEADS, S_IMG, HD)).astype(np.float32)
    kp = rng.standard_normal((1, HEADS, P_TXT, HD)).astype(np.float32)
    vp = rng.standard_normal((1, HEADS, P_TXT, HD)).astype(np.float32)
    t0 = O.now()
    O.attention(q, ko, vo, kp, vp, mode=O.CANDLE)
    t_att = O.now() - t0
    log(f"cpu baseline: attention {t_att:.2f}s")
    scale = S_IMG / rows
    ms = (t_rows + t_gemm + t_att) * scale * 1e3
    return {"value": round(ms, 1), "unit": "ms/block-step", "cores": O.num_threads(), "cpu_model": cpu_model(),
            "isa": "-march=" + O.isa() if O.isa() == "native" else "-march=x86-64-v3 (native build failed)",
            **cpu_counts(), "kind": "port",
            "sample": f"{rows} of 4096 token rows through q/k/v/out/gate_up/down quantized matmuls, "
                      f"two LayerNorm x (1 + scale), q/k RMSNorm + RoPE, SwiGLU and the gated residuals, plus "
                      f"attention of {rows} queries over 4352 keys, timed and scaled x{scale:g}",
            "sample_seconds": round(t_rows + t_gemm + t_att, 2)}


if __name__ == "__main__":
    main()
