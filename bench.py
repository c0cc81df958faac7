#!/usr/bin/env python
"""Benchmark of the rational-attention kernel path on one MI355X.

A "step" is one causal bf16 rational-attention forward + backward (autograd
API: rational_attention(...) then out.backward(dO)) at B=4, H=16, S=4096,
D=128 with ALiBi, inputs resident in HBM. ``value`` is the algorithmic
throughput 7*B*H*S^2*D / step time in TFLOP/s. The same JSON line carries:
  * roofline  -- the dominant C-ABI call of the step (kat_attn_bwd or
                 kat_attn_fwd), timed with HIP events on its launch stream
                 inside the timed region, against the dense bf16 MFMA peak;
  * fused_ops -- HBM GB/s of mean_error_norm, rational_swiglu and
                 rational_softmax fwd+bwd at their benchmark shapes (bf16),
                 with the 256 MB last-level cache flushed before each rep
                 by reading (not writing) a 512 MB buffer, so no dirty lines
                 of the flush are written back inside the timed region;
  * cpu_baseline -- the CPU oracle (fp32) on a bounded sample of the same
                 workload (one (b, h) head), on this host's cores; and
    cpu_baselines -- the same for the fused ops (the full config-2 shapes)
                 and the config-4 training step (one block on a
                 2-row batch slice plus embed / head / loss, extrapolated);
  * config5_attention -- fwd+bwd of the 1.3 B model's attention shape
                 (B=2, H=16, S=8192, D=128, bf16);
  * head_dims  -- fwd+bwd at D = 32, 64 and 256 (bf16, S=4096, the headline's
                 B*H*D, so the same flops), all on the MFMA kernels;
  * fp32_attention -- fwd+bwd in fp32 (B=4, H=16, S=2048, D=64) on the fp32
                 MFMA kernels, against the 157.3 TFLOP/s fp32 peak;
  * attention_variants -- fwd+bwd of the padding-mask / non-causal attention
                 extension at the same shape (right-padded batch, non-causal,
                 both), TFLOP/s over the (query, key) pairs each attends;
  * decode     -- kat_attn_decode over bf16 KV caches (us per call, HBM GB/s
                 of the K and V bytes) and generate() tokens/s with the KV
                 cache against the reference's re-run-the-prefix loop;
  * device     -- CU count, measured bf16 MFMA loop rates (fixed and random
                 operands, beside the 2.5 PF spec peak), a measured 1 GiB
                 device-copy bandwidth, and power_scaling: equal-work
                 attention blocks on 64 vs 256 CUs (the clock drop under load);
  * model_step / model_step_large -- one training step (bf16 autocast
                 forward + loss + backward, no optimizer) of the 109.5 M-parameter
                 model at batch 16 x 2048 and of the 1.3 B-parameter model at
                 batch 2 x 8192 (reported, not the metric): tokens/s and MFU.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-fused]
                       [--no-variants] [--no-decode] [--no-model] [--no-model-large]
                       [--no-config5] [--no-head-dims]
       python bench.py --copy-calibration   (one plain 1 GiB device copy, for
                                             scaling HBM byte counters)
"""

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "attn fwd+bwd TFLOP/s (% MFMA peak) at S=4096; fused-op HBM GB/s (% peak)"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
PEAK_FP32_TFLOPS = 157.3   # MI355X fp32 (vector and dense matrix)

# HBM bytes per call at the benchmark shape come from the committed rocprofv3
# summary profiles/attention_bench_hbm_traffic.md: FETCH_SIZE and WRITE_SIZE
# passes over this bench (summed over the call's kernels), each scaled by what
# the same counter reads for a plain copy of known size. Its lines
# "traffic <call> <bytes>" are read here.
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "attention_bench_hbm_traffic.md")


def measured_traffic():
    """{call: bytes} from the summary's "traffic <call> <bytes>" lines, plus
    "commit" -> the commit its line "commit <sha>" names (the build that was
    profiled)."""
    out = {}
    try:
        for line in open(TRAFFIC_SUMMARY):
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic":
                out[parts[1]] = int(parts[2])
            elif len(parts) == 2 and parts[0] == "commit":
                out["commit"] = parts[1]
    except OSError:
        pass
    return out


def attention_inputs(torch, B, H, T, D, dev, seed=0, dtype=None):
    g = torch.Generator().manual_seed(seed)
    ts = [torch.randn(B, H, T, D, generator=g).to(dtype or torch.bfloat16) for _ in range(4)]
    return [t.to(dev) for t in ts]


def bench_attention(torch, F, steps, warmup, B=4, H=16, T=4096, D=128, dtype=None):
    dev = torch.device("cuda:0")
    q, k, v, do = attention_inputs(torch, B, H, T, D, dev, dtype=dtype)
    for t in (q, k, v):
        t.requires_grad_(True)
    slopes = torch.tensor([2.0 ** (-(i + 1) / 2) for i in range(H)], dtype=torch.float32,
                          device=dev)
    scale = 1.0 / math.sqrt(D)

    def step(ev=None):
        for t in (q, k, v):
            t.grad = None
        if ev is not None:
            ev[0].record()
        out = F.rational_attention(q, k, v, slopes, scale)
        if ev is not None:
            ev[1].record()
        out.backward(do)
        if ev is not None:
            ev[2].record()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    t0 = time.perf_counter()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        step(evs[i])
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / steps
    fwd = sorted(e[0].elapsed_time(e[1]) for e in evs)
    bwd = sorted(e[1].elapsed_time(e[2]) for e in evs)
    unit = B * H * T * T * D  # one causal S x S x D matmul = 2 * (S^2 / 2) * D flops
    return dict(ms=ms, wall_ms=wall * 1e3 / steps, fwd_ms=sum(fwd) / steps, bwd_ms=sum(bwd) / steps,
                fwd_median_ms=fwd[steps // 2], bwd_median_ms=bwd[steps // 2],
                flops_step=7 * unit, flops_fwd=2 * unit, flops_bwd=5 * unit)


def bench_config1(torch, F, steps=50, warmup=10, B=2, H=12, T=512, D=64):
    """the fp32 causal forward (B=2, H=12, S=512, D=64,
    slopes 2^(-8(i+1)/12), scale 1/8) the reference benchmarks against its
    PyTorch CPU path; the fp32 MFMA kernels run it. Also the fwd+bwd step.
    TFLOP/s count the same causal units as the headline (forward 2, fwd+bwd 7
    x B*H*S^2*D flop)."""
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(1)
    q, k, v, do = (torch.randn(B, H, T, D, generator=g).to(dev) for _ in range(4))
    slopes = torch.tensor([2.0 ** (-8.0 * (i + 1) / H) for i in range(H)], dtype=torch.float32,
                          device=dev)
    scale = 1.0 / math.sqrt(D)
    unit = B * H * T * T * D

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    fwd_ms = timed(lambda: F.rational_attention_forward(q, k, v, slopes, scale))
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))

    def step():
        for t in (qg, kg, vg):
            t.grad = None
        F.rational_attention(qg, kg, vg, slopes, scale).backward(do)
    step_ms = timed(step)
    return {"shape": {"B": B, "H": H, "S": T, "D": D}, "dtype": "fp32", "steps": steps,
            "kernels": "fp32 MFMA (v_mfma_f32_16x16x4_f32), forward and recompute backward",
            "fwd_ms": round(fwd_ms, 4), "fwd_TFLOPs": round(2 * unit / (fwd_ms * 1e-3) / 1e12, 3),
            "fwd_bwd_ms": round(step_ms, 4),
            "fwd_bwd_TFLOPs": round(7 * unit / (step_ms * 1e-3) / 1e12, 3),
            "frac_fp32_peak_fwd": round(2 * unit / (fwd_ms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS, 4)}


def bench_attention_variants(torch, F, steps=10, warmup=3, B=4, H=16, T=4096, D=128):
    """fwd+bwd of the masked / non-causal attention extension at the benchmark
    shape (bf16). TFLOP/s count the (query, key) pairs each variant attends:
    7 matmuls x 2 D flops per pair, the same accounting as the headline metric
    (whose causal pairs are ~T^2 / 2 per head)."""
    dev = torch.device("cuda:0")
    q, k, v, do = attention_inputs(torch, B, H, T, D, dev)
    for t in (q, k, v):
        t.requires_grad_(True)
    slopes = torch.tensor([2.0 ** (-(i + 1) / 2) for i in range(H)], dtype=torch.float32,
                          device=dev)
    scale = 1.0 / math.sqrt(D)
    lens = [T, T - T // 8, T - T // 4, T - 3 * T // 8]  # right padding, 0-37.5% of keys
    pad = torch.zeros(B, T, dtype=torch.bool)
    for b, n in enumerate(lens):
        pad[b, :n] = True
    out = {}
    for name, km, causal in (("causal_padded", pad, True), ("noncausal", None, False),
                             ("noncausal_padded", pad, False)):
        kmc = torch.ones(B, T, dtype=torch.bool) if km is None else km
        if causal:
            pairs = int(kmc.to(torch.int64).cumsum(1).sum()) * H
        else:
            pairs = int(kmc.to(torch.int64).sum(1).sum()) * T * H
        kmd = None if km is None else km.to(dev)

        def step():
            for t in (q, k, v):
                t.grad = None
            F.rational_attention_masked(q, k, v, slopes, scale, key_mask=kmd,
                                        causal=causal).backward(do)
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        flops = 7 * 2 * D * pairs
        out[name] = dict(ms=round(ms, 4), pairs=pairs, TFLOPs=round(flops / ms / 1e9, 2),
                         valid_keys=lens if km is not None else [T] * B)
    return out


def bench_decode(torch, F, reps=50):
    """kat_attn_decode (one query per (b, h) against a bf16 KV cache) at a
    few cache shapes: time per call and HBM GB/s of the K and V bytes it must
    read (2 B H n D x 2 bytes; q and out are negligible), from `reps` calls
    replayed in a HIP graph (`us`) and issued eagerly from Python
    (`us_eager_calls`, where the wrapper's host time shows); plus the model's
    generate() with its KV cache against the reference's loop, which re-runs
    the whole prefix for every token (algebraic_model.py:239-265)."""
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(3)
    res = {}
    for B, H, n, D in ((1, 16, 4096, 128), (16, 16, 4096, 128), (4, 16, 32768, 128)):
        q = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(dev)
        kc = torch.randn(B, n, H, D, generator=g).to(torch.bfloat16).to(dev)
        vc = torch.randn(B, n, H, D, generator=g).to(torch.bfloat16).to(dev)
        k4, v4 = kc.permute(0, 2, 1, 3), vc.permute(0, 2, 1, 3)
        slopes = torch.tensor([2.0 ** (-(i + 1) / 2) for i in range(H)], device=dev)
        for _ in range(5):
            F.rational_attention_decode(q, k4, v4, slopes, 1 / math.sqrt(D))
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            F.rational_attention_decode(q, k4, v4, slopes, 1 / math.sqrt(D))
        e1.record()
        torch.cuda.synchronize()
        us_eager = e0.elapsed_time(e1) / reps * 1e3
        # the same calls replayed from a captured HIP graph, as generate() runs
        # its decode step: the launch work of the Python wrapper drops out
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            F.rational_attention_decode(q, k4, v4, slopes, 1 / math.sqrt(D))
        torch.cuda.current_stream().wait_stream(st)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                F.rational_attention_decode(q, k4, v4, slopes, 1 / math.sqrt(D))
        graph.replay()
        torch.cuda.synchronize()
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / reps * 1e3
        del graph
        nbytes = 2 * B * H * n * D * 2
        res[f"B{B}_H{H}_n{n}_D{D}"] = dict(us=round(us, 2), us_eager_calls=round(us_eager, 2),
                                            bytes=nbytes, GBs=round(nbytes / us / 1e3, 1),
                                            frac_hbm_peak=round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4))
        del q, kc, vc, k4, v4
    # model generate: config-4 model, batch 8, 512-token prompt, 64 new tokens
    from fastalgebraictransformer_amd import AlgebraicTransformerLM
    torch.manual_seed(0)
    m = AlgebraicTransformerLM(32000, 768, 12, 12, dropout=0.0).to(dev).eval()
    prompt = torch.randint(0, 32000, (8, 512), device=dev)
    gen = {}
    for name, use_cache in (("kv_cache", True), ("reference_loop", False)):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            m.generate(prompt, 4, top_k=1, use_cache=use_cache)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            m.generate(prompt, 64, top_k=1, use_cache=use_cache)
            torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        gen[name] = dict(s=round(dt, 3), new_tokens_per_s=round(8 * 64 / dt, 1))
    gen["speedup"] = round(gen["reference_loop"]["s"] / gen["kv_cache"]["s"], 2)
    res["generate"] = dict(model="AlgebraicTransformerLM(32000, 768, 12, 12)", batch=8,
                           prompt=512, new_tokens=64, dtype="bf16 autocast", **gen)
    del m
    return res


def device_info(torch, lib):
    """CU count, measured MFMA loop rate and device-copy bandwidth."""
    import ctypes
    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(dev)
    cus = props.multi_processor_count
    blocks, iters = 8 * cus, 20000
    out = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
    flops = ctypes.c_double(0.0)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    best = 0.0
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        rc = lib.kat_probe_mfma_bf16(ctypes.c_void_p(out.data_ptr()), blocks, iters, ctypes.byref(flops), stream)
        e1.record()
        torch.cuda.synchronize()
        if rc != 0:
            raise RuntimeError("kat_probe_mfma_bf16 failed")
        best = max(best, flops.value / (e0.elapsed_time(e1) * 1e-3) / 1e12)
    # the same loop on random operands, two waves per SIMD, ~4 ms per launch so
    # that the clock settles: the MFMA rate real (toggling) data sustains
    rblocks, riters = cus, 10000
    rout = torch.empty(rblocks * 512, dtype=torch.float32, device=dev)
    rates = []
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        rc = lib.kat_probe_mfma_bf16_random(ctypes.c_void_p(rout.data_ptr()), rblocks, riters,
                                            ctypes.byref(flops), stream)
        e1.record()
        torch.cuda.synchronize()
        if rc != 0:
            raise RuntimeError("kat_probe_mfma_bf16_random failed")
        rates.append(flops.value / (e0.elapsed_time(e1) * 1e-3) / 1e12)
    rand_tflops = sorted(rates)[1]
    n = 1 << 29
    x = torch.ones(n, dtype=torch.bfloat16, device=dev)
    y = torch.empty_like(x)
    y.copy_(x)
    ts = []
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        y.copy_(x)
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    copy_gbs = 4 * n / (min(ts) * 1e-3) / 1e9  # 2 bytes read + 2 written per element
    del x, y, out, rout
    return {"name": props.name, "arch": getattr(props, "gcnArchName", ""), "cus": cus,
            "mfma_bf16_loop_tflops": round(best, 1),
            "mfma_bf16_random_operand_loop_tflops": round(rand_tflops, 1),
            "mfma_bf16_spec_tflops": PEAK_BF16_TFLOPS, "copy_1GiB_GBs": round(copy_gbs, 1),
            "hbm_spec_GBs": PEAK_HBM_GBS}


def power_scaling(torch, F):
    """The same attention blocks on more of the chip: the non-causal forward
    (kat_attn_fwd_masked, every 128-query block attends all 8192 keys, so all
    blocks do equal work) with 1, 4 and 8 heads: 64 blocks (64 CUs busy, one
    block each), 256 (every CU, one block each) and 512 (two per CU, the
    attention kernels' occupancy). Each size runs 30 calls back to back (a few
    ms, enough for the clock to settle). With a clock independent of load the
    first two would take equal time; the ratio is the slowdown the chip's
    power management imposes when every CU is busy."""
    from fastalgebraictransformer_amd import forward as FW
    dev = torch.device("cuda:0")
    T, D = 8192, 128
    res = {}
    for BH in (1, 4, 8):
        g = torch.Generator().manual_seed(0)
        q, k, v = (torch.randn(1, BH, T, D, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
        slopes = torch.full((BH,), 2.0 ** -8, device=dev)
        o = torch.empty_like(q)
        L = torch.empty(1, BH, T, device=dev)
        call = lambda: FW._attn_fwd_into(q, k, v, o, L, slopes, 1 / math.sqrt(D), False, 1e-6,
                                         extended=True)
        for _ in range(3):
            call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = 30
        e0.record()
        for _ in range(n):
            call()
        e1.record()
        torch.cuda.synchronize()
        res[f"blocks_{BH * T // 128}"] = round(e0.elapsed_time(e1) / n, 4)
    return {"workload": "non-causal bf16 forward, T=8192, D=128, 128 queries per block",
            "ms_per_call": res,
            "slowdown_256_vs_64_cus": round(res["blocks_256"] / res["blocks_64"], 3)}


MODEL_CONFIGS = {
    # config 4: the ~125M model, batch 16 x 2048 (default bench)
    "small": dict(vocab=32000, d_model=768, n_head=12, n_layers=12, d_ffn=None, batch=16, seq=2048),
    # config 5: the ~1.3B decoder at long context, batch 2 x 8192 (--model-large)
    "large": dict(vocab=50000, d_model=2048, n_head=16, n_layers=24, d_ffn=5632, batch=2, seq=8192),
}


def bench_model_step(torch, which="small", steps=5, warmup=2):
    """Training step of AlgebraicTransformerLM at a model config: bf16 autocast
    forward + cross-entropy, backward (no optimizer); random init from seed 0,
    token ids and labels uniform in [0, vocab)."""
    from fastalgebraictransformer_amd.algebraic_model import AlgebraicTransformerLM
    c = MODEL_CONFIGS[which]
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    model = AlgebraicTransformerLM(c["vocab"], c["d_model"], c["n_head"], c["n_layers"], d_ffn=c["d_ffn"],
                                   block_size=c["seq"]).to(dev)
    model.train()
    g = torch.Generator().manual_seed(0)
    B, S = c["batch"], c["seq"]
    ids = torch.randint(0, c["vocab"], (B, S), generator=g).to(dev)
    labels = torch.randint(0, c["vocab"], (B, S), generator=g).to(dev)

    def step():
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            _, loss = model(ids, labels)
        loss.backward()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    params = sum(p.numel() for p in model.parameters())
    peak_gib = torch.cuda.max_memory_allocated() / 2 ** 30
    # 6 N per token for the dense layers, plus causal attention fwd+bwd =
    # 7 B H S^2 D per layer (config 4: 25.86 TFLOP per step)
    D = c["d_model"] // c["n_head"]
    flops = 6 * params * B * S + c["n_layers"] * 7 * B * c["n_head"] * S * S * D
    del model, ids, labels
    torch.cuda.empty_cache()
    name = f"AlgebraicTransformerLM({c['vocab']}, {c['d_model']}, {c['n_head']}, {c['n_layers']}" + (
        f", d_ffn={c['d_ffn']})" if c["d_ffn"] else ")")
    return {"model": name, "params": params, "batch": [B, S], "ms_per_step": round(ms, 3),
            "tokens_per_s": round(B * S / (ms * 1e-3), 1),
            "tflops_step": round(flops / 1e12, 2), "mfu": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "peak_mem_gib": round(peak_gib, 1),
            "note": "reported, not the metric; dropout 0.1 (model default)"}


def bench_fused(torch, F, reps=10):
    """fwd+bwd of each fused op at the benchmark shapes; GB/s from the
    algorithmic bytes (each tensor read or written once)."""
    dev = torch.device("cuda:0")
    bf = torch.bfloat16
    g = torch.Generator().manual_seed(1)
    flush = torch.ones(512 * 1024 * 1024 // 4, dtype=torch.float32, device=dev)
    res = {}

    def timed(fn):
        # every rep: flush, then the step between two events; all reps are
        # enqueued before one synchronisation, so the host runs ahead of the
        # GPU and the events bracket the step's GPU work rather than Python's
        # dispatch latency in front of its first kernel
        evs = []
        for _ in range(reps + 2):
            flush.sum()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            evs.append((e0, e1))
        torch.cuda.synchronize()
        ts = sorted(e0.elapsed_time(e1) for e0, e1 in evs[2:])
        return ts[len(ts) // 2]

    # mean_error_norm: x [16384, 4096] bf16, gamma fp32
    N, C = 16384, 4096
    x = torch.randn(N, C, generator=g).to(bf).to(dev).requires_grad_(True)
    w = (1 + 0.02 * torch.randn(C, generator=g)).to(dev).requires_grad_(True)
    dy = torch.randn(N, C, generator=g).to(bf).to(dev)

    def norm_step():
        x.grad = w.grad = None
        F.mean_error_norm(x, w).backward(dy)
    nbytes = (2 * N * C * 2 + C * 4 + N * 4) + (3 * N * C * 2 + 2 * C * 4 + N * 4)
    t = timed(norm_step)
    res["mean_error_norm"] = dict(shape=[N, C], ms=t, bytes=nbytes, GBs=nbytes / t / 1e6)
    del x, dy

    # residual add fused with the norm: fp32 stream x [16384, 4096] plus a
    # bf16 branch r (the model under autocast); beside it the unfused pair
    # (torch add, then the norm) it replaces
    xs = torch.randn(N, C, generator=g).to(dev).requires_grad_(True)
    rb = torch.randn(N, C, generator=g).to(bf).to(dev).requires_grad_(True)
    dh = torch.randn(N, C, generator=g).to(dev)
    dy = torch.randn(N, C, generator=g).to(dev)

    def add_norm_step():
        xs.grad = rb.grad = w.grad = None
        h, y = F.add_mean_error_norm(xs, rb, w)
        torch.autograd.backward([h, y], [dh, dy])

    def add_then_norm_step():
        xs.grad = rb.grad = w.grad = None
        h = xs + rb
        torch.autograd.backward([h, F.mean_error_norm(h, w)], [dh, dy])
    # fwd: x, r read, h, y written; bwd: dy, dh, h read, dx, dr written
    nbytes = N * C * (4 + 2 + 4 + 4) + N * C * (4 + 4 + 4 + 4 + 2) + 3 * C * 4 + 2 * N * 4
    t = timed(add_norm_step)
    t_unfused = timed(add_then_norm_step)
    res["add_mean_error_norm"] = dict(shape=[N, C], ms=t, bytes=nbytes, GBs=nbytes / t / 1e6,
                                      unfused_ms=t_unfused)
    del xs, rb, dh, dy, w

    # rational_swiglu: gate, value [16384, 11008] bf16
    N, C = 16384, 11008
    ga = torch.randn(N, C, generator=g).to(bf).to(dev).requires_grad_(True)
    va = torch.randn(N, C, generator=g).to(bf).to(dev).requires_grad_(True)
    dy = torch.randn(N, C, generator=g).to(bf).to(dev)

    def swiglu_step():
        ga.grad = va.grad = None
        F.rational_swiglu(ga, va).backward(dy)
    nbytes = 3 * N * C * 2 + 5 * N * C * 2
    t = timed(swiglu_step)
    res["rational_swiglu"] = dict(shape=[N, C], ms=t, bytes=nbytes, GBs=nbytes / t / 1e6)
    del ga, va, dy

    # rational_softmax: scores [4096, 4096] ~ N(0, 4) bf16
    N, C = 4096, 4096
    s = (2 * torch.randn(N, C, generator=g)).to(bf).to(dev).requires_grad_(True)
    dy = torch.randn(N, C, generator=g).to(bf).to(dev)

    def softmax_step():
        s.grad = None
        F.rational_softmax(s).backward(dy)
    nbytes = 2 * N * C * 2 + 4 * N * C * 2
    t = timed(softmax_step)
    res["rational_softmax"] = dict(shape=[N, C], ms=t, bytes=nbytes, GBs=nbytes / t / 1e6)
    for r in res.values():
        r["frac_hbm_peak"] = r["GBs"] / PEAK_HBM_GBS
    return res


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_threads(torch):
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    return cores


def cpu_baselines(torch):
    """The CPU oracle (fp32 on the bf16-rounded inputs) on the other measured
    workloads, on this host's cores: the fused ops fwd+bwd at the full config-2
    shapes, and the config-4 training step extrapolated from one
    AlgebraicBlock fwd+bwd on a 2-row batch slice at T = 2048 (the reference's
    CPU attention, torch norm and SwiGLU formulas) plus the embedding, head and
    loss on the same slice."""
    import oracle as O
    cores = _cpu_threads(torch)
    g = torch.Generator().manual_seed(1)
    bf = torch.bfloat16
    res = {}

    def timed(fn):
        t0 = time.perf_counter()
        fn()
        return time.perf_counter() - t0

    def rowop(name, rows, cols, nbytes, fn, reps=3):
        ts = sorted(timed(fn) for _ in range(reps))
        t = ts[len(ts) // 2]
        res[name] = {"value": round(nbytes / t / 1e9, 2), "unit": "GB/s", "cores": cores,
                     "kind": "port",
                     "sample": f"the full [{rows}, {cols}] shape, oracle fp32 fwd+bwd, median of "
                               f"{reps} ({t:.2f} s); the GPU line's algorithmic bytes"}

    N, C = 16384, 4096
    x = torch.randn(N, C, generator=g).to(bf)
    w = 1 + 0.02 * torch.randn(C, generator=g)
    dy = torch.randn(N, C, generator=g).to(bf)

    def norm():
        _, mu = O.mean_error_norm_fwd(x, w, dtype=torch.float32)
        O.mean_error_norm_bwd(dy, x, w, mu, dtype=torch.float32)
    rowop("mean_error_norm", N, C, (2 * N * C * 2 + C * 4 + N * 4) + (3 * N * C * 2 + 2 * C * 4 + N * 4),
          norm)
    del x, dy
    N, C = 16384, 11008
    ga, va, dy2 = (torch.randn(N, C, generator=g).to(bf) for _ in range(3))

    def swiglu():
        O.swiglu_fwd(ga, va, dtype=torch.float32)
        O.swiglu_bwd(dy2, ga, va, dtype=torch.float32)
    rowop("rational_swiglu", N, C, 8 * N * C * 2, swiglu)
    del ga, va, dy2
    N, C = 4096, 4096
    sx = (2 * torch.randn(N, C, generator=g)).to(bf)
    dy3 = torch.randn(N, C, generator=g).to(bf)

    def softmax():
        p = O.rational_softmax_fwd(sx, dtype=torch.float32)
        O.rational_softmax_bwd(dy3, sx, p, dtype=torch.float32)
    rowop("rational_softmax", N, C, 6 * N * C * 2, softmax)

    # config 4: one block on 2 x 2048 tokens, then embedding + head + loss
    from fastalgebraictransformer_amd.algebraic_model import AlgebraicBlock
    torch.manual_seed(0)
    blk = AlgebraicBlock(768, 12, 2048, dropout=0.0)
    xb = torch.randn(2, 2048, 768, generator=g, requires_grad=True)

    def block():
        blk(xb).backward(torch.ones(2, 2048, 768))
    tb = timed(block)
    emb = torch.nn.Embedding(32000, 768)
    ids = torch.randint(0, 32000, (2, 2048), generator=g)

    def head():
        h = emb(ids)
        logits = torch.nn.functional.linear(h, emb.weight)
        torch.nn.functional.cross_entropy(logits.view(-1, 32000), ids.view(-1)).backward()
    th = timed(head)
    step = 8 * (12 * tb + th)  # 16 rows = 8 slices of 2; 12 blocks
    res["model_step"] = {"value": round(16 * 2048 / step, 1), "unit": "tokens/s", "cores": cores,
                         "kind": "port",
                         "sample": f"EXTRAPOLATION: AlgebraicTransformerLM(32000, 768, 12, 12) step at "
                                   f"16 x 2048 = 8 x (12 x one block fwd+bwd on 2 x 2048 tokens "
                                   f"[{tb:.2f} s] + embedding/head/loss on 2 x 2048 [{th:.2f} s]), fp32"}
    return res


def cpu_baseline(torch, S=4096, D=128, reps=3):
    """CPU oracle (fp32) forward + backward of one (b, h) head of the workload
    (heads are independent, so this is an exact 1/64 slice), on every core this
    process may run on."""
    import oracle as O
    cores = _cpu_threads(torch)
    g = torch.Generator().manual_seed(0)
    q, k, v, do = (torch.randn(1, 1, S, D, generator=g).to(torch.bfloat16) for _ in range(4))
    slopes = torch.tensor([2.0 ** -0.5])
    scale = 1.0 / math.sqrt(D)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        o, L = O.attention_fwd(q, k, v, slopes, scale, dtype=torch.float32)
        O.attention_bwd(q, k, v, o, L, do, slopes, scale, dtype=torch.float32)
        ts.append(time.perf_counter() - t0)
    t = sorted(ts)[len(ts) // 2]
    flops = 7 * S * S * D
    return {"value": flops / t / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"1 of 64 (b,h) heads at S={S}, D={D}: oracle fp32 fwd+bwd, "
                      f"median of {reps} ({t:.2f} s per head); {cpu_model()}, "
                      f"affinity {cores} of os.cpu_count() {os.cpu_count()}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-fused", action="store_true")
    ap.add_argument("--no-variants", action="store_true",
                    help="skip the masked / non-causal attention variants")
    ap.add_argument("--no-decode", action="store_true",
                    help="skip the KV-cache decode attention and generate() timings")
    ap.add_argument("--no-model", action="store_true", help="skip the model training step")
    ap.add_argument("--no-model-large", action="store_true",
                    help="skip the ~1.3B model step (batch 2 x 8192, ~47 GB; reported only)")
    ap.add_argument("--no-config5", action="store_true",
                    help="skip the attention fwd+bwd at the 1.3B model's shape (B=2, H=16, S=8192)")
    ap.add_argument("--no-head-dims", action="store_true",
                    help="skip the attention fwd+bwd at D = 32, 64 and 256 and in fp32")
    ap.add_argument("--no-device", action="store_true", help="skip the MFMA / copy probes")
    ap.add_argument("--no-config1", action="store_true",
                    help="skip the config-1 fp32 attention timing (B=2, H=12, S=512, D=64)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain device-to-device copy of 1 GiB (3 times): the "
                         "reference for scaling the FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the kernels shard by (batch, head) with no communication; see the design notes)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    if args.copy_calibration:
        assert torch.cuda.is_available(), "bench.py needs a GPU"
        n = 1 << 29  # bf16 elements: 1 GiB read + 1 GiB written per copy
        x = torch.ones(n, dtype=torch.bfloat16, device="cuda:0")
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": 2 * n, "copy_calibration_bytes_written": 2 * n,
                          "copies": 3}), flush=True)
        return
    import fastalgebraictransformer_amd as F
    from fastalgebraictransformer_amd import _lib
    _lib.load()
    assert torch.cuda.is_available(), "bench.py needs a GPU"

    att = bench_attention(torch, F, args.steps, args.warmup)
    value = att["flops_step"] / (att["ms"] * 1e-3) / 1e12
    fwd_tf = att["flops_fwd"] / (att["fwd_ms"] * 1e-3) / 1e12
    bwd_tf = att["flops_bwd"] / (att["bwd_ms"] * 1e-3) / 1e12
    dom = "kat_attn_bwd" if att["bwd_ms"] >= att["fwd_ms"] else "kat_attn_fwd"
    ach = bwd_tf if dom == "kat_attn_bwd" else fwd_tf
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(att["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (q, k, v, dO ~ N(0,1) from seed 0)",
        "config": {"workload": "rational_attention fwd+bwd, causal, ALiBi, bf16 in / fp32 acc",
                   "B": 4, "H": 16, "S": 4096, "D": 128,
                   "slopes": "2^(-(i+1)/2)", "scale": "1/sqrt(128)"},
        "roofline": {"bound": "mfma", "call": dom, "achieved": round(ach, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(ach / PEAK_BF16_TFLOPS, 4),
                     "traffic": measured_traffic().get(dom),
                     "traffic_source": {"profile": os.path.relpath(TRAFFIC_SUMMARY, ROOT),
                                        "commit": measured_traffic().get("commit")}},
        "kernels": {"kat_attn_fwd": {"ms": round(att["fwd_ms"], 4), "median_ms": round(att["fwd_median_ms"], 4),
                                     "TFLOPs": round(fwd_tf, 2), "algorithmic_flops": att["flops_fwd"]},
                    "kat_attn_bwd": {"ms": round(att["bwd_ms"], 4), "median_ms": round(att["bwd_median_ms"], 4),
                                     "TFLOPs": round(bwd_tf, 2), "algorithmic_flops": att["flops_bwd"]}},
        "frac_mfma_peak_step": round(value / PEAK_BF16_TFLOPS, 4),
    }
    if not args.no_config5:
        a5 = bench_attention(torch, F, 10, 3, B=2, H=16, T=8192, D=128)
        t5 = a5["flops_step"] / (a5["ms"] * 1e-3) / 1e12
        line["config5_attention"] = {
            "shape": {"B": 2, "H": 16, "S": 8192, "D": 128}, "dtype": "bf16", "steps": 10,
            "ms_per_step": round(a5["ms"], 4), "TFLOPs": round(t5, 2),
            "frac_mfma_peak": round(t5 / PEAK_BF16_TFLOPS, 4),
            "fwd_ms": round(a5["fwd_ms"], 4), "bwd_ms": round(a5["bwd_ms"], 4)}
    if not args.no_head_dims:
        hd = {}
        for Dh, Hh in ((32, 64), (64, 32), (256, 8)):
            ah = bench_attention(torch, F, 10, 3, B=4, H=Hh, T=4096, D=Dh)
            th = ah["flops_step"] / (ah["ms"] * 1e-3) / 1e12
            hd[f"D{Dh}"] = {"shape": {"B": 4, "H": Hh, "S": 4096, "D": Dh}, "ms_per_step": round(ah["ms"], 4),
                            "TFLOPs": round(th, 2), "frac_mfma_peak": round(th / PEAK_BF16_TFLOPS, 4),
                            "fwd_ms": round(ah["fwd_ms"], 4), "bwd_ms": round(ah["bwd_ms"], 4)}
        line["head_dims"] = hd
        af = bench_attention(torch, F, 10, 3, B=4, H=16, T=2048, D=64, dtype=torch.float32)
        tf = af["flops_step"] / (af["ms"] * 1e-3) / 1e12
        line["fp32_attention"] = {
            "shape": {"B": 4, "H": 16, "S": 2048, "D": 64}, "dtype": "fp32",
            "kernels": "fp32 MFMA (v_mfma_f32_16x16x4_f32)", "ms_per_step": round(af["ms"], 4),
            "TFLOPs": round(tf, 2), "frac_fp32_peak": round(tf / PEAK_FP32_TFLOPS, 4),
            "fwd_ms": round(af["fwd_ms"], 4), "bwd_ms": round(af["bwd_ms"], 4),
            "fwd_TFLOPs": round(af["flops_fwd"] / (af["fwd_ms"] * 1e-3) / 1e12, 2),
            "bwd_TFLOPs": round(af["flops_bwd"] / (af["bwd_ms"] * 1e-3) / 1e12, 2)}
    if not args.no_config1:
        line["config1_fp32"] = bench_config1(torch, F)
    if not args.no_variants:
        line["attention_variants"] = bench_attention_variants(torch, F)
    if not args.no_decode:
        line["decode"] = bench_decode(torch, F)
    if not args.no_fused:
        fused = bench_fused(torch, F)
        line["fused_ops"] = {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                                 for kk, vv in r.items()} for k, r in fused.items()}
    if not args.no_device:
        line["device"] = device_info(torch, _lib.load())
        line["device"]["power_scaling"] = power_scaling(torch, F)
    if not args.no_model:
        line["model_step"] = bench_model_step(torch, "small")
    if not args.no_model_large:
        line["model_step_large"] = bench_model_step(torch, "large", steps=3, warmup=1)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(torch)
        line["cpu_baseline"]["value"] = round(line["cpu_baseline"]["value"], 5)
        line["cpu_baselines"] = cpu_baselines(torch)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
