#!/usr/bin/env python3
"""Benchmark of the MI355X paged KV-cache attention path (one GPU).

Headline workload: Qwen3-4B-shape decode, batch 1 --
one step = the op genllm_paged_attention (PagedAttentionImpl::execute):
append one token's K/V, then split-K attention over ~8193 cached keys
(q [1,32,1,128], 8 KV heads, 512+ pages drawn from a shuffled 2048-page pool).
Steps rotate over 16 independent layers (~540 MB of touched KV) so the 256 MB
MALL cannot serve them; each layer's context grows by one token per visit, as
in a real decode loop, and the algorithmic bytes are counted per step.

value = whole-step algorithmic HBM bytes / GPU time of the op step (GB/s):
one HIP event pair on the launch stream around the timed steps, queued while a
bounded spin kernel holds the GPU, so the events see GPU time only; the same
steps with the host in the loop (wall clock) and the host cost of one op call,
from Python and from C++ (tests/cpp/test_ops_hip --host-cost), are reported
beside it under "host".  roofline = the dominant kernels (paged_decode_kernel,
split-K attention, then paged_decode_merge_kernel, the log-sum-exp merge of the
splits) timed alone the same way, against 8 TB/s.  The kernel time may not
exceed the op step's time; the bench exits with an error if it does.  Its HBM
traffic is measured in the same run: two child rocprofv3 --pmc passes
(FETCH_SIZE, WRITE_SIZE) over the same launches and a 256 MiB copy that scales
the counters, started before this process touches the GPU.
Secondary figures (same line): the headline op step on fp16 layers, config 2
fused append GB/s, config 4 causal
prefill TFLOPS, the non-paged FlashAttention path at config 4's shape, the
Qwen3.5 shape (head_dim 256, 8 q / 2 kv heads: 8K-context decode GB/s and
2048-token prefill TFLOPS), config 5 36-layer long-context decode (eager and
replayed as one HIP graph), and the Qwen3-4B fused Q/K/V projection feeding
the path (decode GEMV GB/s, 2048-token GEMM TFLOPS).  cpu_baseline = the
oracle (single thread) on a bounded sample of the headline workload.

--only {headline,f16,append,prefill,flash,qwen35,longctx,linear,copy,traffic,
prefill_scale,decode_scale} runs one workload alone (for rocprofv3 passes);
the line then carries only that workload's figures.  prefill_scale (the
prefill kernel at 2K-16K tokens) and decode_scale (the decode kernels at
8K-256K keys) run only this way.  --no-traffic skips the child counter passes (they are
skipped anyway when the bench itself runs under rocprofv3).
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import shutil
import statistics
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "paged decode attn µs/layer + achieved HBM GB/s (Qwen3-4B, 8K ctx); prefill TFLOPS"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
PAGE = 16
COPY_MIB = 256  # calibration copy of the counter passes


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=16, help="rotation depth of the headline workload")
    ap.add_argument("--only", choices=["headline", "f16", "append", "prefill", "flash", "qwen35", "longctx", "linear",
                                       "copy", "traffic", "prefill_scale", "decode_scale"], default=None)
    ap.add_argument("--no-traffic", action="store_true", help="skip the child rocprofv3 --pmc traffic passes")
    ap.add_argument("--skip-secondary", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    return ap.parse_args()


def decode_step_bytes(n_keys: int, Hq=32, Hkv=8, D=128) -> int:
    """Algorithmic bytes of one op step: K/V reads of n_keys tokens, the appended
    token's K/V read + write, q read, out write, page ids (k and v) read."""
    kv = n_keys * Hkv * D * 2 * 2
    append = 2 * (2 * Hkv * D * 2)
    qo = 2 * Hq * D * 2
    ids = ((n_keys + PAGE - 1) // PAGE) * 8
    return kv + append + qo + ids


def decode_kernel_bytes(n_keys: int, Hq=32, Hkv=8, D=128) -> int:
    """K/V of n_keys tokens + q + out + page ids."""
    return n_keys * Hkv * D * 2 * 2 + 2 * Hq * D * 2 + ((n_keys + PAGE - 1) // PAGE) * 8


def time_kernels(torch, fn, n, warm=5):
    """GPU time per launch of fn(i): one pair of HIP events on the launch
    stream around n back-to-back launches, queued while the GPU is held busy by
    a bounded spin kernel so that it never waits for the host.  (An event pair
    around every launch would add about 2 us to each and 7 us per launch to
    the timeline at this size, measured on MI355X.)"""
    host_s = 0.0
    for i in range(warm):
        t0 = time.perf_counter()
        fn(i)
        host_s = max(host_s, time.perf_counter() - t0)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # hold the GPU (~2.4e9 spin cycles per second) for 3x the host's queueing time
    torch.cuda._sleep(int(2.4e9 * max(0.002, 3.0 * n * (host_s + 20e-6))))
    start.record(stream)
    for i in range(n):
        fn(warm + i)
    stop.record(stream)
    torch.cuda.synchronize()
    return 1e3 * start.elapsed_time(stop) / n


# ----------------------------------------------------------- read floors
_probe = None


def probe_lib():
    """libgenllm_probe.so (genllm_amd/csrc/probes.hip): read-floor probes that
    move exactly one kernel's bytes with its access pattern and no arithmetic."""
    global _probe
    if _probe is None:
        import ctypes as C
        L = C.CDLL(os.path.join(ROOT, "genllm_amd", "libgenllm_probe.so"))
        P, i32 = C.c_void_p, C.c_int32
        L.genllm_probe_stream_read.argtypes = [P, C.c_size_t, P, P]
        L.genllm_probe_decode_read.argtypes = [P, P, P, P, i32, i32, i32, i32, i32, P, P]
        L.genllm_probe_append_copy.argtypes = [P, P, P, P, P, P, i32, i32, i32, P]
        _probe = L
    return _probe


def _probe_call(name, *args):
    rc = getattr(probe_lib(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed ({rc})")


def decode_pps(torch, n_pages, Hkv, D=128):
    """The decode kernel's default plan: pages per split (about one workgroup
    per CU) and kv heads per workgroup (4 once a one-head plan reaches 48
    pages per split, for head_dim 128 and kv heads in groups of 4)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    pps, heads = max(2, -(-n_pages * Hkv // cus)), 1
    if D == 128 and Hkv % 4 == 0 and pps >= 48:
        pps, heads = max(2, -(-n_pages * (Hkv // 4) // cus)), 4
    return max(pps, -(-n_pages // 256)), heads


def floor_entry(probe_us, nbytes, kernel_us, what):
    gbs = nbytes / (probe_us * 1e-6) / 1e9
    return {"probe_us": round(probe_us, 3), "bytes": nbytes, "GB_s": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "kernel_us": round(kernel_us, 3),
            "kernel_over_probe": round(kernel_us / probe_us, 3), "probe": what}


def stream_floor(torch, nbytes, copies, iters=40):
    """A contiguous stream of nbytes, rotating over `copies` buffers (more than
    the 256 MB MALL holds), 16-byte nontemporal loads."""
    bufs = [torch.empty(nbytes // 2, dtype=torch.bfloat16, device="cuda") for _ in range(copies)]
    for b in bufs:
        b.zero_()
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    us = time_kernels(torch, lambda i: _probe_call("genllm_probe_stream_read", bufs[i % copies].data_ptr(),
                                                   (nbytes // 16) * 16, sink.data_ptr(), stream), iters)
    del bufs
    return us


# ----------------------------------------------------------------- headline
HQ3, HKV3, D3, POOL3, N3 = 32, 8, 128, 2048, 8192
DECODE_KERNEL_LABEL = ("paged_decode_kernel<128, 8> (split-K attention, split merge in the same launch)"
                       if os.environ.get("GENLLM_DECODE_MERGE") == "fused" else
                       "paged_decode_kernel<128, 8> + paged_decode_merge_kernel<128, 4> (split-K attention, "
                       "then the log-sum-exp merge of the splits)")


def decode_layers(np, torch, paged, synth, call, L, f16=False):
    """L Qwen3-4B-shape layers of config 3: 8192 cached tokens each in a
    shuffled 2048-page pool, pools ~ N(0,1), and per layer a q, k, v of one
    token; bf16 layers, or fp16 layers with f16."""
    Hq, Hkv, D, pool_pages, n0 = HQ3, HKV3, D3, POOL3, N3
    seed = synth.config_seed(3)
    fill = "genllm_fill_normal_f16" if f16 else "genllm_fill_normal_bf16"
    gen = synth.normal_f16 if f16 else synth.normal_bf16
    dev = paged.to_device_f16 if f16 else paged.to_device_bf16
    mgr = paged.PagedAttentionManager(L * 2 * pool_pages * PAGE * Hkv * D * 2)
    for l in range(L):
        mgr.init_layer(l, Hkv, D, paged.DTYPE_F16 if f16 else paged.DTYPE_BF16)
        mgr.reserve_layer(l, pool_pages)
        mgr.fragment(l, synth.shuffled(seed + 2 * l, pool_pages), synth.shuffled(seed + 2 * l + 1, pool_pages))
        mgr.append_kv_pages(l, n0)
        info = mgr.get_layer(l)
        n_el = pool_pages * PAGE * Hkv * D
        call(fill, info.k_pool, n_el, seed + 100 + l, 0, None)
        call(fill, info.v_pool, n_el, seed + 200 + l, 0, None)
    q = [dev(gen(seed + 300 + l, (1, Hq, 1, D))) for l in range(L)]
    kn = [dev(gen(seed + 400 + l, (1, Hkv, 1, D))) for l in range(L)]
    vn = [dev(gen(seed + 500 + l, (1, Hkv, 1, D))) for l in range(L)]
    torch.cuda.synchronize()
    return mgr, q, kn, vn, seed


def time_op_steps(torch, op_step, args):
    """The op step timed two ways.  host_loop_s: wall clock around the steps
    issued one after another from Python (host in the loop; labelled, not the
    value).  step_s: one HIP event pair on the launch stream around the same
    number of further steps, queued while a bounded spin kernel holds the GPU,
    so that it never waits for the host (as the roofline kernel is timed);
    queue_s is the host time per call meanwhile.  op_step(i) returns the
    step's algorithmic bytes; total_bytes is the sum over the event-timed
    steps.  Returns (host_loop_s, step_s, queue_s, total_bytes)."""
    for i in range(args.warmup):
        op_step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        op_step(args.warmup + i)
    torch.cuda.synchronize()
    host_loop_s = (time.perf_counter() - t0) / args.steps
    base = args.warmup + args.steps
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(2.4e9 * max(0.002, 3.0 * args.steps * (host_loop_s + 20e-6))))
    start.record(stream)
    total_bytes = 0
    q0 = time.perf_counter()
    for i in range(args.steps):
        total_bytes += op_step(base + i)
    queue_s = (time.perf_counter() - q0) / args.steps
    stop.record(stream)
    torch.cuda.synchronize()
    step_s = 1e-3 * start.elapsed_time(stop) / args.steps
    return host_loop_s, step_s, queue_s, total_bytes


def decode_launcher(np, torch, paged, mgr, q, L):
    """fn(i): one stateless decode launch (genllm_paged_decode) over layer i % L
    at 8193 cached keys -- the headline's dominant kernel alone."""
    Hq, Hkv, D, n_keys = HQ3, HKV3, D3, N3 + 1
    ws = torch.zeros(paged.decode_workspace_bytes(Hq, Hkv, 1, D, POOL3), dtype=torch.uint8, device="cuda")
    infos = [mgr.get_layer(l) for l in range(L)]
    o2 = torch.empty((Hq, 1, D), dtype=torch.bfloat16, device="cuda")
    qh = [t.view(Hq, 1, D) for t in q]
    scale = 1.0 / np.sqrt(D)

    def launch(i):
        inf = infos[i % L]
        paged.paged_decode(qh[i % L], o2, inf.k_pool, inf.v_pool, inf.k_ids, inf.v_ids, (n_keys + 15) // 16,
                           n_keys, Hkv, scale, ws)

    return launch, n_keys


def headline(args, np, torch, paged, synth, call):
    Hq, Hkv, D = HQ3, HKV3, D3
    G = Hq // Hkv
    scale = 1.0 / np.sqrt(D)
    pool_pages, n0, L = POOL3, N3, args.layers
    mgr, q, kn, vn, seed = decode_layers(np, torch, paged, synth, call, L)
    out = [torch.empty((1, Hq, 1, D), dtype=torch.bfloat16, device="cuda") for _ in range(L)]
    cached = [n0] * L

    def op_step(i):
        l = i % L
        paged.paged_attention(mgr, l, q[l], kn[l], vn[l], out[l], G, scale)
        cached[l] += 1
        return decode_step_bytes(cached[l])

    # value and ms_per_step: the GPU time of the op step; the wall clock of the
    # host loop beside it
    host_loop_s, step_s, queue_s, total_bytes = time_op_steps(torch, op_step, args)

    # dominant kernels alone: the split-K decode and its merge kernel, 8193
    # keys, rotating over the same 16 layers
    kernel_launch, n_keys = decode_launcher(np, torch, paged, mgr, q, L)
    n_k = max(args.steps, 200)
    k_mean = time_kernels(torch, kernel_launch, n_k, warm=args.warmup)
    if k_mean > 1.03 * step_s * 1e6:  # once more before refusing
        k_mean = time_kernels(torch, kernel_launch, n_k, warm=args.warmup)
    if k_mean > 1.03 * step_s * 1e6:
        print(f"bench.py: inconsistent timing -- the decode kernels alone ({k_mean:.2f} us per launch) take "
              f"longer than the whole op step ({step_s * 1e6:.2f} us); refusing to report", file=sys.stderr)
        sys.exit(3)
    kbytes = decode_kernel_bytes(n_keys)
    achieved = kbytes / (k_mean * 1e-6) / 1e9
    # read floors: the split kernel's exact page loads without the math (same
    # plan, same rotating layers), and a contiguous stream of the same bytes
    n_pages = (n_keys + PAGE - 1) // PAGE
    pps, hpw = decode_pps(torch, n_pages, HKV3)
    infos = [mgr.get_layer(l) for l in range(L)]
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    cs = torch.cuda.current_stream().cuda_stream
    pat_us = time_kernels(torch, lambda i: _probe_call(
        "genllm_probe_decode_read", infos[i % L].k_pool, infos[i % L].v_pool, infos[i % L].k_ids,
        infos[i % L].v_ids, n_pages, HKV3, D3, pps, hpw, sink.data_ptr(), cs), n_k, warm=args.warmup)
    str_us = stream_floor(torch, kbytes, 16)
    floors = {"decode_config3_pattern": floor_entry(pat_us, kbytes, k_mean,
                                                    f"the split kernel's page loads, {pps} pages per split, "
                                                    f"{hpw} kv head(s) per workgroup, no math, no merge"),
              "decode_config3_stream": floor_entry(str_us, kbytes, k_mean, "contiguous stream of the same bytes")}
    res = {
        "value": round(total_bytes / (step_s * args.steps) / 1e9, 1),
        "ms_per_step": round(step_s * 1e3, 5),
        "us_per_layer": round(step_s * 1e6, 2),
        "step_timing": "GPU time of the op step: one HIP event pair on the launch stream around the timed steps, "
                       "queued behind a spin kernel (the GPU never waits for the host)",
        "host": {"loop_us_per_step": round(host_loop_s * 1e6, 2),
                 "loop_note": "wall clock of the same op steps issued one after another from Python, host in the loop",
                 "python_us_per_call": round(queue_s * 1e6, 2),
                 "python_note": "host time of one op call from Python (asserts, ctypes, C bookkeeping, two launches)"},
        "config": {"workload": "BASELINE config 3: Qwen3-4B-shape paged decode, batch 1, 8K context, "
                               "append 1 token then attend (op genllm_paged_attention)",
                   "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "context_start": n0 + 1,
                   "context_end": max(cached), "pool_pages": pool_pages, "rotating_layers": L},
        "roofline": {"kernel": DECODE_KERNEL_LABEL,
                     "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": kbytes, "avg_launch_us": round(k_mean, 3), "launches": n_k,
                     "timing": "one HIP event pair on the launch stream around back-to-back launches (GPU kept "
                               "fed: host queued ahead behind a spin kernel) / launches"},
        "read_floor": floors,
    }
    return res, mgr, seed


# ---------------------------------------------------------------- secondary
def f16_config3(args, np, torch, paged, synth, call):
    """The headline op step on fp16 layers (fp16 K/V pools, q and out): the
    same shape, rotation and timing, the fp16 MFMAs in the split kernel."""
    Hq, Hkv, D, L = HQ3, HKV3, D3, args.layers
    G, scale = Hq // Hkv, 1.0 / np.sqrt(D)
    mgr, q, kn, vn, _ = decode_layers(np, torch, paged, synth, call, L, f16=True)
    out = [torch.empty((1, Hq, 1, D), dtype=torch.float16, device="cuda") for _ in range(L)]
    cached = [N3] * L

    def op_step(i):
        l = i % L
        paged.paged_attention(mgr, l, q[l], kn[l], vn[l], out[l], G, scale)
        cached[l] += 1
        return decode_step_bytes(cached[l])

    host_loop_s, step_s, _, total_bytes = time_op_steps(torch, op_step, args)
    mgr.close()
    gbs = total_bytes / (step_s * args.steps) / 1e9
    return {"us_per_step": round(step_s * 1e6, 3), "GB_s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "host_loop_us_per_step": round(host_loop_s * 1e6, 2), "dtype": "f16",
            "workload": "config 3 op step (append 1 token, attend over 8193+ keys) on fp16 layers, "
                        f"{L} rotating layers, timed as the headline"}


def append_cfg2(np, torch, paged, synth, call):
    S, Hkv, D, pool = 4096, 8, 128, 1024
    seed = synth.config_seed(2)
    copies = 16  # 256 MB of k/v inputs: the 256 MB MALL cannot serve them between uses
    m2 = paged.PagedAttentionManager(copies * (2 * pool * PAGE * Hkv * D * 2 + 8 * pool + 4096) + (1 << 20))
    ks, vs = [], []
    for c in range(copies):
        m2.init_layer(c, Hkv, D)
        m2.reserve_layer(c, pool)
        m2.fragment(c, synth.shuffled(seed + 2 * c, pool), synth.shuffled(seed + 2 * c + 1, pool))
        k = torch.empty((S, Hkv, D), dtype=torch.bfloat16, device="cuda")
        v = torch.empty_like(k)
        paged.fill_normal_bf16(k, seed + 10 + c)
        paged.fill_normal_bf16(v, seed + 20 + c)
        ks.append(k)
        vs.append(v)
    gamma = torch.from_numpy(synth.uniform_f32(seed, (D,), 0.5, 1.5)).cuda()
    cos, sin = paged.rope_cache(1e6, D, S)
    cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    n_app = copies * (pool // (S // PAGE))  # each copy takes 4 chunks of 256 pages

    def app(i):
        c = i % copies
        paged.qk_norm_rope_append(m2, c, ks[c], vs[c], gamma, 1e-6, cos_d, sin_d, 0)

    for i in range(copies):  # warm-up: first launches load the code object
        app(i)
    torch.cuda.synchronize()
    m2.reset()  # every copy starts from an empty layer again (same allocation sequence)
    # the first chunk of every copy is the timing warm-up, the other three are timed
    avg_us = time_kernels(torch, app, n_app - copies, warm=copies)
    app_bytes = 2 * S * Hkv * D * 2 * 2 + S * (D // 2) * 4 * 2 + D * 4 + (S // PAGE) * 8
    # read floor: the same K/V rows moved into 256 shuffled pages of each copy's
    # pool with the kernel's lane map, no norm or RoPE
    ids = [(torch.from_numpy(synth.shuffled(seed + 2 * c, pool)[:S // PAGE].astype("int32")).cuda(),
            torch.from_numpy(synth.shuffled(seed + 2 * c + 1, pool)[:S // PAGE].astype("int32")).cuda())
           for c in range(copies)]
    infos = [m2.get_layer(c) for c in range(copies)]
    cs = torch.cuda.current_stream().cuda_stream
    cp_us = time_kernels(torch, lambda i: _probe_call(
        "genllm_probe_append_copy", ks[i % copies].data_ptr(), vs[i % copies].data_ptr(), infos[i % copies].k_pool,
        infos[i % copies].v_pool, ids[i % copies][0].data_ptr(), ids[i % copies][1].data_ptr(), S, Hkv, D, cs),
        n_app - copies, warm=copies)
    copy_bytes = 2 * S * Hkv * D * 2 * 2
    m2.close()
    gbs = app_bytes / (avg_us * 1e-6) / 1e9
    return {"avg_launch_us": round(avg_us, 3), "bytes": app_bytes, "GB_s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "launches": n_app - copies,
            "note": "GPU time of the C call (qk_norm_rope_append: host page allocation, then kv_append_kernel with "
                    "the 256 new page ids in its launch arguments), back to back, GPU kept fed",
            "read_floor": floor_entry(cp_us, copy_bytes, avg_us, "the kernel's K/V row movement into shuffled pages "
                                      "(its lane map and stores), no norm, RoPE or tables")}


def prefill_cfg4(np, torch, paged, synth, call, iters=40):
    Hq, Hkv, D, S = 16, 8, 128, 2048
    seed = synth.config_seed(4)
    copies = 4
    m4 = paged.PagedAttentionManager(copies * (2 * 128 * PAGE * Hkv * D * 2 + 8 * 128 + 4096) + (1 << 20))
    qs = []
    for c in range(copies):
        m4.init_layer(c, Hkv, D)
        m4.reserve_layer(c, 128)
        m4.fragment(c, synth.shuffled(seed + 2 * c, 128), synth.shuffled(seed + 2 * c + 1, 128))
        m4.append_kv_pages(c, S)
        inf = m4.get_layer(c)
        call("genllm_fill_normal_bf16", inf.k_pool, 128 * PAGE * Hkv * D, seed + 30 + c, 0, None)
        call("genllm_fill_normal_bf16", inf.v_pool, 128 * PAGE * Hkv * D, seed + 40 + c, 0, None)
        qq = torch.empty((S, Hq, D), dtype=torch.bfloat16, device="cuda")
        paged.fill_normal_bf16(qq, seed + 50 + c)
        qs.append(qq)
    o4 = torch.empty((S, Hq, D), dtype=torch.bfloat16, device="cuda")
    infos = [m4.get_layer(c) for c in range(copies)]

    def pre(i):
        inf = infos[i % copies]
        paged.paged_prefill(qs[i % copies], o4, inf.k_pool, inf.v_pool, inf.k_ids, inf.v_ids, 128, S, Hkv,
                            1.0 / np.sqrt(D), q_layout="token")

    avg_us = time_kernels(torch, pre, iters)
    m4.close()
    flops = 4 * D * Hq * S * (S + 1) // 2
    tfl = flops / (avg_us * 1e-6) / 1e12
    return {"avg_launch_us": round(avg_us, 3), "flops": flops, "TFLOPS": round(tfl, 1),
            "frac_bf16_peak": round(tfl / BF16_PEAK_TFLOPS, 4)}


def flash_cfg4(np, torch, paged, synth, call, iters=40):
    """FlashAttentionImpl (attention.cpp:39-121, the kv_cache_per_layer = 0
    branch) at config 4's shape: q, out [1,16,2048,128] and k, v [1,8,2048,128]
    contiguous head-major, causal -- the prefill kernel with identity pages."""
    Hq, Hkv, D, S = 16, 8, 128, 2048
    seed = synth.config_seed(4)
    copies = 4
    qs, ks, vs = [], [], []
    for c in range(copies):
        q = torch.empty((1, Hq, S, D), dtype=torch.bfloat16, device="cuda")
        k = torch.empty((1, Hkv, S, D), dtype=torch.bfloat16, device="cuda")
        v = torch.empty_like(k)
        paged.fill_normal_bf16(q, seed + 60 + c)
        paged.fill_normal_bf16(k, seed + 70 + c)
        paged.fill_normal_bf16(v, seed + 80 + c)
        qs.append(q), ks.append(k), vs.append(v)
    o = torch.empty((1, Hq, S, D), dtype=torch.bfloat16, device="cuda")

    def run(i):
        c = i % copies
        paged.flash_attention(qs[c], ks[c], vs[c], o, Hq // Hkv, 1.0 / np.sqrt(D))

    avg_us = time_kernels(torch, run, iters)
    flops = 4 * D * Hq * S * (S + 1) // 2
    tfl = flops / (avg_us * 1e-6) / 1e12
    return {"avg_launch_us": round(avg_us, 3), "flops": flops, "TFLOPS": round(tfl, 1),
            "frac_bf16_peak": round(tfl / BF16_PEAK_TFLOPS, 4)}


def prefill_scale(np, torch, paged, synth, call, iters=10):
    """The prefill kernel (FlashAttention form, causal) past config 4's size:
    the same kernel at 2K-16K tokens for Qwen3 head counts and at head_dim 256.
    Not part of the default run (bench.py --only prefill_scale)."""
    out = []
    for i, (Hq, Hkv, S, D) in enumerate([(16, 8, 2048, 128), (32, 8, 2048, 128), (16, 8, 4096, 128),
                                         (32, 8, 8192, 128), (16, 8, 16384, 128), (8, 2, 2048, 256),
                                         (8, 2, 8192, 256)]):
        q = torch.empty((1, Hq, S, D), dtype=torch.bfloat16, device="cuda")
        k = torch.empty((1, Hkv, S, D), dtype=torch.bfloat16, device="cuda")
        v = torch.empty_like(k)
        paged.fill_normal_bf16(q, 7000 + 3 * i)
        paged.fill_normal_bf16(k, 7001 + 3 * i)
        paged.fill_normal_bf16(v, 7002 + 3 * i)
        o = torch.empty_like(q)
        avg_us = time_kernels(torch, lambda _: paged.flash_attention(q, k, v, o, Hq // Hkv, 1.0 / np.sqrt(D)), iters)
        flops = 4 * D * Hq * S * (S + 1) // 2
        tfl = flops / (avg_us * 1e-6) / 1e12
        out.append({"q_heads": Hq, "kv_heads": Hkv, "S": S, "head_dim": D, "avg_launch_us": round(avg_us, 2),
                    "TFLOPS": round(tfl, 1), "frac_bf16_peak": round(tfl / BF16_PEAK_TFLOPS, 4)})
        del q, k, v, o
    return {"shapes": out}


def decode_scale(np, torch, paged, synth, call, iters=40):
    """The decode kernel pair (stateless genllm_paged_decode, Qwen3-4B heads)
    from 8K to 256K cached keys, each layer in its own shuffled pool; enough
    layers rotate that the MALL cannot hold them.  Not part of the default
    run (bench.py --only decode_scale)."""
    Hq, Hkv, D = HQ3, HKV3, D3
    out = []
    for n_keys in (8193, 32761, 131073, 262145):
        n_pages = (n_keys + PAGE - 1) // PAGE
        pool = n_pages + 8
        layer_bytes = 2 * pool * PAGE * Hkv * D * 2
        L = max(1, -(-(1 << 30) // layer_bytes))
        mgr = paged.PagedAttentionManager(L * layer_bytes + (1 << 20))
        for l in range(L):
            mgr.init_layer(l, Hkv, D)
            mgr.reserve_layer(l, pool)
            mgr.fragment(l, synth.shuffled(5000 + 2 * l, pool), synth.shuffled(5001 + 2 * l, pool))
            mgr.append_kv_pages(l, n_keys)
            info = mgr.get_layer(l)
            call("genllm_fill_normal_bf16", info.k_pool, pool * PAGE * Hkv * D, 5100 + l, 0, None)
            call("genllm_fill_normal_bf16", info.v_pool, pool * PAGE * Hkv * D, 5200 + l, 0, None)
        infos = [mgr.get_layer(l) for l in range(L)]
        q = torch.empty((Hq, 1, D), dtype=torch.bfloat16, device="cuda")
        paged.fill_normal_bf16(q, 5300)
        o = torch.empty_like(q)
        ws = torch.zeros(paged.decode_workspace_bytes(Hq, Hkv, 1, D, pool), dtype=torch.uint8, device="cuda")

        def launch(i):
            inf = infos[i % L]
            paged.paged_decode(q, o, inf.k_pool, inf.v_pool, inf.k_ids, inf.v_ids, n_pages, n_keys, Hkv,
                               1.0 / np.sqrt(D), ws)

        avg_us = time_kernels(torch, launch, iters)
        nbytes = decode_kernel_bytes(n_keys)
        gbs = nbytes / (avg_us * 1e-6) / 1e9
        out.append({"n_keys": n_keys, "layers_rotated": L, "avg_launch_us": round(avg_us, 2), "bytes": nbytes,
                    "GB_s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)})
        mgr.close()
        del ws
    return {"shapes": out}


def qwen35_d256(np, torch, paged, synth, call, iters=100):
    """The paged op's kernels at Qwen3.5's attention shape (Qwen35.hpp:14-16:
    head_dim 256, 8 q / 2 kv heads): decode of one query at 8193 cached keys
    (the split-K decode kernel at D = 256; 16 layers of pools rotate so the
    MALL cannot serve them) and a causal 2048-token prefill (the D = 256
    prefill kernel)."""
    Hq, Hkv, D = 8, 2, 256
    seed = synth.config_seed(3) + 256
    pool, n_keys, L = 1024, 8193, 16
    n_pages = (n_keys + 15) // 16
    m = paged.PagedAttentionManager(L * (2 * pool * PAGE * Hkv * D * 2 + 8 * pool + 4096) + (1 << 20))
    for l in range(L):
        m.init_layer(l, Hkv, D)
        m.reserve_layer(l, pool)
        m.fragment(l, synth.shuffled(seed + 2 * l, pool), synth.shuffled(seed + 2 * l + 1, pool))
        m.append_kv_pages(l, n_keys)
        inf = m.get_layer(l)
        call("genllm_fill_normal_bf16", inf.k_pool, pool * PAGE * Hkv * D, seed + 100 + l, 0, None)
        call("genllm_fill_normal_bf16", inf.v_pool, pool * PAGE * Hkv * D, seed + 200 + l, 0, None)
    q = torch.empty((L, Hq, 1, D), dtype=torch.bfloat16, device="cuda")
    paged.fill_normal_bf16(q, seed + 300)
    o = torch.empty((Hq, 1, D), dtype=torch.bfloat16, device="cuda")
    ws = torch.zeros(paged.decode_workspace_bytes(Hq, Hkv, 1, D, pool), dtype=torch.uint8, device="cuda")
    infos = [m.get_layer(l) for l in range(L)]

    def dec(i):
        inf = infos[i % L]
        paged.paged_decode(q[i % L], o, inf.k_pool, inf.v_pool, inf.k_ids, inf.v_ids, n_pages, n_keys, Hkv,
                           1.0 / np.sqrt(D), ws)

    d_us = time_kernels(torch, dec, iters)
    m.close()
    d_bytes = decode_kernel_bytes(n_keys, Hq, Hkv, D)
    d_gbs = d_bytes / (d_us * 1e-6) / 1e9

    S, copies = 2048, 4
    mp = paged.PagedAttentionManager(copies * (2 * 128 * PAGE * Hkv * D * 2 + 8 * 128 + 4096) + (1 << 20))
    qs = []
    for c in range(copies):
        mp.init_layer(c, Hkv, D)
        mp.reserve_layer(c, 128)
        mp.fragment(c, synth.shuffled(seed + 50 + 2 * c, 128), synth.shuffled(seed + 51 + 2 * c, 128))
        mp.append_kv_pages(c, S)
        inf = mp.get_layer(c)
        call("genllm_fill_normal_bf16", inf.k_pool, 128 * PAGE * Hkv * D, seed + 130 + c, 0, None)
        call("genllm_fill_normal_bf16", inf.v_pool, 128 * PAGE * Hkv * D, seed + 140 + c, 0, None)
        qq = torch.empty((S, Hq, D), dtype=torch.bfloat16, device="cuda")
        paged.fill_normal_bf16(qq, seed + 150 + c)
        qs.append(qq)
    op = torch.empty((S, Hq, D), dtype=torch.bfloat16, device="cuda")
    pinfos = [mp.get_layer(c) for c in range(copies)]

    def pre(i):
        inf = pinfos[i % copies]
        paged.paged_prefill(qs[i % copies], op, inf.k_pool, inf.v_pool, inf.k_ids, inf.v_ids, 128, S, Hkv,
                            1.0 / np.sqrt(D), q_layout="token")

    p_us = time_kernels(torch, pre, 40)
    mp.close()
    flops = 4 * D * Hq * S * (S + 1) // 2
    tfl = flops / (p_us * 1e-6) / 1e12
    return {"decode": {"n_keys": n_keys, "avg_launch_us": round(d_us, 3),
                       "bytes": d_bytes,
                       "GB_s": round(d_gbs, 1), "frac_hbm": round(d_gbs / HBM_PEAK_GBS, 4)},
            "prefill": {"S": S, "avg_launch_us": round(p_us, 3), "flops": flops, "TFLOPS": round(tfl, 1),
                        "frac_bf16_peak": round(tfl / BF16_PEAK_TFLOPS, 4)}}


def longctx_cfg5(np, torch, paged, synth, call, iters=10):
    Hq, Hkv, D, N, pool, layers = 32, 8, 128, 32761, 4096, 36
    seed = synth.config_seed(5)
    m5 = paged.PagedAttentionManager(layers * (2 * pool * PAGE * Hkv * D * 2 + 8 * pool + 4096) + (1 << 20))
    for l in range(layers):
        m5.init_layer(l, Hkv, D)
        m5.reserve_layer(l, pool)
        m5.fragment(l, synth.shuffled(seed + 2 * l, pool), synth.shuffled(seed + 2 * l + 1, pool))
        m5.append_kv_pages(l, N)
        inf = m5.get_layer(l)
        call("genllm_fill_normal_bf16", inf.k_pool, pool * PAGE * Hkv * D, seed + 100 + l, 0, None)
        call("genllm_fill_normal_bf16", inf.v_pool, pool * PAGE * Hkv * D, seed + 200 + l, 0, None)
    q5 = torch.empty((layers, Hq, 1, D), dtype=torch.bfloat16, device="cuda")
    paged.fill_normal_bf16(q5, seed)
    o5 = torch.empty((Hq, 1, D), dtype=torch.bfloat16, device="cuda")
    ws = torch.zeros(paged.decode_workspace_bytes(Hq, Hkv, 1, D, pool), dtype=torch.uint8, device="cuda")
    infos = [m5.get_layer(l) for l in range(layers)]
    n_pages = (N + 15) // 16

    def all_layers(_):
        for l in range(layers):
            inf = infos[l]
            paged.paged_decode(q5[l], o5, inf.k_pool, inf.v_pool, inf.k_ids, inf.v_ids, n_pages, N, Hkv,
                               1.0 / np.sqrt(D), ws)

    avg_us = time_kernels(torch, all_layers, iters, warm=2)
    # read floors: the split kernel's page loads of all 36 layers without the
    # math, and a contiguous stream of one layer's bytes
    pps, hpw = decode_pps(torch, n_pages, Hkv, D)
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    cs = torch.cuda.current_stream().cuda_stream

    def all_probes(_):
        for l in range(layers):
            inf = infos[l]
            _probe_call("genllm_probe_decode_read", inf.k_pool, inf.v_pool, inf.k_ids, inf.v_ids, n_pages, Hkv, D, pps,
                        hpw, sink.data_ptr(), cs)

    pat_us = time_kernels(torch, all_probes, iters, warm=2) / layers
    layer_bytes = decode_kernel_bytes(N)
    str_us = stream_floor(torch, layer_bytes, 8, iters=20)
    floors = {"decode_config5_pattern": floor_entry(pat_us, layer_bytes, avg_us / layers,
                                                    f"the split kernel's page loads per layer, {pps} pages per split, "
                                                    f"{hpw} kv head(s) per workgroup, no math, no merge"),
              "decode_config5_stream": floor_entry(str_us, layer_bytes, avg_us / layers,
                                                   "contiguous stream of one layer's bytes")}
    # the same 36-layer sequence captured once into a HIP graph and replayed
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        all_layers(0)
    g_us = time_kernels(torch, lambda i: graph.replay(), iters, warm=2)
    del graph
    # The decode loop itself: one step (append this token's K/V, attend) of all
    # 36 layers captured once at the device position and replayed token after
    # token (genllm_kv_stage_decode / genllm_paged_attention_step / sync).
    kn = torch.empty((layers, 1, Hkv, 1, D), dtype=torch.bfloat16, device="cuda")
    vn = torch.empty_like(kn)
    paged.fill_normal_bf16(kn, seed + 1)
    paged.fill_normal_bf16(vn, seed + 2)
    n_steps = iters + 2
    for l in range(layers):
        m5.stage_decode(l, n_steps)
    torch.cuda.synchronize()
    o5s = o5.unsqueeze(0)
    step_graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(step_graph):
        for l in range(layers):
            paged.paged_attention_step(m5, l, q5[l].unsqueeze(0), kn[l], vn[l], o5s, Hq // Hkv, 1.0 / np.sqrt(D))
    s_us = time_kernels(torch, lambda i: step_graph.replay(), iters, warm=2)
    for l in range(layers):
        if m5.sync_decode(l) != N + n_steps:
            raise RuntimeError("captured decode loop: device position did not advance once per replay")
    del step_graph
    m5.close()
    b5 = layers * decode_kernel_bytes(N)
    gbs = b5 / (avg_us * 1e-6) / 1e9
    s_bytes = sum(layers * decode_step_bytes(N + 1 + i) for i in range(2, n_steps)) / iters
    return {"total_us": round(avg_us, 2), "us_per_layer": round(avg_us / layers, 3), "bytes": b5,
            "GB_s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "graph_total_us": round(g_us, 2), "graph_us_per_layer": round(g_us / layers, 3),
            "graph_GB_s": round(b5 / (g_us * 1e-6) / 1e9, 1),
            "read_floor": floors,
            "decode_loop_graph": {"us_per_token": round(s_us, 2), "us_per_layer": round(s_us / layers, 3),
                                  "GB_s": round(s_bytes / (s_us * 1e-6) / 1e9, 1), "tokens": iters,
                                  "note": "36-layer append + attend step captured once at the device position "
                                          "and replayed per token (position advanced on the GPU)"}}


def linear_qkv(np, torch, paged, synth, call, iters=40):
    """Qwen3-4B fused Q/K/V projection (hidden 2560 -> (32 + 2*8) * 128 = 6144,
    Qwen3.cpp:130-134) through genllm_linear: one decode token (the
    order-exact GEMV, HBM-bound on the 31.5 MB of weights; 16 weight copies
    rotate so the MALL cannot serve them) and a 2048-token prefill chunk
    (rocBLAS GEMM + epilogue)."""
    K, N, copies = 2560, 6144, 16
    ws_ = [torch.empty((N, K), dtype=torch.bfloat16, device="cuda") for _ in range(copies)]
    for c, w in enumerate(ws_):
        paged.fill_normal_bf16(w, 900 + c)
    x1 = torch.empty((1, K), dtype=torch.bfloat16, device="cuda")
    paged.fill_normal_bf16(x1, 7)
    o1 = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")
    gemv_us = time_kernels(torch, lambda i: paged.linear(x1, ws_[i % copies], o1), iters)
    gemv_bytes = N * K * 2 + K * 2 + N * 2
    M = 2048
    xm = torch.empty((M, K), dtype=torch.bfloat16, device="cuda")
    paged.fill_normal_bf16(xm, 8)
    om = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    wsp = torch.empty(paged.linear_workspace_bytes(M, K, N), dtype=torch.uint8, device="cuda")
    gemm_us = time_kernels(torch, lambda i: paged.linear(xm, ws_[i % copies], om, workspace=wsp), iters // 4)
    gemm_flops = 2 * M * K * N
    return {"gemv_rows": 1, "gemv_avg_launch_us": round(gemv_us, 3), "gemv_bytes": gemv_bytes,
            "gemv_GB_s": round(gemv_bytes / (gemv_us * 1e-6) / 1e9, 1),
            "gemv_frac_hbm": round(gemv_bytes / (gemv_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "gemm_rows": M, "gemm_avg_launch_us": round(gemm_us, 2),
            "gemm_TFLOPS": round(gemm_flops / (gemm_us * 1e-6) / 1e12, 1)}


def copy_calibration(np, torch, paged, synth, call, mib=256, iters=20):
    """A plain device copy of known size (torch copy_), the reference point that
    scales the FETCH_SIZE / WRITE_SIZE counters of the rocprofv3 --pmc passes."""
    src = torch.empty(mib << 19, dtype=torch.bfloat16, device="cuda")
    paged.fill_normal_bf16(src, 1)
    dst = torch.empty_like(src)
    avg_us = time_kernels(torch, lambda i: dst.copy_(src), iters, warm=3)
    nbytes = src.numel() * 2
    return {"bytes_read": nbytes, "bytes_written": nbytes, "avg_launch_us": round(avg_us, 3),
            "GB_s_read_plus_write": round(2 * nbytes / (avg_us * 1e-6) / 1e9, 1)}


def traffic_workload(args, np, torch, paged, synth, call, n=200):
    """The workload of the counter passes: n launches of the headline's decode
    kernel over its rotating layers, then COPY_MIB MiB device copies whose known
    bytes scale the counters (copy_calibration)."""
    mgr, q, kn, vn, seed = decode_layers(np, torch, paged, synth, call, args.layers)
    launch, n_keys = decode_launcher(np, torch, paged, mgr, q, args.layers)
    us = time_kernels(torch, launch, n, warm=8)
    mgr.close()
    cal = copy_calibration(np, torch, paged, synth, call, mib=COPY_MIB, iters=5)
    return {"decode_launches": n, "n_keys": n_keys, "events_us_per_launch": round(us, 3),
            "copy_bytes": cal["bytes_read"]}


def _csv_rows(out_dir, suffix):
    rows = []
    for path in glob.glob(os.path.join(out_dir, "**", "*" + suffix), recursive=True):
        with open(path, newline="") as f:
            rows += list(csv.DictReader(f))
    return rows


def _child_pass(tmp, tag, prof_args, env):
    """One child `rocprofv3 <prof_args> -- bench.py --only traffic` run; returns
    its output directory."""
    exe = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    out_dir = os.path.join(tmp, tag)
    cmd = ["timeout", "-s", "KILL", "150", exe, *prof_args, "-d", out_dir, "-o", "traffic", "--output-format", "csv",
           "--", sys.executable, os.path.abspath(__file__), "--only", "traffic"]
    print(f"bench.py: child rocprofv3 pass {tag}", file=sys.stderr, flush=True)
    with open(os.path.join(tmp, tag + ".log"), "w") as log:
        rc = subprocess.run(cmd, cwd="/tmp", env=env, stdout=log, stderr=subprocess.STDOUT).returncode
    return out_dir, rc


def measure_counters():
    """Measured now, for the headline decode kernels (bench.py --only traffic:
    200 back-to-back launches over the rotating layers, then a COPY_MIB MiB
    copy), in three child rocprofv3 runs started before this process
    initialises the GPU:
      * --pmc FETCH_SIZE and --pmc WRITE_SIZE: KiB per dispatch, each scaled by
        what the same counter reads for the copy of known size -> HBM bytes;
      * --kernel-trace: mean duration of each decode kernel and the trace's
        timeline per decode (first start to last end of the timed launches / n).
    Returns (dict or None, note)."""
    if any(k.startswith("ROCPROF") for k in os.environ):
        return None, "skipped: the bench itself runs under rocprofv3"
    if not (shutil.which("rocprofv3") or os.path.exists("/opt/rocm/bin/rocprofv3")):
        return None, "skipped: rocprofv3 not found"
    tmp = tempfile.mkdtemp(prefix="genllm_prof_", dir="/tmp")
    env = dict(os.environ, TMPDIR="/tmp")
    res = {}
    try:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            out_dir, rc = _child_pass(tmp, counter, ["--pmc", counter], env)
            rows = [r for r in _csv_rows(out_dir, "counter_collection.csv") if r.get("Counter_Name") == counter]
            split = {}
            for r in rows:
                if "paged_decode" in r["Kernel_Name"]:
                    split.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
            # the calibration copy: the largest copy dispatches (small uploads use the same kernel)
            copies = [r for r in rows if "copyBuffer" in r["Kernel_Name"]]
            big = max((int(r["Grid_Size"]) for r in copies), default=0)
            cpy = [float(r["Counter_Value"]) for r in copies if int(r["Grid_Size"]) == big]
            if not split or not cpy:
                return None, f"{counter} pass gave no rows (rc {rc})"
            scale = COPY_MIB * 1024.0 / statistics.mean(cpy)
            kib = sum(statistics.mean(v) for v in split.values())
            res[counter] = {"kib_per_decode": round(kib, 1), "copy_kib_counted": round(statistics.mean(cpy), 1),
                            "scale": round(scale, 5), "bytes": int(kib * 1024.0 * scale)}
        out_dir, rc = _child_pass(tmp, "kernel_trace", ["--kernel-trace"], env)
        rows = [r for r in _csv_rows(out_dir, "kernel_trace.csv") if "paged_decode" in r["Kernel_Name"]]
        kernels = {}
        for r in rows:
            kernels.setdefault(r["Kernel_Name"], []).append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
        if not kernels:
            return None, f"kernel-trace pass gave no rows (rc {rc})"
        n = min(len(v) for v in kernels.values()) - 8  # the first 8 of each are the warm-up
        timed = {k: sorted(v)[-n:] for k, v in kernels.items()}
        per_kernel = {re.search(r"paged_decode\w*<[^>]*>", k).group(0):
                      round(statistics.mean(e - b for b, e in v) / 1e3, 3) for k, v in timed.items()}

        def spread(durs):  # nearest-rank p10, median, p90 of the traced durations, us
            s = sorted(durs)
            return {q: round(s[min(len(s) - 1, int(round(f * (len(s) - 1))))] / 1e3, 3)
                    for q, f in (("p10", 0.1), ("median", 0.5), ("p90", 0.9))}

        per_kernel_spread = {re.search(r"paged_decode\w*<[^>]*>", k).group(0): spread([e - b for b, e in v])
                             for k, v in timed.items()}
        t0 = min(v[0][0] for v in timed.values())
        t1 = max(v[-1][1] for v in timed.values())
        # the traced process also timed the same launches with HIP events
        ev = None
        with open(os.path.join(tmp, "kernel_trace.log")) as log:
            for line in log:
                if line.startswith("{") and "events_us_per_launch" in line:
                    ev = json.loads(line)["events_us_per_launch"]
        res["kernel_trace"] = {"mean_us": per_kernel, "p10_median_p90_us": per_kernel_spread,
                               "sum_us": round(sum(per_kernel.values()), 3),
                               "timeline_us_per_decode": round((t1 - t0) / 1e3 / n, 3), "decodes": n,
                               "events_us_per_decode_traced": ev,
                               "note": "durations under rocprofv3 --kernel-trace; events_us_per_decode_traced is "
                                       "the same launches timed with HIP events inside the traced process, so "
                                       "(events_us_per_decode_traced - avg_launch_us) is what the profiler adds "
                                       "per decode (two dispatches)"}
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    res["bytes"] = res["FETCH_SIZE"]["bytes"] + res["WRITE_SIZE"]["bytes"]
    return res, "measured in this run"


def cpp_host_cost(calls=200):
    """Host cost of one PAGED_ATTN dispatch measured from C++: the operator
    test binary's --host-cost mode (calls back to back through
    kernel::dispatch at config 3's shape, no synchronisation), run as a child
    process.  Returns (dict or None, note)."""
    exe = os.path.join(ROOT, "tests", "cpp", "test_ops_hip")
    if not os.access(exe, os.X_OK):
        return None, "skipped: tests/cpp/test_ops_hip not built"
    try:
        r = subprocess.run([exe, "--host-cost", str(calls)], capture_output=True, text=True, timeout=120)
    except subprocess.TimeoutExpired:
        return None, "timed out"
    for line in r.stdout.splitlines():
        if line.startswith("{") and "host_us_per_call" in line:
            return json.loads(line), "measured in this run"
    return None, f"no result (rc {r.returncode})"


def cpu_baseline(mgr, np, paged, synth, args, seed):
    """The oracle (oracle/, single thread) on the headline step, on inputs
    copied back from layer 0 of the GPU run: same pools, same allocator state,
    same q / k / v."""
    import oracle

    Hq, Hkv, D, pool, n0 = 32, 8, 128, 2048, 8192
    ref = oracle.Manager(with_pool=True)
    ref.init_layer(0, Hkv, D)
    ref.reserve_layer(0, pool)
    for which, perm in ((0, synth.shuffled(seed, pool)), (1, synth.shuffled(seed + 1, pool))):
        p = ref.pool(0, which)
        for _ in range(pool):
            p.alloc()
        for b in perm[::-1]:
            p.free(int(b))
    ref.append_kv_pages(0, n0)
    ref.pool_array(0, 0)[:] = mgr.read_pool(0, 0)
    ref.pool_array(0, 1)[:] = mgr.read_pool(0, 1)
    q = synth.normal_bf16(seed + 300, (1, Hq, 1, D))
    k = synth.normal_bf16(seed + 400, (1, Hkv, 1, D))
    v = synth.normal_bf16(seed + 500, (1, Hkv, 1, D))
    times, nbytes = [], 0
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < args.cpu_seconds or len(times) < 3:
        t0 = time.perf_counter()
        ref.paged_attention(0, q, k, v, Hq // Hkv, 1.0 / np.sqrt(D))
        times.append(time.perf_counter() - t0)
        nbytes += decode_step_bytes(ref.num_cached(0))
    total = sum(times)
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(nbytes / total / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{len(times)} op steps (append 1 token + attend over {n0 + 1}..{ref.num_cached(0)} keys, "
                      f"Qwen3-4B shape) of the oracle restatement, gcc -O3 -mavx2 -mfma -mf16c, 1 thread",
            "us_per_step_median": round(1e6 * statistics.median(times), 1),
            "host_cores": os.cpu_count(), "cpu_model": cpu_model}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on exactly one GPU (asked for {args.gpus}); "
              "sharding the path over several GPUs is designed, not built or run here.", file=sys.stderr)
        sys.exit(2)

    # HBM traffic and kernel-trace durations of the headline kernels: child
    # rocprofv3 passes, before this process touches the GPU
    traffic, traffic_note = (None, "skipped (--no-traffic)")
    if not args.only and not args.no_traffic:
        traffic, traffic_note = measure_counters()

    cpp_host, cpp_host_note = (None, "skipped (--only)")
    if not args.only:
        cpp_host, cpp_host_note = cpp_host_cost()

    import numpy as np
    import torch

    from genllm_amd import paged, synth
    from genllm_amd._lib import call

    torch.cuda.set_device(0)
    common = (np, torch, paged, synth, call)
    if args.only == "traffic":
        print(json.dumps({"only": args.only, **traffic_workload(args, *common)}), flush=True)
        return
    if args.only == "f16":
        print(json.dumps({"only": args.only, **f16_config3(args, *common)}), flush=True)
        return
    if args.only and args.only != "headline":
        fn = {"append": append_cfg2, "prefill": prefill_cfg4, "flash": flash_cfg4, "qwen35": qwen35_d256,
              "longctx": longctx_cfg5, "linear": linear_qkv, "copy": copy_calibration,
              "prefill_scale": prefill_scale, "decode_scale": decode_scale}[args.only]
        print(json.dumps({"only": args.only, **fn(*common)}), flush=True)
        return

    head, mgr, seed = headline(args, *common)
    result = {
        "metric": METRIC,
        "value": head["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded counter-based normal bf16 K/V/q, Fisher-Yates block tables)",
        "config": head["config"],
        "us_per_layer": head["us_per_layer"],
        "device": torch.cuda.get_device_name(0),
        "roofline": head["roofline"],
        "step_timing": head["step_timing"],
        "host": head["host"],
    }
    if args.only:
        result["read_floor"] = head["read_floor"]
    result["host"]["cpp_us_per_call"] = cpp_host["host_us_per_call"] if cpp_host else None
    result["host"]["cpp_note"] = ("host time of one PAGED_ATTN dispatch through kernel::dispatch, from C++ "
                                  "(tests/cpp/test_ops_hip --host-cost): " + cpp_host_note)
    if traffic:
        result["roofline"]["traffic"] = traffic["bytes"]
        result["roofline"]["traffic_x_algorithmic"] = round(traffic["bytes"] / head["roofline"]["bytes_per_launch"],
                                                            4)
        result["roofline"]["traffic_counters"] = {k: traffic[k] for k in ("FETCH_SIZE", "WRITE_SIZE")}
        result["roofline"]["kernel_trace"] = traffic["kernel_trace"]
    result["roofline"]["profiler_note"] = traffic_note
    if not args.skip_secondary and not args.only:
        result["secondary"] = {"append_config2": append_cfg2(*common), "prefill_config4": prefill_cfg4(*common),
                               "flash_config4": flash_cfg4(*common), "qwen35_head_dim_256": qwen35_d256(*common),
                               "longctx_config5": longctx_cfg5(*common), "linear_qkv_4b": linear_qkv(*common),
                               "f16_config3": f16_config3(args, *common)}
        # read floors (probes that move each kernel's bytes with its access
        # pattern and no arithmetic), next to the kernels they bound
        sec = result["secondary"]
        result["secondary"]["read_floor"] = {
            **head["read_floor"], **sec["longctx_config5"].pop("read_floor"),
            "append_config2_copy": sec["append_config2"].pop("read_floor")}
    if not args.skip_cpu and not args.only:
        result["cpu_baseline"] = cpu_baseline(mgr, np, paged, synth, args, seed)
    mgr.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
