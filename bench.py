"""Benchmark: Q8_0 GEMV HBM throughput on one MI355X (one LFM-style layer's GEMVs + LM head).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one pass of the decode hot path over one synthetic layer at T=1: the
GEMVs fused q|k|v 3072x2048, o_proj 2048x2048, gate+up 16384x2048, down
2048x8192 and the LM head 65536x2048 (fp32 logits), from packed Q8_0 weights
resident in HBM, each quantizing its fp32 x (K=2048 or 8192) to Q8_0 in its own
prologue (q8_gemv_fused_kernel, PQ_PRO_F32). The weights rotate over enough
copies (>= 600 MB) that no step reads another step's weights out of the 256 MB
Infinity Cache.

Prints ONE JSON line. value = algorithmic bytes per step / time per step (GB/s);
roofline = the GEMV kernel's algorithmic bytes / its launch period, timed with
HIP events on the launch stream over back-to-back launches of each shape (the
period includes the dispatch gap between launches), against 8 TB/s;
cpu_baseline = the reference's own CPU GEMV (.auto/lfm3/q8_gemv_cpu.c gemv_q8,
compiled into oracle/_ref) on the host cores over a bounded sample of the same
shapes.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "pulsar-asm_amd"))

HBM_PEAK_GBS = 8000.0
SHAPES = [  # name, N, K, output dtype
    ("qkv", 3072, 2048, "bf16"),
    ("o_proj", 2048, 2048, "bf16"),
    ("gate_up", 16384, 2048, "bf16"),
    ("down", 2048, 8192, "bf16"),
    ("lm_head", 65536, 2048, "f32"),
]


def measured_traffic():
    """HBM bytes per step of the 5 GEMV launches, from the two rocprofv3 --pmc
    passes summarised in profiles/q8_gemv_hbm_traffic.md (None if absent)."""
    import re
    path = os.path.join(ROOT, "profiles", "q8_gemv_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"\| step \(5 GEMVs\) \| [0-9.]+ \| ([0-9.]+) \|", open(path).read())
    return int(float(m.group(1)) * 1e6) if m else None


def graph_of(torch, fn):
    """fn's launches (on torch's current stream) captured into one HIP graph,
    after one eager run on a side stream: the timed regions replay graphs so the
    GPU, not the Python launch loop, sets the pace."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def timed_replay(torch, g, stream, reps=1):
    """Milliseconds per replay of g, HIP events on the launch stream: two
    untimed replays (clocks settle), then the median of reps timed replays."""
    from pulsar_amd.hiptime import Event
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    ev = [Event() for _ in range(reps + 1)]
    ev[0].record(stream)
    for i in range(reps):
        g.replay()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    t = sorted(ev[i].elapsed_ms(ev[i + 1]) for i in range(reps))
    return t[len(t) // 2]


def gemv_bytes(N, K, out):
    """Algorithmic HBM bytes of one GEMV: codes, fp16 scales, the fp32 x, y."""
    return N * K + N * (K // 32) * 2 + 4 * K + N * (4 if out == "f32" else 2)


def gpu_desc(torch, pq):
    """Device name, CU count and the shader clock measured on the device (pq_clock_mhz)."""
    p = torch.cuda.get_device_properties(0)
    out = torch.zeros(2, dtype=torch.float32, device="cuda:0")
    pq.check(pq.lib().pq_clock_mhz(out.data_ptr(), pq.stream_ptr()), "pq_clock_mhz")
    torch.cuda.synchronize()
    return {"name": p.name, "gcn_arch": getattr(p, "gcnArchName", None), "cus": p.multi_processor_count,
            "clock_MHz": round(float(out[0].item()))}


def cpu_baseline(seconds=10.0):
    """The reference's gemv_q8 (fp32 x, fp32 scales) over the same shapes, on all host cores."""
    import ctypes as C
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle
    ref = pyoracle.ref()
    kind = "reference"
    if ref is None:
        kind = "port"
    data = []
    for i, (name, N, K, _) in enumerate(SHAPES):
        W = pyoracle.gen_codes(20261201 + 4 * i, N * K).reshape(N, K)
        S = pyoracle.gen_scales(20261201 + 4 * i + 1, N * (K // 32)).view(np.float16).astype(np.float32)
        x = pyoracle.gen_normal(20261201 + 4 * i + 2, K)
        y = np.empty(N, np.float32)
        data.append((N, K, W, S.reshape(N, K // 32), x, y))

    def run_step():
        for (N, K, W, S, x, y) in data:
            if ref is not None:
                ref.ref_q8_gemv(W.ctypes.data_as(C.c_void_p), S.ctypes.data_as(C.c_void_p),
                                x.ctypes.data_as(C.c_void_p), y.ctypes.data_as(C.c_void_p), C.c_int(N), C.c_int(K))
            else:
                y[:] = pyoracle.q8_gemv_a11(W, S, x)

    nbytes = sum(N * K + N * (K // 32) * 4 + K * 4 + N * 4 for (N, K, *_r) in data)

    def timed(sec):
        run_step()
        steps = 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < sec:
            run_step()
            steps += 1
        return steps, (time.perf_counter() - t0) / steps

    threads = int(ref.ref_max_threads()) if ref is not None else 1
    steps, dt = timed(seconds)
    one = None
    if ref is not None and threads > 1:   # the same routine on one core, a shorter sample
        ref.ref_set_threads(1)
        s1, dt1 = timed(seconds / 2)
        ref.ref_set_threads(threads)
        one = {"value": round(nbytes / dt1 / 1e9, 2), "ms_per_step": round(dt1 * 1e3, 3), "passes": s1}
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(nbytes / dt / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": kind,
            "ms_per_step": round(dt * 1e3, 3), "one_core": one,
            "host": f"{model}, nproc {os.cpu_count()}",
            "sample": f"{steps} passes of the 5 layer+LM-head GEMV shapes through gemv_q8 "
                      f"(q8_gemv_cpu.c:29-58, OpenMP over rows; fp32 x and fp32 scales, {nbytes / 1e6:.1f} MB/pass)"}


def decode_bench(pq, n_steps=64, n_prompt=256):
    """Backbone decode tok/s: the synthetic 24-layer LFM3-style model, a 256-token
    prompt (chunked prefill), then n_steps T=1 greedy steps timed on the engine's stream."""
    import numpy as np
    from pulsar_amd.engine import LFM3_SYNTH, Engine, synth_fill
    from pulsar_amd.hiptime import Event
    e = Engine(**LFM3_SYNTH)
    e.load_synthetic()
    prompt = synth_fill(5, LFM3_SYNTH["seed"] + 4 * 5000, n_prompt, float(LFM3_SYNTH["vocab"]))
    st = e.stream()
    a, c = Event(), Event()
    e.reset()
    e.feed(prompt)                       # warm-up prefill and steps
    e.decode(4, want_ids=False)
    e.sync()
    e.reset()
    a.record(st)
    e.feed(prompt)                       # the timed prefill (32-position chunks)
    b2 = Event()
    b2.record(st)
    e.decode(n_steps, want_ids=False)
    c.record(st)
    e.sync()
    prefill_ms = a.elapsed_ms(b2)
    ms = b2.elapsed_ms(c) / n_steps
    wbytes = e.weight_bytes()
    kv = 8 * 2 * 8 * 64 * 2  # attention layers x (k, v) x kv heads x dim x fp16, per position
    mean_pos = n_prompt + n_steps / 2
    tok_bytes = wbytes + kv * mean_pos
    e.close()
    return {"tok_s": round(1e3 / ms, 1), "ms_per_token": round(ms, 4), "steps": n_steps,
            "positions": f"{n_prompt}..{n_prompt + n_steps}", "bytes_per_token": int(tok_bytes),
            "GB/s": round(tok_bytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(tok_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "prefill_ms_256": round(prefill_ms, 2)}


def prefill_gemm_bench(pq, torch, dev, g, T=512, chunk=32, reps=3, rotate_mb=600):
    """The layer's GEMMs and the LM head (config-2 weights) over T=512 positions
    in 32-position chunks (int8 MFMA), each chunk reading a different copy of the
    weights (>= 600 MB rotated) as a layer-by-layer prefill re-reads its weights
    from HBM per chunk. Its roofline is HBM (weight bytes per chunk); the same
    work as one T=512 launch per GEMM is reported against the int8 MFMA peak."""
    from pulsar_amd.hiptime import Event
    shapes = [(name, N, K) for (name, N, K, _) in SHAPES]
    per_set = sum(pq.lib().pq_q8_packed_codes_bytes(N, K) + pq.lib().pq_q8_packed_scales_bytes(N, K)
                  for (_, N, K) in shapes)
    ncopy = max(2, -(-rotate_mb * 1000000 // per_set))
    sets = []
    for _ in range(ncopy):
        ws = {}
        for (name, N, K) in shapes:
            codes = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
            scales = (torch.randn((N, K // 32), device=dev, generator=g).abs() * 0.01).half().view(torch.int16)
            ws[name] = pq.Q8Weight(codes, scales)
            del codes, scales
        sets.append(ws)
    xs = {K: pq.q8_quant(torch.randn((T, K), device=dev, generator=g)) for K in (2048, 8192)}
    outs = {name: torch.empty((T, N), dtype=torch.bfloat16, device=dev) for (name, N, K) in shapes}
    wsz = max(pq.lib().pq_q8_gemm_workspace_bytes(N, K, t) for (_, N, K) in shapes for t in (chunk, T))
    wsp = torch.empty(max(wsz, 16), dtype=torch.uint8, device=dev)
    stream = pq.stream_ptr()

    def run():
        for ci, c0 in enumerate(range(0, T, chunk)):
            ws = sets[ci % ncopy]
            for (name, N, K) in shapes:
                qx, dx = xs[K]
                pq.q8_gemm(ws[name], qx[c0:c0 + chunk], dx[c0:c0 + chunk], out_dtype=pq.DT_BF16,
                           out=outs[name][c0:c0 + chunk], ws=wsp)

    def run_full(r):
        ws = sets[r % ncopy]
        for (name, N, K) in shapes:
            qx, dx = xs[K]
            pq.q8_gemm(ws[name], qx, dx, out_dtype=pq.DT_BF16, out=outs[name], ws=wsp)

    g_run = graph_of(torch, run)
    ms = timed_replay(torch, g_run, stream, reps)
    del g_run
    ops = sum(2 * N * K * T for (_, N, K) in shapes)
    wbytes = per_set * (T // chunk)
    g_full = graph_of(torch, lambda: [run_full(r) for r in range(ncopy)])
    ms_full = timed_replay(torch, g_full, stream, reps) / ncopy
    del g_full
    return {"T": T, "chunk": chunk, "gemms": [f"{n}:{N}x{K}" for (n, N, K) in shapes], "ms": round(ms, 4),
            "TOPS": round(ops / (ms * 1e-3) / 1e12, 2), "int8_peak_frac": round(ops / (ms * 1e-3) / 1e12 / 5000.0, 4),
            "weight_bytes_read": wbytes, "GB/s": round(wbytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "ops": ops,
            "weight_copies_rotated": ncopy,
            "single_launch_ms": round(ms_full, 4), "single_launch_TOPS": round(ops / (ms_full * 1e-3) / 1e12, 2),
            "single_launch_int8_peak_frac": round(ops / (ms_full * 1e-3) / 1e12 / 5000.0, 4)}


def prefill_profile_workload(pq, torch, dev, reps=3):
    """A workload for rocprofv3 counter runs (--prefill-profile): each GEMM of
    the layer and the LM head, one weight copy, `reps` eager launches over T=512
    positions and then `reps` over one 32-position chunk, bf16 y. Prints a line
    per (GEMM, T) as it finishes; nothing is timed here."""
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    for (name, N, K, _) in SHAPES:
        codes = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
        scales = (torch.randn((N, K // 32), device=dev, generator=g).abs() * 0.01).half().view(torch.int16)
        w = pq.Q8Weight(codes, scales)
        del codes, scales
        for T in (512, 32):
            qx, dx = pq.q8_quant(torch.randn(T, K, device=dev, generator=g))
            y = torch.empty(T, N, dtype=torch.bfloat16, device=dev)
            wsp = torch.empty(max(16, pq.lib().pq_q8_gemm_workspace_bytes(N, K, T)), dtype=torch.uint8, device=dev)
            for _ in range(reps):
                pq.q8_gemm(w, qx, dx, out_dtype=pq.DT_BF16, out=y, ws=wsp)
            torch.cuda.synchronize()
            print(f"prefill profile: {name} {N}x{K} T={T} x{reps}", flush=True)
        del w
        torch.cuda.empty_cache()


def ref_numerics_bench(pq, torch, dev, g, reps=20, rotate_mb=700):
    """The config-2 step through the reference-numerics GEMV (pq_q8r_gemv: the
    reference's own order, bf16 x, fp32 weight scales, row-major codes),
    weights rotated over > 256 MB. Bytes per step: codes + fp32 scales + the
    bf16 x + y."""
    set_bytes = sum(N * K + N * (K // 32) * 4 for (_, N, K, _) in SHAPES)
    ncopy = max(2, math.ceil(rotate_mb * 1e6 / set_bytes))
    copies = []
    for _ in range(ncopy):
        ws = {}
        for (name, N, K, _) in SHAPES:
            ws[name] = (torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g),
                        torch.randn((N, K // 32), device=dev, generator=g).abs() * 0.01)
        copies.append(ws)
    xs = {K: torch.randn(K, device=dev, generator=g).to(torch.bfloat16) for K in (2048, 8192)}
    outs = {name: torch.empty(N, dtype=torch.float32 if o == "f32" else torch.bfloat16, device=dev)
            for (name, N, K, o) in SHAPES}
    stream = pq.stream_ptr()

    def gemv(ws, name, N, K, o):
        c, sc = ws[name]
        pq.q8r_gemv(c, sc, xs[K], out_dtype=pq.DT_F32 if o == "f32" else pq.DT_BF16, out=outs[name])

    def step(i):
        for (name, N, K, o) in SHAPES:
            gemv(copies[i % ncopy], name, N, K, o)

    gr = graph_of(torch, lambda: [step(i) for i in range(reps)])
    ms = timed_replay(torch, gr, stream, 3) / reps
    del gr
    per = {}
    for (name, N, K, o) in SHAPES:
        gsh = graph_of(torch, lambda: [gemv(copies[i % ncopy], name, N, K, o) for i in range(30)])
        per[name] = round(timed_replay(torch, gsh, stream, 5) / 30 * 1e3, 2)
        del gsh
    nbytes = sum(N * K + N * (K // 32) * 4 + 2 * K + N * (4 if o == "f32" else 2) for (_, N, K, o) in SHAPES)
    del copies
    torch.cuda.empty_cache()
    return {"us_per_step": round(ms * 1e3, 2), "bytes_per_step": nbytes, "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "per_shape_us": per,
            "weight_copies_rotated": ncopy}


def qlow_bench(pq, torch, dev, g, rotate_mb=600):
    """The four layer GEMVs of the config-2 workload (q|k|v, o_proj, gate+up,
    down) in the reference's Q4 and Q5 formats (pq_qlow_gemv), weights
    rotated. Bytes: packed codes + half2 scales + bf16 x + bf16 y."""
    shapes = [s_ for s_ in SHAPES if s_[0] != "lm_head"]
    stream = pq.stream_ptr()
    res = {}
    for bits in (4, 5):
        set_bytes = sum(pq.lib().pq_qlow_packed_codes_bytes(N, K, bits) + pq.lib().pq_qlow_packed_scales_bytes(N, K, bits)
                        for (_, N, K, _) in shapes)
        ncopy = max(2, math.ceil(rotate_mb * 1e6 / set_bytes))
        copies = []
        for _ in range(ncopy):
            ws = {}
            for (name, N, K, _) in shapes:
                q = torch.randint(0, 2 ** bits, (N, K), dtype=torch.uint8, device=dev, generator=g)
                sc = torch.randn((N, K // 32, 2), device=dev, generator=g).abs().mul(0.01).half().view(torch.int16)
                ws[name] = pq.QlowWeight(q, sc, bits)
                del q, sc
            copies.append(ws)
        xs = {K: torch.randn(K, device=dev, generator=g).to(torch.bfloat16) for K in (2048, 8192)}
        outs = {name: torch.empty(N, dtype=torch.bfloat16, device=dev) for (name, N, K, _) in shapes}

        def step(i):
            for (name, N, K, _) in shapes:
                pq.qlow_gemv(copies[i % ncopy][name], xs[K], out=outs[name])

        reps = 20
        gr = graph_of(torch, lambda: [step(i) for i in range(reps)])
        ms = timed_replay(torch, gr, stream, 3) / reps
        del gr
        per = {}
        for (name, N, K, _) in shapes:
            gsh = graph_of(torch, lambda: [pq.qlow_gemv(copies[i % ncopy][name], xs[K], out=outs[name])
                                           for i in range(30)])
            per[name] = round(timed_replay(torch, gsh, stream, 5) / 30 * 1e3, 2)
            del gsh
        del copies
        torch.cuda.empty_cache()
        nbytes = set_bytes + sum(2 * K + 2 * N for (_, N, K, _) in shapes)
        res[f"q{bits}"] = {"us_per_step": round(ms * 1e3, 2), "bytes_per_step": nbytes,
                           "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                           "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "per_shape_us": per,
                           "weight_copies_rotated": ncopy}
    return res


def ternary_codes(torch, N, K, dev, g):
    """Weights uniform in {-1, 0, +1}: codes {0, 1, 2} packed four per byte."""
    c = torch.randint(0, 3, (N, K // 4, 4), dtype=torch.uint8, device=dev, generator=g)
    return (c[..., 0] | (c[..., 1] << 2) | (c[..., 2] << 4) | (c[..., 3] << 6)).contiguous()


def ternary_bench(pq, torch, dev, g, reps=50, rotate_mb=400):
    """PQ2_0 x Q8_K GEMVs of a Qwen3-8B-shaped FFN at T=1: gate and up 12288x4096,
    down 4096x12288, weights rotated over > 256 MB."""
    from pulsar_amd.hiptime import Event
    shapes = [("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]
    per_set = sum(N * K // 4 + N * K // 128 * 2 for (_, N, K) in shapes)
    ncopy = max(2, -(-rotate_mb * 1000000 // per_set))
    sets = []
    for _ in range(ncopy):
        sets.append({name: (ternary_codes(torch, N, K, dev, g),
                            (torch.randn((N, K // 128), device=dev, generator=g).abs() * 0.01).half()
                            .view(torch.int16))
                     for (name, N, K) in shapes})
    x4 = pq.q8k_quant(torch.randn(4096, device=dev, generator=g))
    x12 = pq.q8k_quant(torch.randn(12288, device=dev, generator=g))
    outs = {name: torch.empty(N, dtype=torch.float32, device=dev) for (name, N, K) in shapes}
    stream = pq.stream_ptr()

    def gemv(i, name, N, K):
        ws = sets[i % ncopy]
        pq.tq2_gemv(ws[name][0], ws[name][1], x12 if K == 12288 else x4, K, N, out=outs[name])

    # launch period per shape: back-to-back launches, weights rotating, HIP events on the launch stream
    per = []
    for (name, N, K) in shapes:
        gsh = graph_of(torch, lambda: [gemv(i, name, N, K) for i in range(reps)])
        per.append(timed_replay(torch, gsh, stream, 3) / reps)
        del gsh
    step_bytes = sum(N * K // 4 + N * K // 128 * 2 + K // 256 * 292 + N * 4 for (_, N, K) in shapes)
    us = sum(per) * 1e3
    return {"shapes": [f"{n}:{N}x{K}" for (n, N, K) in shapes], "us_per_step": round(us, 2),
            "bytes_per_step": step_bytes, "GB/s": round(step_bytes / (us * 1e-6) / 1e9, 1),
            "hbm_frac": round(step_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "per_shape_us": [round(p * 1e3, 2) for p in per], "weight_copies_rotated": ncopy}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the decode and prefill measurements")
    ap.add_argument("--calib", action="store_true",
                    help="also run a plain elementwise kernel over 256 MiB (counter calibration for rocprofv3 --pmc)")
    ap.add_argument("--rotate-mb", type=int, default=600)
    ap.add_argument("--prefill-profile", action="store_true",
                    help="only run the prefill GEMMs (3 launches each at T=512 and T=32) for counter runs; no JSON")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: there is no multi-GPU path (the GEMV would shard by rows, with an "
              "all-gather of the outputs). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import pulsar_amd as pq

    dev = torch.device("cuda:0")
    if args.prefill_profile:
        prefill_profile_workload(pq, torch, dev)
        return
    torch.manual_seed(20261201)
    g = torch.Generator(device=dev)
    g.manual_seed(20261201)
    set_bytes = sum(pq.lib().pq_q8_packed_codes_bytes(N, K) + pq.lib().pq_q8_packed_scales_bytes(N, K)
                    for (_, N, K, _) in SHAPES)
    ncopy = max(2, math.ceil(args.rotate_mb * 1e6 / set_bytes))
    copies = []
    for c in range(ncopy):
        ws = {}
        for (name, N, K, _) in SHAPES:
            codes = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
            scales = (torch.randn((N, K // 32), device=dev, generator=g).abs() * 0.01).half().view(torch.int16)
            ws[name] = pq.Q8Weight(codes, scales)
            del codes, scales
        copies.append(ws)
    x2 = torch.randn(2048, device=dev, generator=g)
    x8 = torch.randn(8192, device=dev, generator=g)
    outs = {name: torch.empty(N, dtype=torch.float32 if o == "f32" else torch.bfloat16, device=dev)
            for (name, N, K, o) in SHAPES}
    torch.cuda.synchronize()

    from pulsar_amd.hiptime import Event
    stream = pq.stream_ptr()

    def gemv(ws, name, N, K, o):
        pq.gemv_fused(ws[name], pq.PRO_F32, out_dtype=pq.DT_F32 if o == "f32" else pq.DT_BF16, out=outs[name],
                      xf=x8 if K == 8192 else x2)

    def step(i):
        ws = copies[i % ncopy]
        for (name, N, K, o) in SHAPES:
            gemv(ws, name, N, K, o)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # the K timed steps, captured as one graph (launches as the engine issues them)
    g_steps = graph_of(torch, lambda: [step(i) for i in range(args.steps)])
    ms_per_step = timed_replay(torch, g_steps, stream) / args.steps
    del g_steps

    # launch period of the GEMV kernel per shape: back-to-back launches of that
    # shape (weights rotating over the copies), HIP events on the launch stream
    per = {}
    nper = 30
    for (name, N, K, o) in SHAPES:
        gsh = graph_of(torch, lambda: [gemv(copies[i % ncopy], name, N, K, o) for i in range(nper)])
        per[name] = timed_replay(torch, gsh, stream, reps=5) / nper
        del gsh

    step_bytes = sum(gemv_bytes(N, K, o) for (_, N, K, o) in SHAPES)
    gemv_ms = sum(per.values())
    achieved = step_bytes / (gemv_ms * 1e-3) / 1e9
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    per_shape = {name: {"us": round(per[name] * 1e3, 2),
                        "GB/s": round(gemv_bytes(N, K, o) / (per[name] * 1e-3) / 1e9, 1)}
                 for (name, N, K, o) in SHAPES}
    lm = [s_ for s_ in SHAPES if s_[0] == "lm_head"][0]

    line = {
        "metric": "Q8 GEMV HBM GB/s (% of peak); backbone decode tok/s on 1 MI355X",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xint8->int32, fp32 scales",
        "data": "synthetic (seeded uniform int8 codes, |N(0,1)|*0.01 fp16 scales, N(0,1) x)",
        "config": {"workload": "one LFM-style layer's T=1 Q8_0 GEMVs + LM head (hidden 2048)",
                   "gpu": gpu_desc(torch, pq),
                   "gemvs": [f"{n}:{N}x{K}" for (n, N, K, _) in SHAPES],
                   "bytes_per_step": step_bytes, "weight_copies_rotated": ncopy,
                   "rotated_MB": round(ncopy * set_bytes / 1e6, 1)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": "q8_gemv_fused_kernel (5 shapes, launch period)", "per_shape": per_shape,
                     "lm_head_frac": round(gemv_bytes(*lm[1:]) / (per["lm_head"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "cpu_baseline": None if args.no_cpu else cpu_baseline(),
    }
    if args.calib:
        src = torch.randn(64 << 20, device=dev)          # 256 MiB read + 256 MiB written per call
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    if not args.no_extra:
        del copies
        torch.cuda.empty_cache()
        line["decode"] = decode_bench(pq)
        line["prefill_gemm"] = prefill_gemm_bench(pq, torch, dev, g)
        line["ternary_gemv"] = ternary_bench(pq, torch, dev, g)
        line["ref_numerics_gemv"] = ref_numerics_bench(pq, torch, dev, g)
        line["qlow_gemv"] = qlow_bench(pq, torch, dev, g)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
