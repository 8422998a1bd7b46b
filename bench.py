"""Benchmark: Q8_0 GEMV HBM throughput on one MI355X (one LFM-style layer's GEMVs + LM head).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one pass of the decode hot path over one synthetic layer at T=1: the
GEMVs fused q|k|v 3072x2048, o_proj 2048x2048, gate+up 16384x2048, down
2048x8192 and the LM head 65536x2048 (fp32 logits), from packed Q8_0 weights
resident in HBM, each quantizing its fp32 x (K=2048 or 8192) to Q8_0 in its own
prologue (q8_gemv_fused_kernel, PQ_PRO_F32). Every shape reads its weights from
its own pool of >= 300 MB of distinct copies, rotated launch by launch, so no
launch finds its weights in the 256 MB Infinity Cache.

Prints ONE JSON line. value = algorithmic bytes per step / time per step (GB/s;
the K steps are one captured graph, the median of 5 timed replays, HIP events
on the launch stream). roofline = the GEMV kernel's algorithmic bytes per
launch / its average launch duration over that timed region (the region's
time / its 5K launches; every launch of the step is q8_gemv_fused_kernel),
against 8 TB/s, with each shape's back-to-back launch period beside it. cpu_baseline = the reference's own CPU
GEMV (.auto/lfm3/q8_gemv_cpu.c gemv_q8, compiled into oracle/_ref) on the host
cores over a bounded sample of the same shapes. The other keys are the single
8192x2048 GEMV, the 24-layer backbone decode and its prompt prefill, the prefill
GEMMs, the ternary GEMVs, the reference-numerics GEMVs and Q4/Q5, each with its
own roofline and, where the reference has a CPU path, its CPU figure.
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "pulsar-asm_amd"))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
ROTATE_MB = 300          # distinct weight bytes per shape, rotated (> the 256 MB Infinity Cache)
SHAPES = [  # name, N, K, output dtype
    ("qkv", 3072, 2048, "bf16"),
    ("o_proj", 2048, 2048, "bf16"),
    ("gate_up", 16384, 2048, "bf16"),
    ("down", 2048, 8192, "bf16"),
    ("lm_head", 65536, 2048, "f32"),
]


def measured_traffic():
    """HBM bytes of one step's 5 GEMV launches, from the two rocprofv3 --pmc
    passes summarised in profiles/q8_gemv_hbm_traffic.md (None if absent)."""
    import re
    path = os.path.join(ROOT, "profiles", "q8_gemv_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"\| step \(5 GEMVs\) \| [0-9.]+ \| ([0-9.]+) \|", open(path).read())
    return int(float(m.group(1)) * 1e6) if m else None


def profile_traffic(fname):
    """Measured HBM bytes per launch from a counter summary under profiles/
    (tables `| shape | kernel | grid | algorithmic MB | FETCH_SIZE KiB |
    WRITE_SIZE KiB | measured HBM MB | ratio |`, one per `## ` section):
    {section: {shape: bytes}} ({} if the file is absent)."""
    import re
    path = os.path.join(ROOT, "profiles", fname)
    if not os.path.exists(path):
        return {}
    out, sec = {}, ""
    for line in open(path):
        if line.startswith("## "):
            sec = line[3:].strip()
        m = re.match(r"\| ([^|`]+) \| `[^`]+` \| \d+ \| [0-9.]+ \| [0-9.]+ \| [0-9.]+ \| ([0-9.]+) \| [0-9.]+ \|", line)
        if m:
            out.setdefault(sec, {})[m.group(1).strip()] = int(float(m.group(2)) * 1e6)
    return out


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


def timed_replay(torch, g, stream, reps=5):
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
    return statistics.median(ev[i].elapsed_ms(ev[i + 1]) for i in range(reps))


def period_ms(torch, launch, n, stream):
    """Launch period: n back-to-back launches (launch(i), rotating weights) in one
    graph, median of 5 replays, divided by n (includes the gap between launches)."""
    g = graph_of(torch, lambda: [launch(i) for i in range(n)])
    ms = timed_replay(torch, g, stream) / n
    del g
    return ms


def copies_for(nbytes, min_mb=ROTATE_MB):
    return max(2, math.ceil(min_mb * 1e6 / nbytes))


def q8_pool(pq, torch, dev, g, N, K, min_mb=ROTATE_MB):
    """Distinct packed Q8_0 copies of an N x K weight, >= min_mb in all."""
    per = pq.lib().pq_q8_packed_codes_bytes(N, K) + pq.lib().pq_q8_packed_scales_bytes(N, K)
    pool = []
    for _ in range(copies_for(per, min_mb)):
        codes = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
        scales = (torch.randn((N, K // 32), device=dev, generator=g).abs() * 0.01).half().view(torch.int16)
        pool.append(pq.Q8Weight(codes, scales))
        del codes, scales
    return pool, per


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


# ------------------------------------------------------------------ CPU side
def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle
    return pyoracle


def _host():
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return f"{model}, nproc {os.cpu_count()}"


def _timed(fn, sec):
    """(passes, seconds per pass) of fn over about sec seconds, after one untimed pass."""
    fn()
    n = 0
    t0 = time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= sec:
            return n, dt / n


def _all_and_one_core(ref, fn, sec):
    """fn timed on the OpenMP team (all cores), then on one core for half as long."""
    threads = int(ref.ref_max_threads())
    n_all, dt_all = _timed(fn, sec)
    n_one, dt_one = None, None
    if threads > 1:
        ref.ref_set_threads(1)
        try:
            n_one, dt_one = _timed(fn, sec / 2)
        finally:
            ref.ref_set_threads(threads)
    return threads, (n_all, dt_all), (n_one, dt_one)


def cpu_q8_gemv(shapes, seconds):
    """The reference's gemv_q8 (fp32 x, fp32 scales; q8_gemv_cpu.c:29-58, OpenMP
    over rows) over the given (N, K) shapes: GB/s of its own bytes per pass, on
    all host cores and on one."""
    import ctypes as C
    import numpy as np
    orc = _oracle()
    ref = orc.ref()
    if ref is None:
        return None
    data = []
    for i, (N, K) in enumerate(shapes):
        W = orc.gen_codes(20261201 + 4 * i, N * K).reshape(N, K)
        S = orc.gen_scales(20261201 + 4 * i + 1, N * (K // 32)).view(np.float16).astype(np.float32)
        x = orc.gen_normal(20261201 + 4 * i + 2, K)
        data.append((N, K, W, S.reshape(N, K // 32), x, np.empty(N, np.float32)))

    def run():
        for (N, K, W, S, x, y) in data:
            ref.ref_q8_gemv(W.ctypes.data_as(C.c_void_p), S.ctypes.data_as(C.c_void_p),
                            x.ctypes.data_as(C.c_void_p), y.ctypes.data_as(C.c_void_p), C.c_int(N), C.c_int(K))

    nbytes = sum(N * K + N * (K // 32) * 4 + K * 4 + N * 4 for (N, K) in shapes)
    threads, (n, dt), (n1, dt1) = _all_and_one_core(ref, run, seconds)
    return {"value": round(nbytes / dt / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "reference",
            "ms_per_pass": round(dt * 1e3, 3),
            "one_core": None if dt1 is None else {"value": round(nbytes / dt1 / 1e9, 2),
                                                  "ms_per_pass": round(dt1 * 1e3, 3), "passes": n1},
            "host": _host(),
            "sample": f"{n} passes of {len(shapes)} GEMV shape(s) {['%dx%d' % s for s in shapes]} through gemv_q8 "
                      f"(q8_gemv_cpu.c:29-58; fp32 x and fp32 scales, {nbytes / 1e6:.1f} MB/pass)"}


def cpu_ternary(shapes, seconds):
    """The reference's pq2_gemv_cpu (pq2_host.c:82-104) on the config-5 shapes:
    row slices on an OpenMP team (ref_pq2_gemv_rows; rows are independent), and
    the serial routine on one core."""
    import ctypes as C
    import numpy as np
    orc = _oracle()
    ref = orc.ref()
    if ref is None:
        return None
    data = []
    for i, (N, K) in enumerate(shapes):
        codes = orc.gen_ternary(777 + i, N * K // 4)
        S = orc.gen_scales(778 + i, N * K // 128)
        xq = orc.q8k_quant(orc.gen_normal(779 + i, K))
        data.append((N, K, codes, S, xq, np.empty(N, np.float32)))

    def run():
        for (N, K, c, s, xq, y) in data:
            ref.ref_pq2_gemv_rows(C.c_int(N), C.c_int(K), c.ctypes.data_as(C.c_void_p), s.ctypes.data_as(C.c_void_p),
                                  xq.ctypes.data_as(C.c_void_p), y.ctypes.data_as(C.c_void_p))

    nbytes = sum(N * K // 4 + N * K // 128 * 2 + K // 256 * 292 + N * 4 for (N, K) in shapes)
    threads, (n, dt), (n1, dt1) = _all_and_one_core(ref, run, seconds)
    return {"value": round(nbytes / dt / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "reference",
            "us_per_pass": round(dt * 1e6, 1),
            "one_core": None if dt1 is None else {"value": round(nbytes / dt1 / 1e9, 2),
                                                  "us_per_pass": round(dt1 * 1e6, 1), "passes": n1},
            "host": _host(),
            "sample": f"{n} passes of the gate, up and down GEMVs through pq2_gemv_cpu "
                      f"({nbytes / 1e6:.1f} MB/pass)"}


def cpu_backbone(cfg, n_prompt=8, n_steps=12):
    """The oracle's 24-layer backbone (the C restatement, OpenMP over
    GEMV rows): decode tok/s after a short prompt. A port, not the reference's
    code: the reference's x86 LFM3 engine is a stub."""
    import numpy as np
    orc = _oracle()
    m = orc.Model(**{k: v for k, v in cfg.items() if k != "prefill_chunk"})
    r = m.feed(orc.gen_tokens(5, n_prompt, cfg["vocab"]))
    t0 = time.perf_counter()
    for _ in range(n_steps):
        r = m.feed(np.array([r], np.int32))
    dt = (time.perf_counter() - t0) / n_steps
    m.close()
    return {"value": round(1.0 / dt, 2), "unit": "tok/s", "cores": int(orc.lib().orc_max_threads()), "kind": "port",
            "ms_per_token": round(dt * 1e3, 1), "host": _host(),
            "sample": f"{n_steps} greedy T=1 steps of the oracle backbone after a {n_prompt}-token prompt"}


# ------------------------------------------------------------------ GPU side
def config1_bench(pq, torch, dev, g, stream, n=100):
    """The single Q8_0 GEMV, 8192x2048, fp32 x quantized in the prologue, fp32 y."""
    N, K = 8192, 2048
    pool, per = q8_pool(pq, torch, dev, g, N, K)
    x = torch.randn(K, device=dev, generator=g)
    y = torch.empty(N, dtype=torch.float32, device=dev)

    def launch(i):
        pq.gemv_fused(pool[i % len(pool)], pq.PRO_F32, out_dtype=pq.DT_F32, out=y, xf=x)

    per_ms = period_ms(torch, launch, n, stream)
    nb = gemv_bytes(N, K, "f32")
    ncopy = len(pool)
    del pool
    torch.cuda.empty_cache()
    return {"gemv": f"{N}x{K}", "bytes": nb, "us": round(per_ms * 1e3, 2),
            "GB/s": round(nb / (per_ms * 1e-3) / 1e9, 1), "hbm_frac": round(nb / (per_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "timed": f"{n} back-to-back launches in one graph, median of 5 replays",
            "weight_copies_rotated": ncopy, "rotated_MB": round(ncopy * per / 1e6, 1)}


def decode_bench(pq, n_steps=64, n_prompt=256, reps=3):
    """Backbone decode tok/s: the synthetic 24-layer LFM3-style model, a 256-token
    prompt (layer-major prefill), then n_steps T=1 greedy steps timed on the
    engine's stream; the median over reps prompt + decode runs. The prompt is
    also timed in the reference's 32-position chunks."""
    from pulsar_amd.engine import LFM3_SYNTH, Engine, synth_fill
    from pulsar_amd.hiptime import Event
    e = Engine(**LFM3_SYNTH)
    e.load_synthetic()
    prompt = synth_fill(5, LFM3_SYNTH["seed"] + 4 * 5000, n_prompt, float(LFM3_SYNTH["vocab"]))
    st = e.stream()
    e.reset()
    e.feed(prompt)                       # warm-up prefill and steps
    e.decode(4, want_ids=False)
    e.sync()
    pre, dec = [], []
    for _ in range(reps):
        a, b, c = Event(), Event(), Event()
        e.reset()
        a.record(st)
        e.feed(prompt)                   # the timed prefill (one 256-position chunk per layer)
        b.record(st)
        e.decode(n_steps, want_ids=False)
        c.record(st)
        e.sync()
        pre.append(a.elapsed_ms(b))
        dec.append(b.elapsed_ms(c) / n_steps)
    ms, prefill_ms = statistics.median(dec), statistics.median(pre)
    e.set_chunk(32)                      # the reference's 32-position chunks, layer-major
    pre32 = []
    for _ in range(reps):
        a, b = Event(), Event()
        e.reset()
        a.record(st)
        e.feed(prompt)
        b.record(st)
        e.sync()
        pre32.append(a.elapsed_ms(b))
    prefill32_ms = statistics.median(pre32)
    wbytes = e.weight_bytes()
    kv = 8 * 2 * 8 * 64 * 2  # attention layers x (k, v) x kv heads x dim x fp16, per position
    mean_pos = n_prompt + n_steps / 2
    tok_bytes = wbytes + kv * mean_pos
    e.close()
    return {"tok_s": round(1e3 / ms, 1), "ms_per_token": round(ms, 4), "steps": n_steps, "runs": reps,
            "positions": f"{n_prompt}..{n_prompt + n_steps}", "bytes_per_token": int(tok_bytes),
            "GB/s": round(tok_bytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(tok_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "prefill_ms_256": round(prefill_ms, 2), "prefill_tok_s": round(n_prompt / (prefill_ms * 1e-3), 1),
            "prefill_chunk": LFM3_SYNTH["prefill_chunk"], "prefill_order": "layer-major",
            "prefill_ms_256_chunk32": round(prefill32_ms, 2)}


# the real LFM3 backbone's shapes and layer pattern (synthetic weights): 13
# conv layers, 6 full and 5 sliding-window attention layers, head_dim 128,
# FFN 7680, vocab 128000, 7-tap conv
LFM3_REAL = dict(hidden=2048, ffn=7680, vocab=128000, nlayers=24, nh=16, nkv=4, hd=128, rot=64, ntaps=7, ctx=2048,
                 eps=1e-5, theta=1e6, seed=20261201, attn_mask=sum(1 << l for l in range(2, 24, 2)),
                 slide_mask=sum(1 << l for l in range(4, 24, 4)), slide_win=256, slide_rot=128, slide_theta=1e4,
                 prefill_chunk=256)


def decode_variant(pq, cfg, n_steps=32, n_prompt=256, blob=None):
    """tok/s of n_steps greedy steps after a 256-token prompt (median of 3 runs)
    for another engine configuration (synthetic weights, or those of a blob)."""
    from pulsar_amd.engine import Engine, synth_fill
    from pulsar_amd.hiptime import Event
    e = Engine(**cfg)
    if blob:
        e.load_blob(blob)
    else:
        e.load_synthetic()
    prompt = synth_fill(5, cfg["seed"] + 4 * 5000, n_prompt, float(cfg["vocab"]))
    st = e.stream()
    e.reset()
    e.feed(prompt)
    e.decode(2, want_ids=False)
    e.sync()
    pre, dec = [], []
    for _ in range(3):
        a, b, c = Event(), Event(), Event()
        e.reset()
        a.record(st)
        e.feed(prompt)
        b.record(st)
        e.decode(n_steps, want_ids=False)
        c.record(st)
        e.sync()
        pre.append(a.elapsed_ms(b))
        dec.append(b.elapsed_ms(c) / n_steps)
    ms = statistics.median(dec)
    wbytes = e.weight_bytes()
    e.close()
    return {"tok_s": round(1e3 / ms, 1), "ms_per_token": round(ms, 4), "weight_bytes": wbytes,
            "GB/s": round(wbytes / (ms * 1e-3) / 1e9, 1), "hbm_frac": round(wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "prefill_ms_256": round(statistics.median(pre), 2), "steps": n_steps}


def lowbit_blob(pq, torch, dev, g, cfg, bits, path):
    """An .lfm3q8 file of the synthetic backbone's shapes with random weights,
    written with the product's own blob writer: every layer's linears Q4 / Q5
    (dtype 6 / 7, packed on the GPU by pq_qlow_pack into the exporter's tiled
    payload) but the attention gate_proj (16 or 32 rows), which stays Q8 as in
    the real LFM3 shapes; the tied table Q8; the norms and conv taps fp32."""
    import numpy as np
    from pulsar_amd.blob import write_blob
    H, F = cfg["hidden"], cfg["ffn"]
    qd, kd = cfg["nh"] * cfg["hd"], cfg["nkv"] * cfg["hd"]

    def q8(N, K):
        c = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
        s = (torch.randn((N, K // 32), device=dev, generator=g).abs() * 0.01).half().float()
        return c.cpu().numpy(), s.cpu().numpy()

    def low(N, K):
        c = torch.randint(0, 2 ** bits, (N, K), dtype=torch.uint8, device=dev, generator=g)
        dp = (torch.randn((N, K // 32), device=dev, generator=g).abs() * (2560.0 / 2 ** bits)).half()
        mn = (-(2 ** bits - 1) * 0.5 * dp.float() / 128.0).half()
        w = pq.QlowWeight(c, torch.stack([dp, mn], -1).view(torch.int16).contiguous(), bits)
        return ("qlow", bits, N, K, w.pcodes.cpu().numpy(), w.pscales.cpu().numpy().view(np.uint16))

    def vec(n, a, b):
        return (a + b * torch.randn(n, device=dev, generator=g)).cpu().numpy().astype(np.float32)

    ts = [("lfm.model.embed_tokens.weight", q8(cfg["vocab"], H))]
    for l in range(cfg["nlayers"]):
        P = f"lfm.model.layers.{l}."
        if (cfg["attn_mask"] >> l) & 1:
            ts += [(P + "self_attn.q_proj.weight", low(qd, H)), (P + "self_attn.k_proj.weight", low(kd, H)),
                   (P + "self_attn.v_proj.weight", low(kd, H)), (P + "self_attn.gate_proj.weight", q8(cfg["nh"], H)),
                   (P + "self_attn.o_proj.weight", low(H, qd)),
                   (P + "self_attn.q_norm.weight", vec(cfg["hd"], 1.0, 0.1)),
                   (P + "self_attn.k_norm.weight", vec(cfg["hd"], 1.0, 0.1))]
        else:
            ts += [(P + "conv.in_proj.weight", low(3 * H, H)), (P + "conv.out_proj.weight", low(H, H)),
                   (P + "conv.conv.weight", vec(H * cfg["ntaps"], 0.0, 0.5).reshape(H, 1, cfg["ntaps"]))]
        ts += [(P + "feed_forward.w1.weight", low(F, H)), (P + "feed_forward.w3.weight", low(F, H)),
               (P + "feed_forward.w2.weight", low(H, F))]
        for nm, a, b in (("operator_norm", 1.0, 0.1), ("post_operator_norm", 4.0, 0.4), ("ffn_norm", 1.0, 0.1),
                         ("post_ffn_norm", 4.0, 0.4)):
            ts.append((P + nm + ".weight", vec(H, a, b)))
    ts.append(("lfm.model.embedding_norm.weight", vec(H, 1.0, 0.1)))
    kinds = ["full_attention" if (cfg["attn_mask"] >> l) & 1 else "conv" for l in range(cfg["nlayers"])]
    write_blob(path, {"hidden_size": H, "vocab_size": cfg["vocab"], "layer_types": kinds}, ts)


def decode_lowbit(pq, torch, dev, g, bits=4, n_steps=32, n_prompt=256):
    """The synthetic 24-layer backbone with Q4 (or Q5) linears from an .lfm3q8
    file, under the reference numerics (bf16 activations, as the reference runs
    its low-bit tensors): decode tok/s after a 256-token prompt, the bytes a step
    reads (the packed low-bit payloads) and their rate."""
    import tempfile
    from pulsar_amd.engine import LFM3_SYNTH
    cfg = dict(LFM3_SYNTH, numerics=1)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, f"q{bits}.lfm3q8")
        lowbit_blob(pq, torch, dev, g, cfg, bits, path)
        out = decode_variant(pq, cfg, n_steps=n_steps, n_prompt=n_prompt, blob=path)
    out["weights"] = f"Q{bits} linears (gate_proj Q8), Q8 table"
    return out


def prefill_gemm_bench(pq, torch, dev, g, stream, gpu, T=512, chunk=32):
    """Config 3: the layer's GEMMs and the LM head on fp32 activations over
    T=512 positions in 32-position chunks. Each chunk quantizes its fp32 rows
    (pq_q8_quant_f32, inside the timed region) and runs the five int8-MFMA
    GEMMs on a different copy of the weights (>= 300 MB rotated), as a prefill
    that streams its weights per chunk re-reads them from HBM. Reported against
    HBM (weight bytes per chunk), the int8 MFMA peak, and the VALU ceiling of
    the R1 epilogue (three VALU lane-ops per 32-MAC block product); the same
    work as one T=512 launch per GEMM is reported beside it."""
    shapes = [(name, N, K) for (name, N, K, _) in SHAPES]
    per_set = sum(pq.lib().pq_q8_packed_codes_bytes(N, K) + pq.lib().pq_q8_packed_scales_bytes(N, K)
                  for (_, N, K) in shapes)
    ncopy = copies_for(per_set)
    sets = []
    for _ in range(ncopy):
        ws = {}
        for (name, N, K) in shapes:
            codes = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
            scales = (torch.randn((N, K // 32), device=dev, generator=g).abs() * 0.01).half().view(torch.int16)
            ws[name] = pq.Q8Weight(codes, scales)
            del codes, scales
        sets.append(ws)
    xf = {K: torch.randn((T, K), device=dev, generator=g) for K in (2048, 8192)}
    q = {K: (torch.empty((T, K), dtype=torch.int8, device=dev), torch.empty((T, K // 32), dtype=torch.float32,
                                                                             device=dev)) for K in (2048, 8192)}
    outs = {name: torch.empty((T, N), dtype=torch.bfloat16, device=dev) for (name, N, K) in shapes}
    wsz = max(pq.lib().pq_q8_gemm_workspace_bytes(N, K, t) for (_, N, K) in shapes for t in (chunk, T))
    wsp = torch.empty(max(wsz, 16), dtype=torch.uint8, device=dev)

    def quant(K, c0, c1):
        qx, dx = q[K]
        pq.check(pq.lib().pq_q8_quant_f32(xf[K][c0:c1].data_ptr(), qx[c0:c1].data_ptr(), dx[c0:c1].data_ptr(), K,
                                          c1 - c0, pq.stream_ptr()), "pq_q8_quant_f32")

    def run():
        for ci, c0 in enumerate(range(0, T, chunk)):
            ws = sets[ci % ncopy]
            for K in (2048, 8192):
                quant(K, c0, c0 + chunk)
            for (name, N, K) in shapes:
                qx, dx = q[K]
                pq.q8_gemm(ws[name], qx[c0:c0 + chunk], dx[c0:c0 + chunk], out_dtype=pq.DT_BF16,
                           out=outs[name][c0:c0 + chunk], ws=wsp)

    # the reference's layer-major order (LFM_PF_LM, lfm3_nanode.cu:5935-5955, the engine's prefill order):
    # each GEMM runs its 16 chunks back to back on one weight copy, so its chunks after the first find
    # the weights in the Infinity Cache; successive runs take the next copy (the first chunk is cold)
    def run_layer_major(r):
        ws = sets[r % ncopy]
        for c0 in range(0, T, chunk):
            for K in (2048, 8192):
                quant(K, c0, c0 + chunk)
        for (name, N, K) in shapes:
            qx, dx = q[K]
            for c0 in range(0, T, chunk):
                pq.q8_gemm(ws[name], qx[c0:c0 + chunk], dx[c0:c0 + chunk], out_dtype=pq.DT_BF16,
                           out=outs[name][c0:c0 + chunk], ws=wsp)

    def run_full(r):
        ws = sets[r % ncopy]
        for K in (2048, 8192):
            quant(K, 0, T)
        for (name, N, K) in shapes:
            qx, dx = q[K]
            pq.q8_gemm(ws[name], qx, dx, out_dtype=pq.DT_BF16, out=outs[name], ws=wsp)

    g_run = graph_of(torch, run)
    ms = timed_replay(torch, g_run, stream)
    del g_run
    ops = sum(2 * N * K * T for (_, N, K) in shapes)
    wbytes = per_set * (T // chunk)
    g_full = graph_of(torch, lambda: [run_full(r) for r in range(ncopy)])
    ms_full = timed_replay(torch, g_full, stream) / ncopy
    del g_full
    g_lm = graph_of(torch, lambda: [run_layer_major(r) for r in range(ncopy)])
    ms_lm = timed_replay(torch, g_lm, stream) / ncopy
    del g_lm, sets
    torch.cuda.empty_cache()
    # VALU ceiling of the R1 fold: per (row, position, block) one convert, one
    # multiply and one fma on 64 fp32 lanes per CU per clock
    valu_tops = 64 * gpu["cus"] * gpu["clock_MHz"] * 1e6 * (64 / 3) / 1e12
    tops, tops_full = ops / (ms * 1e-3) / 1e12, ops / (ms_full * 1e-3) / 1e12
    return {"T": T, "chunk": chunk, "gemms": [f"{n}:{N}x{K}" for (n, N, K) in shapes], "ms": round(ms, 4),
            "includes": "fp32 -> Q8_0 activation quantization of every chunk",
            "TOPS": round(tops, 2), "int8_peak_frac": round(tops / INT8_PEAK_TOPS, 4),
            "valu_ceiling_TOPS": round(valu_tops, 1), "valu_ceiling_frac": round(tops / valu_tops, 4),
            "weight_bytes_read": wbytes, "GB/s": round(wbytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "ops": ops,
            "weight_copies_rotated": ncopy,
            "single_launch_ms": round(ms_full, 4), "single_launch_TOPS": round(tops_full, 2),
            "single_launch_int8_peak_frac": round(tops_full / INT8_PEAK_TOPS, 4),
            "single_launch_valu_ceiling_frac": round(tops_full / valu_tops, 4),
            "layer_major": {"ms": round(ms_lm, 4), "TOPS": round(ops / (ms_lm * 1e-3) / 1e12, 2),
                            "int8_peak_frac": round(ops / (ms_lm * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
                            "valu_ceiling_frac": round(ops / (ms_lm * 1e-3) / 1e12 / valu_tops, 4),
                            "order": "each GEMM's 16 chunks back to back on one weight copy (the reference's "
                                     "LFM_PF_LM order); the copy changes per run"}}


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


def _per_shape(pq, torch, stream, shapes, launch_of, nbytes_of, n=30):
    """Per shape: the launch period of n back-to-back launches over its rotated
    pool (one graph, HIP events on the launch stream)."""
    per = {}
    for s in shapes:
        name = s[0]
        prd = period_ms(torch, launch_of(s), n, stream)
        nb = nbytes_of(s)
        per[name] = {"us": round(prd * 1e3, 2), "GB/s": round(nb / (prd * 1e-3) / 1e9, 1)}
    return per


def read_floor(pq, torch, dev, stream, named_bytes, n=40):
    """Per shape: the launch period of pq_stream_read over the same number of
    bytes (a plain streaming read, 1024 x 512 threads, no arithmetic), n
    back-to-back launches at rotating offsets of a 1 GiB buffer, one graph.
    It is the practical ceiling of one launch that reads that many bytes (the
    launch and first-byte latency included), which the GEMV periods are read
    against."""
    pool = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    pool.fill_(1)
    sink = torch.zeros(1, dtype=torch.float32, device=dev)
    out = {}
    for name, nb in named_bytes:
        nb16 = nb // 16 * 16
        span = (nb16 + 4095) // 4096 * 4096
        nslots = max(1, pool.numel() // span)

        def launch(i, nb16=nb16, span=span, nslots=nslots):
            pq.check(pq.lib().pq_stream_read(pool.data_ptr() + (i % nslots) * span, nb16, sink.data_ptr(),
                                             pq.stream_ptr()), "pq_stream_read")
        prd = period_ms(torch, launch, n, stream)
        out[name] = {"us": round(prd * 1e3, 2), "GB/s": round(nb16 / (prd * 1e-3) / 1e9, 1)}
    del pool
    torch.cuda.empty_cache()
    return out


def ref_numerics_bench(pq, torch, dev, g, stream, reps=20):
    """The config-2 step through the reference-numerics GEMV (pq_q8r_gemv: the
    reference's own order, bf16 x, fp32 weight scales, row-major codes), each
    shape from its own >= 300 MB pool. Bytes: codes + fp32 scales + bf16 x + y."""
    pools = {}
    for (name, N, K, _) in SHAPES:
        pools[name] = [(torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g),
                        torch.randn((N, K // 32), device=dev, generator=g).abs() * 0.01)
                       for _ in range(copies_for(N * K + N * (K // 32) * 4))]
    xs = {K: torch.randn(K, device=dev, generator=g).to(torch.bfloat16) for K in (2048, 8192)}
    outs = {name: torch.empty(N, dtype=torch.float32 if o == "f32" else torch.bfloat16, device=dev)
            for (name, N, K, o) in SHAPES}

    def launch_of(s):
        name, N, K, o = s

        def f(i):
            c, sc = pools[name][i % len(pools[name])]
            pq.q8r_gemv(c, sc, xs[K], out_dtype=pq.DT_F32 if o == "f32" else pq.DT_BF16, out=outs[name])
        return f

    def step(i):
        for s in SHAPES:
            launch_of(s)(i)

    gr = graph_of(torch, lambda: [step(i) for i in range(reps)])
    ms = timed_replay(torch, gr, stream) / reps
    del gr
    nb = {s[0]: s[1] * s[2] + s[1] * (s[2] // 32) * 4 + 2 * s[2] + s[1] * (4 if s[3] == "f32" else 2) for s in SHAPES}
    per = _per_shape(pq, torch, stream, SHAPES, launch_of, lambda s: nb[s[0]])
    nbytes = sum(nb.values())
    kern = sum(p["us"] for p in per.values())
    del pools
    torch.cuda.empty_cache()
    return {"us_per_step": round(ms * 1e3, 2), "bytes_per_step": nbytes, "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "period_us_sum": round(kern, 2), "period_hbm_frac": round(nbytes / (kern * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "per_shape": per, "rotated_MB_per_shape": ROTATE_MB}


def qlow_bench(pq, torch, dev, g, stream, reps=20):
    """The four layer GEMVs of the config-2 workload (q|k|v, o_proj, gate+up,
    down) in the reference's Q4 and Q5 formats (pq_qlow_gemv), each shape from
    its own >= 300 MB pool. Bytes: packed codes + half2 scales + bf16 x + bf16 y."""
    shapes = [s_ for s_ in SHAPES if s_[0] != "lm_head"]
    res = {}
    for bits in (4, 5):
        pools, wb = {}, {}
        for (name, N, K, _) in shapes:
            wb[name] = pq.lib().pq_qlow_packed_codes_bytes(N, K, bits) + pq.lib().pq_qlow_packed_scales_bytes(N, K, bits)
            pool = []
            for _ in range(copies_for(wb[name])):
                qc = torch.randint(0, 2 ** bits, (N, K), dtype=torch.uint8, device=dev, generator=g)
                sc = torch.randn((N, K // 32, 2), device=dev, generator=g).abs().mul(0.01).half().view(torch.int16)
                pool.append(pq.QlowWeight(qc, sc, bits))
                del qc, sc
            pools[name] = pool
        xs = {K: torch.randn(K, device=dev, generator=g).to(torch.bfloat16) for K in (2048, 8192)}
        outs = {name: torch.empty(N, dtype=torch.bfloat16, device=dev) for (name, N, K, _) in shapes}

        def launch_of(s):
            name, N, K, _ = s
            return lambda i: pq.qlow_gemv(pools[name][i % len(pools[name])], xs[K], out=outs[name])

        def step(i):
            for s in shapes:
                launch_of(s)(i)

        gr = graph_of(torch, lambda: [step(i) for i in range(reps)])
        ms = timed_replay(torch, gr, stream) / reps
        del gr
        nb = {s[0]: wb[s[0]] + 2 * s[2] + 2 * s[1] for s in shapes}
        per = _per_shape(pq, torch, stream, shapes, launch_of, lambda s: nb[s[0]])
        nbytes = sum(nb.values())
        kern = sum(p["us"] for p in per.values())
        del pools
        torch.cuda.empty_cache()
        floor = read_floor(pq, torch, dev, stream, [(s[0], nb[s[0]]) for s in shapes])
        tr = profile_traffic("qlow_gemv_counters.md").get(f"Q{bits}", {})
        traffic = {s_[0]: tr.get(s_[0].replace("gate_up", "gate+up")) for s_ in shapes}
        res[f"q{bits}"] = {"us_per_step": round(ms * 1e3, 2), "bytes_per_step": nbytes,
                           "traffic": {"per_shape": traffic,
                                       "per_step": sum(traffic.values()) if all(traffic.values()) else None,
                                       "source": "profiles/qlow_gemv_counters.md (HBM bytes per launch, rocprofv3 "
                                                 "FETCH_SIZE / WRITE_SIZE scaled by the calibration kernel)"},
                           "stream_read_floor": {"per_shape": floor,
                                                 "step_us": round(sum(v["us"] for v in floor.values()), 2)},
                           "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                           "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                           "period_us_sum": round(kern, 2),
                           "period_hbm_frac": round(nbytes / (kern * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                           "per_shape": per, "rotated_MB_per_shape": ROTATE_MB}
    return res


def ternary_codes(torch, N, K, dev, g):
    """Weights uniform in {-1, 0, +1}: codes {0, 1, 2} packed four per byte."""
    c = torch.randint(0, 3, (N, K // 4, 4), dtype=torch.uint8, device=dev, generator=g)
    return (c[..., 0] | (c[..., 1] << 2) | (c[..., 2] << 4) | (c[..., 3] << 6)).contiguous()


def ternary_bench(pq, torch, dev, g, stream, reps=20):
    """Config 5: PQ2_0 x Q8_K GEMVs of a Qwen3-8B-shaped FFN at T=1 (gate and up
    12288x4096, down 4096x12288), each shape from its own >= 300 MB pool."""
    shapes = [("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]
    pools = {}
    for (name, N, K) in shapes:
        pools[name] = [(ternary_codes(torch, N, K, dev, g),
                        (torch.randn((N, K // 128), device=dev, generator=g).abs() * 0.01).half().view(torch.int16))
                       for _ in range(copies_for(N * K // 4 + N * K // 128 * 2))]
    x4 = pq.q8k_quant(torch.randn(4096, device=dev, generator=g))
    x12 = pq.q8k_quant(torch.randn(12288, device=dev, generator=g))
    outs = {name: torch.empty(N, dtype=torch.float32, device=dev) for (name, N, K) in shapes}

    def launch_of(s):
        name, N, K = s

        def f(i):
            c, sc = pools[name][i % len(pools[name])]
            pq.tq2_gemv(c, sc, x12 if K == 12288 else x4, K, N, out=outs[name])
        return f

    def step(i):
        for s in shapes:
            launch_of(s)(i)

    gr = graph_of(torch, lambda: [step(i) for i in range(reps)])
    ms = timed_replay(torch, gr, stream) / reps
    del gr

    # gate and up read the same activations: one batched launch for both, as the
    # reference's engine calls them (gemvP_multi), then down
    def gate_up(i):
        a, b = pools["gate"][i % len(pools["gate"])], pools["up"][i % len(pools["up"])]
        pq.tq2_gemv_batch([a, b], x4, 4096, outs=[outs["gate"], outs["up"]])

    def step_b(i):
        gate_up(i)
        launch_of(shapes[2])(i)

    gr = graph_of(torch, lambda: [step_b(i) for i in range(reps)])
    ms_b = timed_replay(torch, gr, stream) / reps
    del gr
    gu_us = period_ms(torch, gate_up, 3 * len(pools["gate"]), stream) * 1e3
    nb = {n: N * K // 4 + N * K // 128 * 2 + K // 256 * 292 + N * 4 for (n, N, K) in shapes}
    per = _per_shape(pq, torch, stream, shapes, launch_of, lambda s: nb[s[0]])
    step_bytes = sum(nb.values())
    kern = sum(p["us"] for p in per.values())
    del pools
    torch.cuda.empty_cache()
    floor = read_floor(pq, torch, dev, stream, [(n, nb[n]) for (n, N, K) in shapes])
    tr = profile_traffic("ternary_gemv_counters.md").get("", {})
    traffic = {n: tr.get(n) for (n, N, K) in shapes}
    return {"shapes": [f"{n}:{N}x{K}" for (n, N, K) in shapes], "us_per_step": round(ms * 1e3, 2),
            "traffic": {"per_shape": traffic, "per_step": sum(traffic.values()) if all(traffic.values()) else None,
                        "batched_gate_up": tr.get("gate+up batched"),
                        "source": "profiles/ternary_gemv_counters.md (HBM bytes per launch, rocprofv3 FETCH_SIZE / "
                                  "WRITE_SIZE scaled by the calibration kernel)"},
            "stream_read_floor": {"per_shape": floor, "step_us": round(sum(v["us"] for v in floor.values()), 2)},
            "bytes_per_step": step_bytes, "GB/s": round(step_bytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "period_us_sum": round(kern, 2), "period_hbm_frac": round(step_bytes / (kern * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "per_shape": per, "rotated_MB_per_shape": ROTATE_MB,
            "batched_gate_up": {"us_per_step": round(ms_b * 1e3, 2), "gate_up_launch_us": round(gu_us, 2),
                                "GB/s": round(step_bytes / (ms_b * 1e-3) / 1e9, 1),
                                "hbm_frac": round(step_bytes / (ms_b * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}}


def gemv_profile_workload(pq, torch, dev, which, copies=3):
    """Eager launches for counter runs (rocprofv3 --pmc): each shape of the
    ternary FFN (gate, up, down, then the batched gate+up launch) or of the
    Q4 / Q5 layer GEMVs (q|k|v, o_proj, gate+up, down) `copies` times, each
    launch on its own weight copy so no launch finds its weights in a cache
    the one before filled. Prints each shape's algorithmic bytes."""
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    out = {}
    if which == "ternary":
        shapes = [("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]
        xs = {K: pq.q8k_quant(torch.randn(K, device=dev, generator=g)) for K in (4096, 12288)}
        w = {name: [(ternary_codes(torch, N, K, dev, g),
                     (torch.randn((N, K // 128), device=dev, generator=g).abs() * 0.01).half().view(torch.int16))
                    for _ in range(copies)] for (name, N, K) in shapes}
        ys = {name: torch.empty(N, dtype=torch.float32, device=dev) for (name, N, K) in shapes}
        for (name, N, K) in shapes:
            for c in range(copies):
                pq.tq2_gemv(w[name][c][0], w[name][c][1], xs[K], K, N, out=ys[name])
            torch.cuda.synchronize()
            out[name] = N * K // 4 + N * K // 128 * 2 + K // 256 * 292 + N * 4
        for c in range(copies):   # the batched gate+up launch, on copies not used above in this order
            pq.tq2_gemv_batch([w["gate"][(c + 1) % copies], w["up"][(c + 2) % copies]], xs[4096], 4096,
                              outs=[ys["gate"], ys["up"]])
        torch.cuda.synchronize()
        out["gate_up_batched"] = out["gate"] + out["up"] - 4096 // 256 * 292
    else:
        bits = 4 if which == "q4" else 5
        xs = {K: torch.randn(K, device=dev, generator=g).to(torch.bfloat16) for K in (2048, 8192)}
        for (name, N, K, _) in [s_ for s_ in SHAPES if s_[0] != "lm_head"]:
            ws = []
            for _ in range(copies):
                qc = torch.randint(0, 2 ** bits, (N, K), dtype=torch.uint8, device=dev, generator=g)
                sc = torch.randn((N, K // 32, 2), device=dev, generator=g).abs().mul(0.01).half().view(torch.int16)
                ws.append(pq.QlowWeight(qc, sc, bits))
                del qc, sc
            torch.cuda.synchronize()
            y = torch.empty(N, dtype=torch.bfloat16, device=dev)
            for c in range(copies):
                pq.qlow_gemv(ws[c], xs[K], out=y)
            torch.cuda.synchronize()
            out[name] = (pq.lib().pq_qlow_packed_codes_bytes(N, K, bits) + pq.lib().pq_qlow_packed_scales_bytes(N, K, bits)
                         + 2 * K + 2 * N)
            del ws
            torch.cuda.empty_cache()
    print(json.dumps({"gemv_profile": which, "algorithmic_bytes": out}), flush=True)


def shard_workload(pq, torch, dev, G=8, resident_mb=128):
    """The config-2 GEMVs at the shapes one of G GPUs runs when the layer is
    sharded: q|k|v, gate+up and the LM head by rows (N/G rows, then an
    all-gather of the outputs), o_proj and down by K in whole 256-wide chunks
    (K/G columns, fp32 partials gathered and added in chunk order, which keeps
    one GPU's bits). Each shape's launch period (pq_q8_gemv on x quantized
    beforehand, G = 1 beside it) over a >= 300 MB rotated pool (weights from
    HBM) and over a pool of about resident_mb (more than the L2s, less than the
    256 MB Infinity Cache: weights from the memory-side cache, as a G-GPU shard
    of the 24-layer backbone, about 225 MB at G = 8, would stay)."""
    g = torch.Generator(device=dev)
    g.manual_seed(20261201)
    stream = pq.stream_ptr()
    out = {}
    for gg in (1, G):
        shapes = [("qkv", 3072 // gg, 2048, "bf16"), ("o_proj", 2048, 2048 // gg, "f32" if gg > 1 else "bf16"),
                  ("gate_up", 16384 // gg, 2048, "bf16"), ("down", 2048, 8192 // gg, "f32" if gg > 1 else "bf16"),
                  ("lm_head", 65536 // gg, 2048, "f32")]
        res = {}
        for (name, N, K, o) in shapes:
            qx, dx = pq.q8_quant(torch.randn(K, device=dev, generator=g))
            y = torch.empty(N, dtype=torch.float32 if o == "f32" else torch.bfloat16, device=dev)
            dt = pq.DT_F32 if o == "f32" else pq.DT_BF16
            nb = N * K + N * (K // 32) * 2 + K + (K // 32) * 4 + N * (4 if o == "f32" else 2)
            row = {"shape": f"{N}x{K}", "out": o, "bytes": nb}
            for regime, mb in (("hbm", ROTATE_MB), ("infinity_cache", resident_mb)):
                pool, _ = q8_pool(pq, torch, dev, g, N, K, min_mb=mb)
                us = period_ms(torch, lambda i: pq.q8_gemv(pool[i % len(pool)], qx, dx, out_dtype=dt, out=y),
                               3 * len(pool), stream) * 1e3
                row[regime] = {"us": round(us, 2), "GB/s": round(nb / (us * 1e-6) / 1e9, 1), "copies": len(pool)}
                del pool
                torch.cuda.empty_cache()
            res[name] = row
        out[f"G{gg}"] = {"per_shape": res,
                         "step_us": {r: round(sum(v[r]["us"] for v in res.values()), 2)
                                     for r in ("hbm", "infinity_cache")}}
    print(json.dumps({"shard_profile": G, **out}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the decode and prefill measurements")
    ap.add_argument("--calib", action="store_true",
                    help="also run a plain elementwise kernel over 256 MiB (counter calibration for rocprofv3 --pmc)")
    ap.add_argument("--prefill-profile", action="store_true",
                    help="only run the prefill GEMMs (3 launches each at T=512 and T=32) for counter runs; no JSON")
    ap.add_argument("--gemv-profile", choices=["ternary", "q4", "q5"],
                    help="only run eager launches of the ternary FFN GEMVs or the Q4 / Q5 layer GEMVs (3 weight "
                         "copies per shape) for counter runs; prints their algorithmic bytes")
    ap.add_argument("--shard-profile", type=int, metavar="G",
                    help="only time the config-2 GEMVs at the shapes one of G GPUs would run (rows or whole K "
                         "chunks split G ways), from HBM and from the Infinity Cache; prints their periods")
    ap.add_argument("--decode-profile", choices=["synth", "real", "synth-ref", "real-ref", "synth-q4"],
                    help="only run one backbone's decode measurement (the synthetic or the real LFM3 shapes, "
                         "-ref: the reference's GEMV numerics, -q4: Q4 linears from a blob) for kernel traces; "
                         "prints its result")
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
    if args.shard_profile:
        if args.shard_profile not in (2, 4, 8):
            print("--shard-profile G: G of 2, 4 or 8 (o_proj's K of 2048 splits in whole 256-wide chunks)",
                  file=sys.stderr)
            sys.exit(2)
        shard_workload(pq, torch, dev, args.shard_profile)
        return
    if args.gemv_profile:
        if args.calib:   # the counter calibration of the traffic runs: 256 MiB read + 256 MiB written
            src = torch.randn(64 << 20, device=dev)
            dst = torch.empty_like(src)
            torch.neg(src, out=dst)
            torch.cuda.synchronize()
            del src, dst
        gemv_profile_workload(pq, torch, dev, args.gemv_profile)
        return
    if args.decode_profile:
        if args.calib:   # the counter calibration of the traffic runs: 256 MiB read + 256 MiB written
            src = torch.randn(64 << 20, device=dev)
            dst = torch.empty_like(src)
            torch.neg(src, out=dst)
            torch.cuda.synchronize()
            del src, dst
        from pulsar_amd.engine import LFM3_SYNTH
        if args.decode_profile == "synth-q4":
            g = torch.Generator(device=dev)
            g.manual_seed(20261201)
            print(json.dumps({"decode_profile": args.decode_profile, **decode_lowbit(pq, torch, dev, g, 4)}))
            return
        cfg = dict(LFM3_SYNTH if args.decode_profile.startswith("synth") else LFM3_REAL)
        if args.decode_profile.endswith("-ref"):
            cfg["numerics"] = 1
        print(json.dumps({"decode_profile": args.decode_profile, **decode_variant(pq, cfg)}))
        return
    torch.manual_seed(20261201)
    g = torch.Generator(device=dev)
    g.manual_seed(20261201)
    pools, per_copy = {}, {}
    for (name, N, K, _) in SHAPES:
        pools[name], per_copy[name] = q8_pool(pq, torch, dev, g, N, K)
    x2 = torch.randn(2048, device=dev, generator=g)
    x8 = torch.randn(8192, device=dev, generator=g)
    outs = {name: torch.empty(N, dtype=torch.float32 if o == "f32" else torch.bfloat16, device=dev)
            for (name, N, K, o) in SHAPES}
    torch.cuda.synchronize()
    stream = pq.stream_ptr()

    def launch_of(s):
        name, N, K, o = s
        return lambda i: pq.gemv_fused(pools[name][i % len(pools[name])], pq.PRO_F32,
                                       out_dtype=pq.DT_F32 if o == "f32" else pq.DT_BF16, out=outs[name],
                                       xf=x8 if K == 8192 else x2)

    def step(i):
        for s in SHAPES:
            launch_of(s)(i)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # the K timed steps, captured as one graph (launches as the engine issues them)
    g_steps = graph_of(torch, lambda: [step(i) for i in range(args.steps)])
    ms_per_step = timed_replay(torch, g_steps, stream) / args.steps
    del g_steps

    # each shape's back-to-back launch period (rotating pool)
    per = _per_shape(pq, torch, stream, SHAPES, launch_of, lambda s: gemv_bytes(*s[1:]), n=40)
    step_bytes = sum(gemv_bytes(N, K, o) for (_, N, K, o) in SHAPES)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    # the roofline kernel: every launch of the timed region is q8_gemv_fused_kernel,
    # so its average launch moves step_bytes / 5 in ms_per_step / 5
    launch_us = ms_per_step * 1e3 / len(SHAPES)
    achieved = (step_bytes / len(SHAPES)) / (launch_us * 1e-6) / 1e9
    gpu = gpu_desc(torch, pq)
    floor = read_floor(pq, torch, dev, stream, [(s[0], gemv_bytes(*s[1:])) for s in SHAPES])
    floor_us = sum(v["us"] for v in floor.values())

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
        "dtype": "int8",
        "dtype_detail": "int8 x int8 -> int32 block dots; fp16 weight scales, fp32 activation scales, fp32 accumulate",
        "data": "synthetic (seeded uniform int8 codes, |N(0,1)|*0.01 fp16 scales, N(0,1) fp32 x)",
        "config": {"workload": "one LFM-style layer's T=1 Q8_0 GEMVs + LM head (hidden 2048)",
                   "gpu": gpu,
                   "gemvs": [f"{n}:{N}x{K}" for (n, N, K, _) in SHAPES],
                   "bytes_per_step": step_bytes, "timed": f"{args.steps} steps in one graph, median of 5 replays",
                   "weight_copies_rotated": {n: len(p) for n, p in pools.items()},
                   "rotated_MB_per_shape": {n: round(len(pools[n]) * per_copy[n] / 1e6, 1) for n in pools}},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     # per launch like achieved: the step's measured bytes over its 5 launches
                     "traffic": (lambda t: t // len(SHAPES) if t else None)(measured_traffic()),
                     "traffic_per_step": measured_traffic(),
                     "kernel": "q8_gemv_fused_kernel: the timed region's 5 x steps launches",
                     "launches": len(SHAPES) * args.steps, "avg_launch_us": round(launch_us, 3),
                     "bytes_per_launch": step_bytes // len(SHAPES), "per_shape_period": per,
                     "lm_head_frac": round(per["lm_head"]["GB/s"] / HBM_PEAK_GBS, 4),
                     "stream_read_floor": {"per_shape": floor, "step_us": round(floor_us, 2),
                                           "GB/s": round(step_bytes / (floor_us * 1e-6) / 1e9, 1),
                                           "gemv_step_over_floor": round(floor_us / (ms_per_step * 1e3), 4),
                                           "what": "pq_stream_read over each shape's algorithmic bytes, launch "
                                                   "periods: a plain read of the same bytes in the same launches"}},
        "cpu_baseline": None,
    }
    del pools
    torch.cuda.empty_cache()
    if args.calib:
        src = torch.randn(64 << 20, device=dev)          # 256 MiB read + 256 MiB written per call
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    if not args.no_extra:
        line["config1_gemv"] = config1_bench(pq, torch, dev, g, stream)
        line["decode"] = decode_bench(pq)
        line["decode_lfm3_real_shapes"] = decode_variant(pq, LFM3_REAL)
        from pulsar_amd.engine import LFM3_SYNTH
        line["decode_ref_numerics"] = decode_variant(pq, dict(LFM3_SYNTH, numerics=1))
        line["decode_ref_numerics_real_shapes"] = decode_variant(pq, dict(LFM3_REAL, numerics=1))
        line["prefill_gemm"] = prefill_gemm_bench(pq, torch, dev, g, stream, gpu)
        line["ternary_gemv"] = ternary_bench(pq, torch, dev, g, stream)
        line["ref_numerics_gemv"] = ref_numerics_bench(pq, torch, dev, g, stream)
        line["qlow_gemv"] = qlow_bench(pq, torch, dev, g, stream)
        line["decode_q4"] = decode_lowbit(pq, torch, dev, g, 4)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_q8_gemv([(N, K) for (_, N, K, _) in SHAPES], 10.0)
        if not args.no_extra:
            from pulsar_amd.engine import LFM3_SYNTH
            line["config1_gemv"]["cpu"] = cpu_q8_gemv([(8192, 2048)], 3.0)
            line["ternary_gemv"]["cpu"] = cpu_ternary([(12288, 4096), (12288, 4096), (4096, 12288)], 4.0)
            line["decode"]["cpu"] = cpu_backbone(LFM3_SYNTH)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
