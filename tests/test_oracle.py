"""Pins the CPU oracle (test infrastructure) independently of its own formulas.

Each check is chosen so that a plausible mistake -- a dropped term, a wrong
index or sign, a transposed operand, a wrong rounding -- fails it: known-answer
vectors, the reference's own CPU routines (oracle/_ref, compiled from the
PULSAR-ASM sources), exact recomputation, library conversions and closed
forms. Runs on the CPU only.
"""
import math

import numpy as np
import pytest


def f32bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------------ scalars
def test_splitmix64_known_answer(orc):
    # splitmix64 seeded with 0: first output 0xe220a8397b1dcdaf, second 0x6e789e6aa1b965f4
    # (Steele/Lea/Flood; the values every splitmix64 implementation reproduces)
    assert orc.lib().orc_sm64_at(0, 0) == 0xE220A8397B1DCDAF
    assert orc.lib().orc_sm64_at(0, 1) == 0x6E789E6AA1B965F4


def test_h2f_all_patterns(orc):
    h = np.arange(65536, dtype=np.uint16)
    got = np.array([orc.lib().orc_h2f(int(v)) for v in h], np.float32)
    want = h.view(np.float16).astype(np.float32)
    same = (f32bits(got) == f32bits(want)) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    ref = orc.ref()
    if ref is not None:   # the reference's own pq2_h2f (pq2_host.c:9-20)
        got_ref = np.array([ref.pq2_h2f(int(v)) for v in h[::7]], np.float32)
        same = (f32bits(got_ref) == f32bits(got[::7])) | (np.isnan(got_ref) & np.isnan(got[::7]))
        assert same.all()


def test_f2h_matches_ieee_casts(orc):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(30000) * 10.0 ** rng.integers(-9, 6, 30000)).astype(np.float32)
    edges = np.array([65504, 65519.996, 65520, 65536, 2 ** -24, 2 ** -25, 1.5 * 2 ** -25, 2 ** -14,
                      6.1e-5, 5.9604645e-08, -0.0, 0.0, np.inf, -np.inf, 1.0009765625, 1.00048828125], np.float32)
    x = np.concatenate([x, edges, -edges])
    got = np.array([orc.lib().orc_f2h(float(v)) for v in x], np.uint16)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f2h_matches_reference_quantizer(orc):
    """quant_row (q8_gemv_cpu.c:63-81) stores (float)(_Float16)(max/127): the
    reference compiler's own f32->f16 conversion."""
    ref = orc.ref()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    import ctypes as C
    rng = np.random.default_rng(5)
    w = (rng.standard_normal(32 * 500) * 10.0 ** rng.integers(-6, 3, 32 * 500).repeat(1)).astype(np.float32)
    q = np.empty(w.size, np.int8)
    s = np.empty(w.size // 32, np.float32)
    ref.ref_q8_quant(w.ctypes.data_as(C.c_void_p), C.c_int(w.size), q.ctypes.data_as(C.c_void_p),
                     s.ctypes.data_as(C.c_void_p))
    amax = np.abs(w.reshape(-1, 32)).max(1).astype(np.float32)
    mine = np.array([orc.lib().orc_h2f(orc.lib().orc_f2h(float(np.float32(a) / np.float32(127.0)))) for a in amax],
                    np.float32)
    assert np.array_equal(f32bits(mine), f32bits(s))


def test_f2bf_rne(orc):
    import torch
    f = orc.lib().orc_f2bf
    # closed forms: exact, tie to even (down and up), carry into the exponent, inf/nan passthrough
    assert f(1.0) == 0x3F80
    assert f(float(np.uint32(0x3F808000).view(np.float32))) == 0x3F80      # tie, even stays
    assert f(float(np.uint32(0x3F818000).view(np.float32))) == 0x3F82      # tie, odd rounds up
    assert f(float(np.uint32(0x3F808001).view(np.float32))) == 0x3F81
    assert f(float(np.uint32(0x3FFFFFFF).view(np.float32))) == 0x4000      # carry
    assert f(float("inf")) == 0x7F80 and f(float("-inf")) == 0xFF80
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(20000) * 10.0 ** rng.integers(-30, 30, 20000)).astype(np.float32)
    got = orc.f2bf(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_expf_accuracy(orc):
    x = np.concatenate([np.linspace(-103.9, 88.72, 150001), np.linspace(-1, 1, 20001)]).astype(np.float32)
    got = orc.expf(x).astype(np.float64)
    true = np.exp(x.astype(np.float64))
    ulp = np.spacing(true.astype(np.float32)).astype(np.float64)
    assert (np.abs(got - true) / ulp).max() <= 2.0
    assert orc.lib().orc_expf(0.0) == 1.0
    assert orc.lib().orc_expf(89.0) == math.inf and orc.lib().orc_expf(-200.0) == 0.0
    assert math.isnan(orc.lib().orc_expf(float("nan")))


def test_pairwise_is_butterfly(orc):
    rng = np.random.default_rng(11)
    for n in (1, 2, 64, 2048):
        v = rng.standard_normal(n).astype(np.float32) * 1e3
        b = v.copy()
        while b.size > 1:
            b = (b[0::2] + b[1::2]).astype(np.float32)
        got = orc.lib().orc_pairwise(v.ctypes.data_as(__import__("ctypes").c_void_p), n)
        assert np.float32(got) == b[0]


# --------------------------------------------------------------- generators
def test_generators(orc):
    c = orc.gen_codes(1, 400000)
    assert c.min() == -127 and c.max() == 127 and abs(c.mean()) < 0.5
    z = orc.gen_normal(2, 400000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    s = orc.gen_scales(3, 100000)
    sv = s.view(np.float16).astype(np.float32)
    assert (sv >= 0).all() and abs(sv.mean() - 0.01 * math.sqrt(2 / math.pi)) < 2e-4
    t = orc.gen_ternary(4, 100000)
    codes = np.stack([(t >> (2 * k)) & 3 for k in range(4)])
    assert codes.max() == 2 and abs(codes.mean() - 1.0) < 0.01
    # counter-based: a prefix of a longer stream is the shorter stream
    assert np.array_equal(orc.gen_codes(9, 1000), orc.gen_codes(9, 5000)[:1000])


# --------------------------------------------------------------- quantizers
def test_q8_quant_properties(orc):
    rng = np.random.default_rng(13)
    x = (rng.standard_normal(64 * 32) * 10.0 ** rng.integers(-3, 3, 64 * 32)).astype(np.float32)
    x[:32] = 0.0
    qx, dx = orc.q8_quant(x)
    xb, qb = x.reshape(-1, 32), qx.reshape(-1, 32).astype(np.int32)
    assert dx[0] == 0 and not qb[0].any()
    amax = np.abs(xb).max(1)
    assert np.array_equal(f32bits(dx), f32bits((amax / np.float32(127)).astype(np.float32)))
    assert np.abs(qb).max() <= 127
    i = np.abs(xb[1:]).argmax(1)
    assert (np.abs(qb[1:][np.arange(63), i]) == 127).all()
    err = np.abs(qb[1:] * dx[1:, None].astype(np.float64) - xb[1:])
    assert (err <= dx[1:, None] * 0.5000001 + 1e-30).all()


def test_q8k_quant_properties(orc):
    rng = np.random.default_rng(17)
    x = rng.standard_normal(4 * 256).astype(np.float32)
    x[256:512] = 0.0
    out = orc.q8k_quant(x)
    for b in range(4):
        blk = out[b * 292:(b + 1) * 292]
        d = blk[:4].view(np.float32)[0]
        qs = blk[4:260].view(np.int8).astype(np.int32)
        bs = blk[260:292].view(np.int16)
        xb = x[b * 256:(b + 1) * 256]
        if b == 1:
            assert d == 0 and not qs.any()
            continue
        j = int(np.argmax(np.abs(xb)))
        assert qs[j] == -127                            # iscale = -127/max maps max to -127
        assert np.array_equal(bs, qs.reshape(16, 16).sum(1))
        assert np.abs(qs * np.float64(d) - xb).max() <= abs(d) * 0.5000001


def test_q8k_quant_is_reference_code(orc):
    """orc_q8k_quant's d and qs equal the reference's own Q8_K block rule run on
    each 256-block: bq1_quant_row_i8 (bq1_cpu.c:40-54, oracle/_ref), which the
    reference states is fwd8.c's q8_K_quant rule (fwd8.c:72-137: first index
    reaching |x|max, iscale = -127/max, the 1.5*2^23 round, min(127, .),
    d = 1/iscale; an all-zero block gives d = 0 and qs = 0). bsums are the
    exact sums of 16 qs (fwd8.c leaves an all-zero block's bsums stale; the
    oracle writes zeros there)."""
    ref = orc.ref()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    import ctypes as C
    ref.bq1_quant_row_i8.restype = C.c_float
    ref.bq1_quant_row_i8.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    rng = np.random.default_rng(29)
    nb = 64
    x = (rng.standard_normal(nb * 256) * rng.choice([1e-30, 1e-3, 1.0, 40.0, 3e4], nb * 256)).astype(np.float32)
    x[256:512] = 0.0                                    # all-zero block
    x[512:768] = np.clip(x[512:768], -4.0, 4.0)         # ties for |x|max: the first index (-9) wins
    x[512 + 7] = -9.0
    x[512 + 100] = x[512 + 200] = 9.0
    x[768:1024] = np.float32(0.5) * rng.integers(-300, 300, 256).astype(np.float32)   # exact halves: ties to even
    x[1024:1280] = 0.0
    x[1024 + 255] = -1e-41                              # a lone subnormal
    out = orc.q8k_quant(x)
    for b in range(nb):
        xb = np.ascontiguousarray(x[b * 256:(b + 1) * 256])
        qr = np.empty(256, np.int8)
        dr = ref.bq1_quant_row_i8(xb.ctypes.data_as(C.c_void_p), qr.ctypes.data_as(C.c_void_p), 256)
        blk = out[b * 292:(b + 1) * 292]
        assert blk[:4].view(np.uint32)[0] == np.float32(dr).view(np.uint32), b
        assert np.array_equal(blk[4:260].view(np.int8), qr), b
        assert np.array_equal(blk[260:292].view(np.int16), qr.astype(np.int32).reshape(16, 16).sum(1)), b


# ------------------------------------------------------------------- GEMVs
def _q8_case(orc, seed, N, K):
    W, S = orc.q8_weights(seed, N, K)
    x = orc.gen_normal(seed + 2, K)
    qx, dx = orc.q8_quant(x)
    return W, S, qx, dx


def test_r1_gemv_vs_exact(orc):
    for N, K in [(97, 2048), (33, 8192), (5, 96), (3, 288)]:
        W, S, qx, dx = _q8_case(orc, 100 + K, N, K)
        y = orc.q8_gemv(W, S, qx, dx)
        ye = orc.q8_gemv_exact(W, S, qx, dx)
        isum = (W.reshape(N, -1, 32).astype(np.int64) * qx.reshape(-1, 32)).sum(-1)
        den = (np.abs(isum) * S.view(np.float16).astype(np.float64) * dx).sum(-1)
        assert (np.abs(y - ye) / den).max() <= 1e-5


def test_r1_gemv_closed_forms(orc):
    """One block: y = fl(fl(dw*dx) * isum). Two 8-block chunks: y = fl(a0 + a1)."""
    W, S, qx, dx = _q8_case(orc, 7, 4, 32)
    y = orc.q8_gemv(W, S, qx, dx)
    isum = (W.astype(np.int64) * qx).sum(1)
    s = (S[:, 0].view(np.float16).astype(np.float32) * dx[0]).astype(np.float32)
    assert np.array_equal(f32bits(y), f32bits((s * isum.astype(np.float32)).astype(np.float32)))
    # a one-block-per-chunk layout: blocks 0 and 8 nonzero, the rest zero
    W, S, qx, dx = _q8_case(orc, 8, 4, 512)
    W = W.copy()
    keep = np.zeros(16, bool)
    keep[[0, 8]] = True
    W.reshape(4, 16, 32)[:, ~keep] = 0
    y = orc.q8_gemv(W, S, qx, dx)
    parts = []
    for b in (0, 8):
        isum = (W[:, 32 * b:32 * b + 32].astype(np.int64) * qx[32 * b:32 * b + 32]).sum(1).astype(np.float32)
        s = (S[:, b].view(np.float16).astype(np.float32) * dx[b]).astype(np.float32)
        parts.append((s * isum).astype(np.float32))
    assert np.array_equal(f32bits(y), f32bits((parts[0] + parts[1]).astype(np.float32)))


def test_a11_is_reference_code(orc):
    """orc_q8_gemv_a11 restates gemv_q8 (q8_gemv_cpu.c:29-58): bit-equal to it."""
    ref = orc.ref()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    import ctypes as C
    for N, K in [(97, 2048), (64, 7680), (13, 64)]:
        W, S, qx, dx = _q8_case(orc, 200 + K, N, K)
        S32 = S.view(np.float16).astype(np.float32)
        x = (qx.astype(np.float32).reshape(-1, 32) * dx[:, None]).reshape(-1).astype(np.float32)
        ya = orc.q8_gemv_a11(W, S32, x)
        yr = np.empty(N, np.float32)
        ref.ref_q8_gemv(W.ctypes.data_as(C.c_void_p), S32.ctypes.data_as(C.c_void_p),
                        x.ctypes.data_as(C.c_void_p), yr.ctypes.data_as(C.c_void_p), C.c_int(N), C.c_int(K))
        assert np.array_equal(f32bits(ya), f32bits(yr))
        # and R1 agrees with the reference's own order within 1e-5 of sum |terms|
        y = orc.q8_gemv(W, S, qx, dx)
        isum = (W.reshape(N, -1, 32).astype(np.int64) * qx.reshape(-1, 32)).sum(-1)
        den = (np.abs(isum) * S32.astype(np.float64) * dx).sum(-1)
        assert (np.abs(y.astype(np.float64) - yr) / den).max() <= 1e-5


def test_gemm_is_per_position_gemv(orc):
    W, S = orc.q8_weights(31, 70, 288)
    x = orc.gen_normal(32, 5 * 288).reshape(5, 288)
    qx, dx = orc.q8_quant(x)
    Y = orc.q8_gemm(W, S, qx, dx)
    for t in range(5):
        assert np.array_equal(f32bits(Y[t]), f32bits(orc.q8_gemv(W, S, qx[t], dx[t])))


@pytest.mark.parametrize("N,K", [(37, 9728), (61, 2560), (8, 4096), (3, 256)])
def test_tq2_is_reference_code(orc, N, K):
    """orc_tq2_gemv restates pq2_gemv_cpu (pq2_host.c:82-104): bit-equal to it
    (the shapes are the reference's pq1t_parity.c row widths, fewer rows)."""
    ref = orc.ref()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    import ctypes as C
    codes = orc.gen_ternary(K + N, N * K // 4)
    S = orc.gen_scales(K + N + 1, N * K // 128)
    xq = orc.q8k_quant(orc.gen_normal(K + N + 2, K))
    y = orc.tq2_gemv(codes, S, xq, N, K)
    yr = np.empty(N, np.float32)
    ref.pq2_gemv_cpu(C.c_int(N), C.c_int(K), codes.ctypes.data_as(C.c_void_p), S.ctypes.data_as(C.c_void_p),
                     xq.ctypes.data_as(C.c_void_p), yr.ctypes.data_as(C.c_void_p))
    assert np.array_equal(f32bits(y), f32bits(yr))
    # the row-sliced OpenMP wrapper the CPU baseline times gives the same rows
    ys = np.full(N, np.nan, np.float32)
    ref.ref_pq2_gemv_rows(C.c_int(N), C.c_int(K), codes.ctypes.data_as(C.c_void_p), S.ctypes.data_as(C.c_void_p),
                          xq.ctypes.data_as(C.c_void_p), ys.ctypes.data_as(C.c_void_p))
    assert np.array_equal(f32bits(ys), f32bits(yr))


def test_tq2_exact_int(orc):
    """The ternary int32 group dots, recomputed in int64 with the code-1 mapping."""
    N, K = 5, 512
    codes = orc.gen_ternary(41, N * K // 4)
    S = np.full(N * K // 128, 0x3C00, np.uint16)       # scale 1.0
    x = orc.gen_normal(42, K)
    xq = orc.q8k_quant(x)
    y = orc.tq2_gemv(codes, S, xq, N, K)
    vals = np.stack([(codes >> (2 * k)) & 3 for k in range(4)], 1).reshape(N, K).astype(np.int64) - 1
    qs = np.concatenate([xq[b * 292 + 4:b * 292 + 260].view(np.int8) for b in range(K // 256)]).astype(np.int64)
    d = np.array([xq[b * 292:b * 292 + 4].view(np.float32)[0] for b in range(K // 256)], np.float64)
    want = (vals.reshape(N, -1, 256) * qs.reshape(-1, 256)).sum(-1) @ d
    assert np.allclose(y, want, rtol=1e-6, atol=1e-6)


# -------------------------------------------------------- layer primitives
def test_rmsnorm_vs_double(orc):
    rng = np.random.default_rng(19)
    x = orc.f2bf(rng.standard_normal(2048).astype(np.float32) * 3)
    w = (1 + 0.1 * rng.standard_normal(2048)).astype(np.float32)
    y = orc.bf2f(orc.rmsnorm(x, w))
    xf = orc.bf2f(x).astype(np.float64)
    want = w * (xf / np.sqrt((xf ** 2).mean() + 1e-5))
    assert np.abs(y - want).max() <= np.abs(want).max() * 2 ** -7


def test_attention_vs_two_pass(orc):
    nh, nkv, hd = 8, 2, 64
    for npos in (1, 5, 64, 65, 300):
        q = orc.f2bf(orc.gen_normal(50 + npos, nh * hd))
        Kc = orc.gen_normal(51 + npos, npos * nkv * hd).astype(np.float16).view(np.uint16)
        Vc = orc.gen_normal(52 + npos, npos * nkv * hd).astype(np.float16).view(np.uint16)
        a = orc.bf2f(orc.attn(q, Kc, Vc, npos, nh, nkv, hd, 0.125))
        b = orc.attn_twopass(q, Kc, Vc, npos, nh, nkv, hd, 0.125)
        assert np.abs(a - b).max() <= np.abs(b).max() * 2 ** -7
        if npos == 1:   # one key: the output is v_0 of the head's kv group, rounded to bf16
            v0 = Vc.view(np.float16).astype(np.float32).reshape(nkv, hd)
            want = orc.f2bf(np.repeat(v0, nh // nkv, axis=0).reshape(-1))
            assert np.array_equal(orc.attn(q, Kc, Vc, 1, nh, nkv, hd, 0.125), want)


def _twopass_bf16cache(q, Kc, Vc, npos, nh, nkv, hd, scale, win=0):
    """Softmax attention in double over a bf16 cache (keys lo..npos-1)."""
    lo = npos - win if win > 0 and npos > win else 0
    qf = orc_bf2f_np(q).astype(np.float64).reshape(nh, hd)
    K = orc_bf2f_np(Kc).astype(np.float64).reshape(npos, nkv, hd)[lo:]
    V = orc_bf2f_np(Vc).astype(np.float64).reshape(npos, nkv, hd)[lo:]
    out = np.empty((nh, hd))
    for h in range(nh):
        g = h // (nh // nkv)
        s = K[:, g] @ qf[h] * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ V[:, g]
    return out.reshape(-1)


def _sim_attn_ref(orc, q, Kc, Vc, npos, nh, nkv, hd, scale, win=0):
    """k_attn_head (lfm3_nanode.cu:503-602) vectorised over keys: lane chains
    [key][32 lanes], the shfl_down trees, thread sums [256 threads], warp
    trees, the segment chains [8 segments] added pairwise."""
    lo = npos - win if win > 0 and npos > win else 0
    np_ = npos - lo
    e = hd // 32
    qf = orc_bf2f_np(q).reshape(nh, 32, e)
    K = orc_bf2f_np(Kc).reshape(npos, nkv, 32, e)[lo:]
    V = orc_bf2f_np(Vc).reshape(npos, nkv, hd)[lo:]
    out = np.empty((nh, hd), np.uint16)
    for h in range(nh):
        g = h // (nh // nkv)
        chain = np.zeros((np_, 32), np.float32)
        for j in range(e):
            chain = chain + qf[h, :, j] * K[:, g, :, j]
        sc = _sim_tree(chain) * np.float32(scale)
        m = np.float32(max(np.float32(-1e30), sc.max()))
        ex = orc.expf(sc - m)
        th = np.zeros(256, np.float32)
        for i0 in range(0, np_, 256):
            blk = ex[i0:i0 + 256]
            th[:blk.size] = th[:blk.size] + blk
        w = _sim_tree(th.reshape(8, 32))
        tot = ((w[0] + w[4]) + (w[2] + w[6])) + ((w[1] + w[5]) + (w[3] + w[7]))
        wt = ex * (np.float32(1) / tot)
        sg = np.zeros((8, hd), np.float32)
        for i in range(np_):
            sg[i % 8] = sg[i % 8] + wt[i] * V[i, g]
        o = ((sg[0] + sg[1]) + (sg[2] + sg[3])) + ((sg[4] + sg[5]) + (sg[6] + sg[7]))
        out[h] = orc.f2bf(o)
    return out.reshape(-1)


def test_attention_reference_order(orc):
    """orc_attn_ref, k_attn_head's order over a bf16 cache: one key gives its
    value row exactly; the 8 value segments add pairwise (16 keys of equal
    score, so every weight is 2^-4: segment 0 holds 1 + 2^-8, the seven others
    2^-24 each; pairwise they sum to 1 + 2^-8 + 3 * 2^-23, above the bf16
    midpoint, 0x3f81, where a sequential sum stays at the midpoint and rounds
    to 0x3f80); against a double-precision softmax within bf16 rounding; and
    against a vectorised transcription of the kernel, bit for bit."""
    bf = lambda a: orc.f2bf(np.asarray(a, np.float32))
    nh, nkv = 4, 2
    for hd in (64, 128):
        q = bf(orc.gen_normal(90 + hd, nh * hd))
        Kc = bf(orc.gen_normal(91 + hd, nkv * hd))
        Vc = bf(orc.gen_normal(92 + hd, nkv * hd) * 3)
        want = np.repeat(Vc.reshape(nkv, hd), nh // nkv, axis=0).reshape(-1)
        assert np.array_equal(orc.attn_ref(q, Kc, Vc, 1, nh, nkv, hd, 0.125), want)
        v = np.zeros((16, nkv, hd), np.float32)
        v[0], v[8], v[1:8] = 16.0, 2.0 ** -4, 2.0 ** -20
        out = orc.attn_ref(bf(np.zeros(nh * hd)), bf(np.ones(16 * nkv * hd)), bf(v), 16, nh, nkv, hd, 0.125)
        assert (out == 0x3F81).all()
    for hd, npos, win in ((64, 300, 0), (128, 600, 0), (128, 300, 100), (64, 700, 256), (128, 5, 0)):
        q = bf(orc.gen_normal(93 + npos, nh * hd))
        Kc = bf(orc.gen_normal(94 + npos, npos * nkv * hd))
        Vc = bf(orc.gen_normal(95 + npos, npos * nkv * hd))
        a = orc.attn_ref(q, Kc, Vc, npos, nh, nkv, hd, 0.125, win)
        b = _twopass_bf16cache(q, Kc, Vc, npos, nh, nkv, hd, 0.125, win)
        assert np.abs(orc.bf2f(a) - b).max() <= np.abs(b).max() * 2 ** -7, (hd, npos, win)
        assert np.array_equal(a, _sim_attn_ref(orc, q, Kc, Vc, npos, nh, nkv, hd, 0.125, win)), (hd, npos, win)


@pytest.mark.parametrize("hd", [64, 128])
def test_attention_window(orc, hd):
    """Sliding-window layers (k_attn_head's lo = npos - win when npos > win,
    lfm3_nanode.cu:515): against the double-precision two-pass softmax over the
    same keys [lo, npos); win = 1 gives the newest value row itself; a window
    at least npos wide is the full attention, bit for bit; a key outside the
    window cannot move the output."""
    nh, nkv = 8, 2
    for npos, win in ((300, 256), (300, 100), (70, 64), (65, 1), (200, 17), (5, 256)):
        q = orc.f2bf(orc.gen_normal(80 + npos + win, nh * hd))
        Kc = orc.gen_normal(81 + npos, npos * nkv * hd).astype(np.float16).view(np.uint16)
        Vc = orc.gen_normal(82 + npos, npos * nkv * hd).astype(np.float16).view(np.uint16)
        a = orc.attn(q, Kc, Vc, npos, nh, nkv, hd, 0.125, win)
        b = orc.attn_twopass(q, Kc, Vc, npos, nh, nkv, hd, 0.125, win)
        assert np.abs(orc.bf2f(a) - b).max() <= np.abs(b).max() * 2 ** -7, (npos, win)
        if win >= npos:
            assert np.array_equal(a, orc.attn(q, Kc, Vc, npos, nh, nkv, hd, 0.125))
        else:
            assert not np.allclose(orc.bf2f(a), orc.attn_twopass(q, Kc, Vc, npos, nh, nkv, hd, 0.125), atol=1e-3)
            lo = npos - win
            K2, V2 = Kc.copy(), Vc.copy()
            K2.reshape(npos, -1)[lo - 1] ^= 0x0400        # perturb the key and value just outside
            V2.reshape(npos, -1)[lo - 1] ^= 0x0400
            assert np.array_equal(a, orc.attn(q, K2, V2, npos, nh, nkv, hd, 0.125, win))
        if win == 1:
            vlast = Vc.view(np.float16).astype(np.float32).reshape(npos, nkv, hd)[-1]
            assert np.array_equal(a, orc.f2bf(np.repeat(vlast, nh // nkv, axis=0).reshape(-1)))


def test_conv_impulse_response(orc):
    H, nt = 64, 3
    taps = orc.gen_normal(60, H * nt)
    one = orc.f2bf(np.ones(H, np.float32))
    zero = np.zeros(H, np.uint16)
    ring = np.zeros(nt * H, np.uint16)
    outs = []
    for step in range(nt + 1):
        x = one if step == 0 else zero
        bcx = np.concatenate([one, one, x])        # B = 1, C = 1, x = impulse
        o, ring = orc.conv_step(ring, taps, bcx, H, nt)
        outs.append(o)
    for k in range(nt):   # step k sees the impulse in ring slot nt-1-k
        assert np.array_equal(outs[k], orc.f2bf(taps.reshape(H, nt)[:, nt - 1 - k]))
    assert not outs[nt].any()


@pytest.mark.parametrize("nt", [3, 7])
def test_conv_step_closed_forms(orc, nt):
    """orc_conv_step follows k_conv7 / k_conv_chunk (lfm3_nanode.cu:901-941): the
    taps summed in ascending order with each product rounded before its add,
    bx = bf16(B*x) shifted in as the newest slot, cy = bf16(acc) before C
    multiplies it. Channels built by hand (tests/conv_cases.py) separate each of
    a descending sum, an fma chain, an unrounded B*x and an unrounded cy from the
    reference's order: each departure changes its own channels' outputs."""
    import conv_cases as cc
    H = 64
    rb, taps, bcx, kinds = cc.build(H, nt)
    want_out, want_ring = cc.expected(H, nt)
    dep = cc.departures(H, nt)
    assert np.array_equal(dep["reference"], want_out)
    for name, kind in (("descending", cc.ORDER), ("fused", cc.FUSED), ("bx unrounded", cc.BX),
                       ("cy unrounded", cc.CY)):
        differs = dep[name] != want_out
        assert differs[kinds == kind].all() and not differs[kinds != kind].any(), name
    out, ring = orc.conv_step(rb.reshape(-1), taps.reshape(-1), bcx, H, nt)
    assert np.array_equal(out, want_out)
    assert np.array_equal(ring.reshape(nt, H), want_ring)


def test_q8_quant_ties_are_reference_code(orc):
    """Where amax/127 is an fp16 value, the reference's quant_row
    (q8_gemv_cpu.c:63-81: sc16 = (float)(_Float16)(amax/127), q = lrintf(x/sc16),
    clamp +-127) and orc_q8_quant (d = amax/127 in fp32, q = rne(x/d)) divide by
    the same d, so their codes must agree bit for bit. Blocks with amax = 127*m*2^k
    (m an fp16 significand) full of exact halves n*d + d/2 pin the ties to even:
    ties away from zero or truncation fail them."""
    import ctypes as C
    import quant_cases as qc
    ref = orc.ref()
    x = qc.tie_blocks()
    q, dx = orc.q8_quant(x)
    xb = x.reshape(-1, 32).astype(np.float64)
    dd = np.repeat(dx.astype(np.float64), 32).reshape(-1, 32)
    assert (xb / dd * 2 % 2 == 1).sum() >= 4 * len(qc.SCALES)     # the ties are really there
    want = qc.rne_codes(x)
    assert np.array_equal(q, want)
    assert (qc.away_codes(x) != want).any()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    qr = np.empty(x.size, np.int8)
    sr = np.empty(x.size // 32, np.float32)
    ref.ref_q8_quant(x.ctypes.data_as(C.c_void_p), C.c_int(x.size), qr.ctypes.data_as(C.c_void_p),
                     sr.ctypes.data_as(C.c_void_p))
    assert np.array_equal(f32bits(sr), f32bits(dx))
    assert np.array_equal(qr, q)


def test_silu_and_gate(orc):
    rng = np.random.default_rng(23)
    a = orc.f2bf(rng.standard_normal(4096).astype(np.float32) * 8)
    b = orc.f2bf(rng.standard_normal(4096).astype(np.float32))
    y = orc.bf2f(orc.silu_mul(a, b))
    af, bf = orc.bf2f(a).astype(np.float64), orc.bf2f(b).astype(np.float64)
    want = af / (1 + np.exp(-af)) * bf
    assert (np.abs(y - want) <= np.abs(want) * 2 ** -7 + 1e-30).all()
    g = orc.f2bf(np.array([0.0, 100.0, -100.0, 1.5], np.float32))
    at = orc.f2bf(np.ones(4 * 8, np.float32))
    out = orc.bf2f(orc.sigmoid_gate(g, at, 4, 8)).reshape(4, 8)
    assert (out[0] == 0.5).all() and (out[1] == 1.0).all() and (out[2] == 0.0).all()


def _argmax_by_key(v):
    """k_argmax's pick written as a key (lfm3_nanode.cu:942-964): among the
    values above -1e30 the largest; on ties the last tree step weighs most, so
    thread slot s = i mod 256 (warp w = s // 32, lane l = s % 32) ranks by
    (bitrev3(w), bitrev5(l)), then i; -1 when none."""
    v = np.asarray(v, np.float32)
    ok = v > np.float32(-1e30)
    if not ok.any():
        return -1
    m = v[ok].max()
    idx = np.flatnonzero(ok & (v == m))
    s = idx & 255
    br = lambda x, b: int(format(int(x), f"0{b}b")[::-1], 2)
    keys = [(br(si >> 5, 3), br(si & 31, 5), int(i)) for si, i in zip(s, idx)]
    return int(idx[min(range(len(idx)), key=lambda k: keys[k])])


def test_argmax_reference_order(orc):
    """k_argmax's tie order, hand-derived from its trees: a later (smaller)
    shfl_down offset outranks an earlier one, so among equal maxima lane 2
    beats lane 1 (offset 2 joins lane 0 to lane 2 before offset 1 meets lane
    1), thread 0's index 256 beats thread 1's index 1, warp 2 beats warp 1
    (64 over 32), and warp 0 beats warp 1 (1 over 32). No value above -1e30
    gives -1; NaN never wins."""
    def at(n, idx, val=3.0, fill=1.0):
        v = np.full(n, fill, np.float32)
        v[idx] = val
        return v
    assert orc.argmax(at(5, [1, 2])) == 2
    assert orc.argmax(at(300, [1, 256])) == 256
    assert orc.argmax(at(100, [32, 64])) == 64
    assert orc.argmax(at(100, [1, 32])) == 1
    assert orc.argmax(at(100, [0, 32])) == 0
    assert orc.argmax(at(1000, [300, 44])) == 44          # one slot: the lower index
    # ties at 1, 3, 4: offset 4 moves lane 4's pair into lane 0, offset 1 keeps it
    assert orc.argmax(np.array([1.0, 3.0, -2.0, 3.0, 3.0], np.float32)) == 4
    assert orc.argmax(np.full(7, -1e30, np.float32)) == -1
    assert orc.argmax(np.full(7, -np.inf, np.float32)) == -1
    assert orc.argmax(np.array([np.nan, 2.0, np.nan], np.float32)) == 1
    assert orc.argmax(np.array([-1e30, -2e30, -9e29], np.float32)) == 2
    rng = np.random.default_rng(41)
    for n in (1, 7, 255, 256, 300, 1000, 4096, 65536):
        for _ in range(8):
            v = rng.integers(0, 4, n).astype(np.float32)
            assert orc.argmax(v) == _argmax_by_key(v), n


def _bf16_rne_exact(v):
    """bf16 bits of the exact rational v rounded to nearest even (normal range)."""
    from fractions import Fraction
    v = Fraction(v)
    if v == 0:
        return 0
    sign, a = (0x8000, -v) if v < 0 else (0, v)
    e = 0
    while a >= 2:
        a /= 2
        e += 1
    while a < 1:
        a *= 2
        e -= 1
    q = a * 128                      # 8 significant bits: q in [128, 256)
    n = q.numerator // q.denominator
    r = q - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    val = Fraction(n, 128) * Fraction(2) ** e
    return sign | int(np.float32(float(val)).view(np.uint32) >> 16)


def test_rmsnorm_rounds_before_weight(orc):
    """k_rmsnorm (lfm3_nanode.cu:433-436) rounds x*rs to bf16 and only then
    multiplies by the weight. x = 1 everywhere gives rs = 1/sqrt(1 + eps) and
    bf16(x*rs) = 1, so the two-round form is bf16(w); with w = 1 + 2^-8 + 2^-20,
    just above the bf16 midpoint between 1 and 1 + 2^-7, that is 1 + 2^-7
    (0x3f81), while one rounding of w*rs (below the midpoint) gives 1 (0x3f80)."""
    n = 2048
    x = np.full(n, 0x3F80, np.uint16)
    w = np.full(n, 1 + 2.0 ** -8 + 2.0 ** -20, np.float32)
    assert np.all(orc.rmsnorm(x, w, 1e-5) == 0x3F81)
    rs = np.float32(1) / np.sqrt(np.float32(1) + np.float32(1e-5))
    assert orc.f2bf(np.float32(w[0]) * rs) == 0x3F80          # the one-round form differs
    # eps = 0: rs = 1 exactly, so both forms give bf16(w)
    assert np.all(orc.rmsnorm(x, w, 0.0) == 0x3F81)


def _f32(v):
    return np.float32(v)


def _sim_tree(s):
    """The shfl_down tree over the last axis (32 lanes): lane l < o adds lane
    l + o, o = 16 .. 1; lane 0's value."""
    s = s.astype(np.float32).copy()
    for o in (16, 8, 4, 2, 1):
        s[..., :o] = s[..., :o] + s[..., o:2 * o]
    return s[..., 0]


def _sim_rms_sumsq(xb):
    """rmsnorm_body's sum (lfm3_nanode.cu:393-405) vectorised: [warp][thread][8]."""
    x = orc_bf2f_np(xb)
    q = (x * x).reshape(-1, 32, 8)
    t = ((q[..., 0] + q[..., 1]) + (q[..., 2] + q[..., 3])) + ((q[..., 4] + q[..., 5]) + (q[..., 6] + q[..., 7]))
    p = _sim_tree(t)
    tot = p[0]
    for w in range(1, p.size):
        tot = _f32(tot + p[w])
    return tot


def _sim_head_sumsq(xb):
    x = orc_bf2f_np(xb)
    q = (x * x).reshape(32, -1)
    t = (q[:, 0] + q[:, 1]) + (q[:, 2] + q[:, 3]) if q.shape[1] == 4 else q[:, 0] + q[:, 1]
    return _sim_tree(t)


def orc_bf2f_np(xb):
    return (np.asarray(xb, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _bits(n, vals):
    """bf16 bits of a vector of n zeros with vals {index: value} set."""
    x = np.zeros(n, np.float32)
    for i, v in vals.items():
        x[i] = v
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def test_rms_sumsq_reference_order(orc):
    """rmsnorm_body's sum of squares, hand-derived cases where its order gives
    another value than an adjacent pairwise tree or a sequential sum (4096^2 =
    2^24 absorbs a lone 1): within a thread, pairwise (squares 2^24, 0, 1, 1:
    2^24 + 2; sequential 2^24); thread 1 meets thread 17 before thread 0
    (squares 2^24 at thread 0, 1 at threads 1 and 17: 2^24 + 2; an adjacent tree
    2^24); the warp partials in order (2^24, 0, 1, 1: 2^24; pairwise 2^24 + 2).
    Then random rows against the vectorised transcription."""
    assert orc.rms_sumsq(_bits(256, {0: 4096.0, 2: 1.0, 3: 1.0})) == 2.0 ** 24 + 2
    assert orc.rms_sumsq(_bits(256, {0: 4096.0, 8: 1.0, 136: 1.0})) == 2.0 ** 24 + 2
    assert orc.rms_sumsq(_bits(1024, {0: 4096.0, 512: 1.0, 768: 1.0})) == 2.0 ** 24
    rng = np.random.default_rng(43)
    for n in (256, 2048, 8192):
        for _ in range(4):
            xb = orc.f2bf((rng.standard_normal(n) * np.exp(2 * rng.standard_normal(n))).astype(np.float32))
            assert orc.rms_sumsq(xb) == _sim_rms_sumsq(xb), n


def test_headnorm_reference_order(orc):
    """k_headnorm (lfm3_nanode.cu:460-479): its sum of squares (32 threads of
    4 at hd = 128: squares 2^24 at thread 0 and 1 at threads 1 and 17 give
    2^24 + 2, an adjacent tree 2^24; hd = 64 in threads of 2), then RMSNorm's
    rounding steps per head with the shared [hd] weight."""
    assert orc.head_sumsq(_bits(128, {0: 4096.0, 4: 1.0, 68: 1.0})) == 2.0 ** 24 + 2
    assert orc.head_sumsq(_bits(64, {0: 4096.0, 2: 1.0, 34: 1.0})) == 2.0 ** 24 + 2
    for nh, hd in ((4, 64), (3, 128)):
        x = orc.f2bf(orc.gen_normal(70 + hd, nh * hd) * 2)
        w = orc.gen_affine(71 + hd, hd, 1.0, 0.1)
        got = orc.headnorm(x, w, nh, hd)
        for h in range(nh):
            xh = x[h * hd:(h + 1) * hd]
            ss = orc.head_sumsq(xh)
            assert ss == _sim_head_sumsq(xh)
            rs = _f32(1) / np.sqrt(_f32(ss * (_f32(1) / _f32(hd)) + _f32(1e-5)))
            r = orc_bf2f_np(orc.f2bf(orc_bf2f_np(xh) * rs))
            assert np.array_equal(got[h * hd:(h + 1) * hd], orc.f2bf(w * r))


def test_embed_row_closed_form(orc):
    """k_dequant_row (lfm3_nanode.cu:138-142): bf16(code * scale), one RNE
    rounding of the product (exact in fp32: 8 x 11 significant bits), with the
    scale of the element's own 32-block."""
    from fractions import Fraction
    # hand-computed: 87 * 1.5009765625 (fp16 0x3e01) = 130.5849609375 -> bf16 131 (0x4303);
    # truncation would give 130 (0x4302)
    W = np.zeros((2, 64), np.int8)
    S = np.full((2, 2), 0x3C00, np.uint16)
    W[1, 0], S[1, 0] = 87, 0x3E01
    W[1, 40], S[1, 1] = -3, 0x3555        # block 1 has its own scale
    row = orc.embed_row(W, S, 1)
    assert row[0] == 0x4303
    assert row[40] == _bf16_rne_exact(-3 * Fraction(int(np.uint16(0x3555).view(np.float16).astype(np.float64) * 2 ** 24), 2 ** 24))
    assert np.all(row[1:32] == 0) and row[32] == 0
    # random rows, every element against the exact rational product
    Wr, Sr = orc.q8_weights(72, 8, 256)
    for tok in (0, 5, 7):
        row = orc.embed_row(Wr, Sr, tok)
        for i in range(256):
            sc = Fraction(float(Sr[tok, i // 32].view(np.float16)))
            assert row[i] == _bf16_rne_exact(int(Wr[tok, i]) * sc), (tok, i)


def _same_rotation(orc, got, want, a, b):
    """The pair (a, b) bit for bit; the other dims are zeros (of either sign:
    0*c - 0*s keeps IEEE's signed zero)."""
    assert got[a] == want[a] and got[b] == want[b], (a, b, got[a], got[b], want[a], want[b])
    assert np.array_equal(orc.bf2f(got), orc.bf2f(want))


@pytest.mark.parametrize("theta,hd,rot", [(1e6, 64, 32), (1e6, 128, 64), (1e4, 64, 64)])
def test_rope_invf_is_build_invf(orc, theta, hd, rot):
    """build_invf (lfm3_nanode.cu:3719-3723) runs on the host in float:
    invf_i = 1.0f / powf(base, (float)(2i) / (float)dim), 0 past rot/2. Pinned
    against the correctly rounded powf (mpmath at 200 bits) and an IEEE float
    divide; the double-precision formula differs in several entries."""
    import mpmath
    mpmath.mp.prec = 200
    invf = orc.rope_invf(hd, rot, theta)
    t = np.float32(theta)
    want = np.zeros(hd // 2, np.float32)
    for i in range(rot // 2):
        e = np.float32(2 * i) / np.float32(hd)
        p = np.float32(float(mpmath.power(mpmath.mpf(float(t)), mpmath.mpf(float(e)))))
        want[i] = np.float32(1) / p
    assert np.array_equal(invf.view(np.uint32), want.view(np.uint32))
    dbl = np.array([1.0 / theta ** (2 * i / hd) for i in range(rot // 2)]).astype(np.float32)
    assert np.count_nonzero(dbl != want[:rot // 2]) >= 5


def test_rope_table_float_angle(orc):
    """Table entries are cos/sin of the fp32 angle fl(pos * invf_i) (k_rope's
    __fmul_rn, lfm3_nanode.cu:491), each correctly rounded to float."""
    import mpmath
    mpmath.mp.prec = 120
    maxpos, hd, rot, theta = 4096, 64, 32, 1e6
    cs = orc.rope_table(maxpos, hd, rot, theta).reshape(maxpos, rot // 2, 2)
    invf = orc.rope_invf(hd, rot, theta)[: rot // 2]
    ang = np.arange(maxpos, dtype=np.float32)[:, None] * invf[None, :]
    assert np.array_equal(cs[..., 0], np.cos(ang.astype(np.float64)).astype(np.float32))
    assert np.array_equal(cs[..., 1], np.sin(ang.astype(np.float64)).astype(np.float32))
    # independent spot checks at 120 bits
    rng = np.random.default_rng(73)
    for p, i in zip(rng.integers(0, maxpos, 48), rng.integers(0, rot // 2, 48)):
        a = mpmath.mpf(float(ang[p, i]))
        assert cs[p, i, 0] == np.float32(float(mpmath.cos(a)))
        assert cs[p, i, 1] == np.float32(float(mpmath.sin(a)))
    # an angle formed in double would give a different table
    ang_d = np.arange(maxpos, dtype=np.float64)[:, None] * invf.astype(np.float64)[None, :]
    assert np.count_nonzero(np.cos(ang_d).astype(np.float32) != cs[..., 0]) > 1000


def test_rope_pairing_sign_and_tail(orc):
    """k_rope (lfm3_nanode.cu:483-498): pairs (i, i + hd/2) for i < rot/2,
    lo' = bf16(lo*c - hi*s), hi' = bf16(hi*c + lo*s); dims in [rot/2, hd/2) and
    their partners are left as they are; position 0 is the identity."""
    maxpos, hd, rot, nh = 1100, 64, 32, 3
    cs = orc.rope_table(maxpos, hd, rot, 1e6).reshape(maxpos, rot // 2, 2)
    x = orc.f2bf(orc.gen_normal(74, nh * hd))
    assert np.array_equal(orc.rope(x, cs.ravel(), 0, nh, hd, rot), x)
    pos = 1000
    for i in range(rot // 2):
        c, s = cs[pos, i]
        for h in range(nh):
            e = np.zeros(nh * hd, np.uint16)
            e[h * hd + i] = 0x3F80                          # lo = 1
            got = orc.rope(e, cs.ravel(), pos, nh, hd, rot)
            want = np.zeros_like(e)
            want[h * hd + i], want[h * hd + i + hd // 2] = orc.f2bf([c])[0], orc.f2bf([s])[0]
            _same_rotation(orc, got, want, h * hd + i, h * hd + i + hd // 2)
            e = np.zeros(nh * hd, np.uint16)
            e[h * hd + i + hd // 2] = 0x3F80                # hi = 1
            got = orc.rope(e, cs.ravel(), pos, nh, hd, rot)
            want = np.zeros_like(e)
            want[h * hd + i], want[h * hd + i + hd // 2] = orc.f2bf([-s])[0], orc.f2bf([c])[0]
            _same_rotation(orc, got, want, h * hd + i, h * hd + i + hd // 2)
    got = orc.rope(x, cs.ravel(), 777, nh, hd, rot).reshape(nh, hd)
    xr = x.reshape(nh, hd)
    for lo, hi in ((rot // 2, hd // 2), (hd // 2 + rot // 2, hd)):
        assert np.array_equal(got[:, lo:hi], xr[:, lo:hi])


# ----------------------------------------------------------------- backbone
TINY = dict(hidden=256, ffn=512, vocab=1000, nlayers=4, nh=4, nkv=2, hd=64, rot=32, ntaps=3, ctx=256,
            eps=1e-5, theta=1e6, seed=20261201, attn_mask=0b1010)


@pytest.mark.parametrize("numerics", [0, 1])
def test_model_batched_equals_sequential(orc, numerics):
    m = orc.Model(**TINY, numerics=numerics)
    prompt = orc.gen_tokens(5, 40, TINY["vocab"])
    r1, lg1 = m.feed(prompt, True)
    h1 = m.hidden()
    m.reset()
    for t in prompt[:-1]:
        m.feed(np.array([t], np.int32))
    r2, lg2 = m.feed(prompt[-1:], True)
    assert r1 == r2 and np.array_equal(f32bits(lg1), f32bits(lg2)) and np.array_equal(h1, m.hidden())
    m.close()


def test_model_head_composition(orc):
    """Logits are the tied Q8 head applied to the final-normed residual, and the
    greedy stream does not collapse onto one token."""
    m = orc.Model(**TINY)
    prompt = orc.gen_tokens(6, 17, TINY["vocab"])
    r, lg = m.feed(prompt, True)
    W, S = m.tensor(-1, 0)
    fn = m.tensor(-1, 1)
    h = orc.rmsnorm(m.hidden(), fn, 1e-5)
    qx, dx = orc.q8_quant_bf16(h)
    assert np.array_equal(f32bits(orc.q8_gemv(W, S, qx, dx)), f32bits(lg))
    assert r == orc.argmax(lg)
    ids = m.greedy(prompt, 16)
    assert len(set(ids.tolist())) >= 6
    m.close()


def test_model_ref_numerics(orc):
    """numerics = 1: the same model with every GEMV in the reference's own order
    (orc_q8r_gemm on bf16 x and the fp32 widening of the same scales): the
    head is that GEMV of the final-normed residual, the greedy stream is live,
    and the logits differ from the Q8_0 x Q8_0 model's (so the switch reaches
    the GEMVs) while staying close to them."""
    m = orc.Model(**TINY, numerics=1)
    prompt = orc.gen_tokens(6, 17, TINY["vocab"])
    r, lg = m.feed(prompt, True)
    W, S = m.tensor(-1, 0)
    h = orc.rmsnorm(m.hidden(), m.tensor(-1, 1), 1e-5)
    want = orc.q8r_gemm(W, S.view(np.float16).astype(np.float32), h[None, :])[0]
    assert np.array_equal(f32bits(want), f32bits(lg)) and r == orc.argmax(lg)
    assert len(set(m.greedy(prompt, 16).tolist())) >= 6
    m.close()
    q = orc.Model(**TINY)
    _, lq = q.feed(prompt, True)
    q.close()
    assert not np.array_equal(f32bits(lq), f32bits(lg))
    assert np.corrcoef(lq, lg)[0, 1] > 0.9


# --------------------------------------------------------- golden fixtures
def test_oracle_reproduces_kernel_fixtures(orc):
    import os
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "kernels.npz"))
    for tag in ("g1", "g2", "g3"):
        qx, dx = orc.q8_quant(d[f"{tag}_x"])
        assert np.array_equal(qx, d[f"{tag}_qx"]) and np.array_equal(f32bits(dx), f32bits(d[f"{tag}_dx"]))
        y = orc.q8_gemm(d[f"{tag}_W"], d[f"{tag}_S"], qx, dx)
        assert np.array_equal(f32bits(y), f32bits(d[f"{tag}_y"]))
    N, K = d["t_y"].size, d["t_x"].size
    assert np.array_equal(orc.q8k_quant(d["t_x"]), d["t_xq"])
    assert np.array_equal(f32bits(orc.tq2_gemv(d["t_codes"], d["t_S"], d["t_xq"], N, K)), f32bits(d["t_y"]))
    assert np.array_equal(orc.attn(d["a_q"], d["a_k"], d["a_v"], 130, 8, 2, 64, 0.125), d["a_out"])


def test_oracle_reproduces_tiny_greedy(orc):
    import json
    import os
    g = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "tiny_greedy.json")))
    m = orc.Model(**g["cfg"])
    assert m.greedy(np.array(g["prompt"], np.int32), len(g["ids"])).tolist() == g["ids"]
    m.close()


# ------------------------------------------------- R2: the reference's own GEMV order
def _bf16(v):
    """float32 values that are bf16-exact -> their bf16 bits."""
    u = np.asarray(v, np.float32).view(np.uint32)
    assert np.all((u & 0xffff) == 0)
    return (u >> 16).astype(np.uint16)


def _leaf_case(values, K=1024):
    """One row whose leaf L (= block L, K = 1024 gives one block per leaf) has
    the value values[L] exactly: code 1 and x = v at the block's first element,
    zeros elsewhere, scale 1."""
    W = np.zeros((1, K), np.int8)
    x = np.zeros(K, np.float32)
    for L, v in enumerate(values):
        W[0, 32 * L] = 1
        x[32 * L] = v
    return W, np.ones((1, K // 32), np.float32), _bf16(x)


def test_r2_leaf_tree_order(orc):
    """The chunk partial is the shfl_down tree 16, 8, 4, 2, 1 over the 32 leaves
    (lfm3_nanode.cu:326). Case A separates it from a sequential fold, case B
    from the ascending tree 1, 2, ..., 16 (closed forms by hand; 2^24 + 1 ties
    to 2^24)."""
    big = float(2 ** 24)
    A = [big] + [1.0] * 31          # tree: 2^24 + 30; sequential: 2^24
    y = orc.q8r_gemm(*_leaf_case(A))
    assert y[0] == np.float32(big + 30)
    B = [0.0] * 32                  # tree 16..1: 2^24; ascending tree: 2^24 + 2
    B[0], B[16], B[24] = big, 1.0, 1.0
    y = orc.q8r_gemm(*_leaf_case(B))
    assert y[0] == np.float32(big)


def test_r2_scale_fma_is_fused(orc):
    """acc = fmaf(s_b, dot_b, acc) (lfm3_nanode.cu:322): leaf 0 of K = 2048 folds
    blocks 0 and 32; block 0 leaves acc = -1, block 32 has s = 1 + 2^-22 and
    dot = 1 + 2^-23, so the fused result 3*2^-23 + 2^-45 differs from the
    unfused 3*2^-23. (The code*x products are exact in fp32, so the dot chain's
    fusing cannot show.)"""
    K = 2048
    W = np.zeros((1, K), np.int8)
    x = np.zeros(K, np.float32)
    S = np.ones((1, K // 32), np.float32)
    W[0, 0], x[0] = -1, 1.0                      # block 0: dot = -1
    W[0, 32 * 32], x[32 * 32] = 1, 1.0           # block 32: dot = 1 + 2^-23
    W[0, 32 * 32 + 1], x[32 * 32 + 1] = 1, 2.0 ** -23
    S[0, 32] = np.float32(1 + 2.0 ** -22)
    y = orc.q8r_gemm(W, S, _bf16(x))
    assert y[0] == np.float32(3 * 2.0 ** -23 + 2.0 ** -45)
    assert y[0] != np.float32(3 * 2.0 ** -23)


def _r2_case(orc, seed, N, K, T=1):
    W, S16 = orc.q8_weights(seed, N, K)
    S = S16.view(np.float16).astype(np.float32)
    xb = orc.f2bf(orc.gen_normal(seed + 3, T * K)).reshape(T, K)
    return W, S, xb


def test_r2_chunks_of_2048(orc):
    """K a multiple of 2048: the chunk partials (each a 32-leaf tree over 64
    blocks) sum from 0 in chunk order (pick(), lfm3_nanode.cu:1763, and
    k_combine_*, 338-345) -- K = 8192 is the in-order sum of its four K = 2048
    slices."""
    W, S, xb = _r2_case(orc, 41, 19, 8192)
    y = orc.q8r_gemm(W, S, xb[0])
    acc = np.zeros(19, np.float32)
    for c in range(4):
        sl = slice(2048 * c, 2048 * (c + 1))
        p = orc.q8r_gemm(np.ascontiguousarray(W[:, sl]), np.ascontiguousarray(S[:, 64 * c:64 * (c + 1)]),
                         np.ascontiguousarray(xb[0, sl]))
        acc = (acc + p).astype(np.float32)
    assert np.array_equal(f32bits(y), f32bits(acc))


@pytest.mark.parametrize("N,K", [(53, 2048), (29, 8192), (17, 7680), (11, 512)])
def test_r2_vs_exact_and_reference_cpu(orc, N, K):
    """Within 1e-5 of sum |terms| of the exact double result and of the
    reference's own CPU GEMV (q8_gemv_cpu.c:29-58, oracle/_ref) on the same
    fp32 scales and bf16 x."""
    W, S, xb = _r2_case(orc, 50 + K, N, K)
    x = orc.bf2f(xb[0])
    y = orc.q8r_gemm(W, S, xb[0]).astype(np.float64)
    terms = W.reshape(N, -1, 32).astype(np.float64) * x.reshape(-1, 32)
    exact = (terms.sum(-1) * S).sum(-1)
    den = (np.abs(terms).sum(-1) * np.abs(S)).sum(-1)
    assert (np.abs(y - exact) / den).max() <= 1e-6
    ref = orc.ref()
    if ref is not None:
        import ctypes as C
        yr = np.empty(N, np.float32)
        ref.ref_q8_gemv(W.ctypes.data_as(C.c_void_p), S.ctypes.data_as(C.c_void_p),
                        x.ctypes.data_as(C.c_void_p), yr.ctypes.data_as(C.c_void_p), C.c_int(N), C.c_int(K))
        assert (np.abs(y - yr) / den).max() <= 1e-5


def test_r2_gemm_is_per_position(orc):
    W, S, xb = _r2_case(orc, 61, 23, 2048, T=3)
    Y = orc.q8r_gemm(W, S, xb)
    for t in range(3):
        assert np.array_equal(f32bits(Y[t]), f32bits(orc.q8r_gemm(W, S, xb[t])))


# ------------------------------------------------ Q4 / Q5: the reference's low-bit order
def _h16(v):
    return np.asarray(v, np.float16).view(np.uint16)


def _qlow_zero(N, K):
    return np.zeros((N, K), np.uint8), np.zeros((N, K // 32, 2), np.uint16), np.zeros(K, np.uint16)


def test_qlow_four_accumulators(orc):
    """a_b folds elements b, b+4, ... (lfm3_qlow.cuh:22-37) and
    acc = (a0 + a1) + (a2 + a3): x = 2^24, 1, 1, 1 at k = 0..3 (q = 0) gives
    acc = 2^24 + 2 where a sequential sum gives 2^24; with d' = 1, mn = 0 the
    output is acc - sg = (2^24 + 2) - 2^24 = 2."""
    Q, S, x = _qlow_zero(1, 2048)
    x[:4] = _bf16([2.0 ** 24, 1.0, 1.0, 1.0])
    S[0, 0] = _h16([1.0, 0.0])
    assert orc.qlow_gemv(Q, S, x)[0] == np.float32(2.0)


def test_qlow_scale_fmas_are_fused(orc):
    """y = fmaf(d', acc - sg, fmaf(mn, sg, y)) (99-101): group 0 leaves y = -1
    (mn = -1, sg = 1), group 1 has d' = 0, mn = 1 + 2^-10 and sg = 1 + 2^-23,
    so the fused inner fma gives 2^-10 + 2^-23 + 2^-33 (unfused: 2^-10 + 2^-23)."""
    Q, S, x = _qlow_zero(1, 2048)
    x[0] = _bf16([1.0])[0]
    x[32], x[33] = _bf16([1.0, 2.0 ** -23])
    S[0, 0] = _h16([0.0, -1.0])
    S[0, 1] = _h16([0.0, 1.0 + 2.0 ** -10])
    want = 2.0 ** -10 + 2.0 ** -23 + 2.0 ** -33
    assert orc.qlow_gemv(Q, S, x)[0] == np.float32(want)
    assert np.float32(want) != np.float32(2.0 ** -10 + 2.0 ** -23)


def test_qlow_k_slices(orc):
    """K = 4096 runs KS = 4 slices (lfm3_nanode.cu:1899) summed in order from 0:
    y_0 = 2^24 from group 0, y_1 = 1 + 1 from groups 40 and 41 gives 2^24 + 2;
    two slices (groups 40, 41 in slice 0) or one chain would give 2^24."""
    Q, S, x = _qlow_zero(1, 4096)
    for g, v in ((0, 2.0 ** 24), (40, 1.0), (41, 1.0)):
        x[32 * g] = _bf16([v])[0]
        S[0, g] = _h16([0.0, 1.0])       # y += mn * sg
    assert orc.qlow_gemv(Q, S, x)[0] == np.float32(2.0 ** 24 + 2)


@pytest.mark.parametrize("bits,N,K", [(4, 37, 2048), (5, 21, 8192), (4, 9, 4096)])
def test_qlow_vs_exact(orc, bits, N, K):
    """Within 1e-5 of sum |terms| of the exact dequantized product
    sum_g (d'/128 * sum q x + mn * sum x) (the identity the decode relies on)."""
    rng = np.random.default_rng(K + bits)
    Q = rng.integers(0, 2 ** bits, (N, K)).astype(np.uint8)
    d = (np.abs(rng.standard_normal((N, K // 32))) * 0.02).astype(np.float16)
    mn = (-rng.random((N, K // 32)) * 0.3).astype(np.float16)
    S = np.stack([(d.astype(np.float32) * 128).astype(np.float16).view(np.uint16), mn.view(np.uint16)], -1)
    xb = orc.f2bf(orc.gen_normal(K + 1, K))
    x = orc.bf2f(xb).astype(np.float64).reshape(-1, 32)
    dp = S[..., 0].view(np.float16).astype(np.float64)
    m = S[..., 1].view(np.float16).astype(np.float64)
    q = Q.reshape(N, -1, 32).astype(np.float64)
    exact = (dp / 128 * (q * x).sum(-1) + m * x.sum(-1)).sum(-1)
    den = (np.abs(dp) * ((1 + q / 128) * np.abs(x)).sum(-1) + np.abs(m) * np.abs(x).sum(-1)).sum(-1)
    y = orc.qlow_gemv(Q, S, xb).astype(np.float64)
    assert (np.abs(y - exact) / den).max() <= 1e-5


# ------------------------------------------- the bf16-table LM head (k_gemv_bf16)
def _bf16_head_case(K, vals):
    """One row of ones and x = vals at the given element indices (exact in bf16)."""
    W = np.full((1, K), 0x3F80, np.uint16)
    x = np.zeros(K, np.float32)
    for k, v in vals.items():
        x[k] = v
    return W, _bf16(x)


def test_bf16_head_leaves_stride_32(orc):
    """orc_bf16_gemv follows k_gemv_bf16 (lfm3_nanode.cu:3517-3534): leaf L sums
    elements L, L+32, L+64, ... in order, rounding each add; the leaves combine as
    the shfl_down tree 16, 8, 4, 2, 1. Closed forms by hand (2^24 + 1 ties to 2^24):
      A: x[0] = x[32] = 1, x[1] = 2^24 -- leaf 0 = 2, leaf 1 = 2^24, tree 2^24 + 2;
         a sequential sum over k, or lanes holding contiguous pairs, give 2^24;
      B: x[0] = 2^24, x[32] = x[64] = 1 -- leaf 0 in order: 2^24; a pairwise
         leaf (x0 + (x32 + x64)) gives 2^24 + 2;
      C: x[0] = x[16] = 1, x[1] = 2^24 -- the tree adds leaves 0 and 16 first
         (2), then leaf 1: 2^24 + 2; a sequential fold over the leaves gives 2^24."""
    big = float(2 ** 24)

    def sequential(x):   # one fp32 chain over k, the departure cases A and C rule out
        s = np.float32(0)
        for v in orc.bf2f(x):
            s = np.float32(s + v)
        return s

    W, x = _bf16_head_case(64, {0: 1.0, 32: 1.0, 1: big})
    assert orc.bf16_gemv(W, x)[0] == np.float32(big + 2) and sequential(x) == np.float32(big)
    W, x = _bf16_head_case(96, {0: big, 32: 1.0, 64: 1.0})
    assert orc.bf16_gemv(W, x)[0] == np.float32(big)
    W, x = _bf16_head_case(64, {0: 1.0, 16: 1.0, 1: big})
    assert orc.bf16_gemv(W, x)[0] == np.float32(big + 2) and sequential(x) == np.float32(big)


def test_bf16_head_vs_exact(orc):
    """Random bf16 rows and x: within 1e-6 of sum |w x| of the exact double sum
    (the products are exact in fp32, only the adds round); rows are independent."""
    rng = np.random.default_rng(71)
    N, K = 37, 2048
    W = orc.f2bf(rng.standard_normal(N * K).astype(np.float32)).reshape(N, K)
    x = orc.f2bf(rng.standard_normal(K).astype(np.float32) * 3)
    y = orc.bf16_gemv(W, x).astype(np.float64)
    t = orc.bf2f(W).astype(np.float64) * orc.bf2f(x).astype(np.float64)
    assert (np.abs(y - t.sum(1)) / np.abs(t).sum(1)).max() <= 1e-6
    assert np.array_equal(f32bits(orc.bf16_gemv(W[5:9], x)), f32bits(orc.bf16_gemv(W, x)[5:9]))


# ------------------------------- the low-bit backbone and the bf16 table (numerics 1)
LOWQ = dict(TINY, numerics=1, lowbit=4, lowbit_mask=0b0110, emb_bf16=1)


def test_model_lowbit_parts(orc):
    """Layers in lowbit_mask list their source tensors as low-bit (all but the
    attention gate_proj, which stays Q8); others all Q8. An R1 model refuses
    low-bit tensors and the bf16 table (they take bf16 activations)."""
    m = orc.Model(**LOWQ)
    H, F = TINY["hidden"], TINY["ffn"]
    assert m.parts(1, 0) == [(0, 256, 4), (256, 128, 4), (384, 128, 4), (512, 4, 8)]
    assert m.parts(2, 0) == [(0, 3 * H, 4)] and m.parts(2, 2) == [(0, F, 4), (F, F, 4)]
    assert m.parts(0, 0) == [(0, 3 * H, 8)] and m.lowbit(0, 0) is None
    Q, S = m.lowbit(1, 3)
    assert Q.shape == (H, F) and Q.max() == 15 and S.shape == (H, F // 32, 2)
    m.close()
    for bad in (dict(LOWQ, numerics=0), dict(TINY, emb_bf16=1), dict(LOWQ, lowbit=3)):
        with pytest.raises(ValueError):
            orc.Model(**bad)


@pytest.mark.parametrize("bits", [4, 5])
def test_model_lowbit_batched_equals_sequential(orc, bits):
    m = orc.Model(**dict(LOWQ, lowbit=bits))
    prompt = orc.gen_tokens(5, 33, TINY["vocab"])
    r1, lg1 = m.feed(prompt, True)
    h1 = m.hidden()
    m.reset()
    for t in prompt[:-1]:
        m.feed(np.array([t], np.int32))
    r2, lg2 = m.feed(prompt[-1:], True)
    assert r1 == r2 and np.array_equal(f32bits(lg1), f32bits(lg2)) and np.array_equal(h1, m.hidden())
    assert len(set(m.greedy(prompt, 16).tolist())) >= 6
    m.close()


def _layer_by_hand(orc, m, cfg, tok):
    """One position through a one-layer model, restated from layer_body
    (lfm3_nanode.cu:3739-3856) with the pinned primitives, every GEMV per
    source tensor (gemv per name, 1916-1923: low-bit -> qlow_gemv, Q8 -> the R2
    GEMV), the bf16 table's row and head (6062-6076, 3536-3573)."""
    H, F, hd, nh, nkv = cfg["hidden"], cfg["ffn"], cfg["hd"], cfg["nh"], cfg["nkv"]

    def gemv(slot, x):
        W, S = m.tensor(0, slot)
        low = m.lowbit(0, slot)
        y = np.empty(W.shape[0], np.float32)
        for r0, n, bits in m.parts(0, slot):
            if bits == 8:
                y[r0:r0 + n] = orc.q8r_gemm(W[r0:r0 + n], S[r0:r0 + n].view(np.float16).astype(np.float32), x)
            else:
                y[r0:r0 + n] = orc.qlow_gemv(low[0][r0:r0 + n], low[1][r0:r0 + n], x)
        return orc.f2bf(y)

    if cfg.get("emb_bf16"):
        x = np.array(m.tensor(-1, 3)[tok])
    else:
        x = orc.embed_row(*m.tensor(-1, 0), tok)
    h1 = orc.rmsnorm(x, m.tensor(0, 4))
    if cfg["attn_mask"] & 1:
        qd, kd = nh * hd, nkv * hd
        w = gemv(0, h1)
        q = orc.headnorm(w[:qd], m.tensor(0, 8), nh, hd)
        k = orc.headnorm(w[qd:qd + kd], m.tensor(0, 9), nkv, hd)
        cs = orc.rope_table(cfg["ctx"], hd, cfg["rot"], cfg["theta"])
        q, k = orc.rope(q, cs, 0, nh, hd, cfg["rot"]), orc.rope(k, cs, 0, nkv, hd, cfg["rot"])
        kc = orc.bf2f(k).astype(np.float16).view(np.uint16)
        vc = orc.bf2f(w[qd + kd:qd + 2 * kd]).astype(np.float16).view(np.uint16)
        a = orc.attn(q, kc, vc, 1, nh, nkv, hd, 1.0 / np.sqrt(np.float32(hd)))
        a = orc.sigmoid_gate(w[qd + 2 * kd:], a, nh, hd)
        h2 = gemv(1, a)
    else:
        bcx = gemv(0, h1)
        out, _ = orc.conv_step(np.zeros(cfg["ntaps"] * H, np.uint16), m.tensor(0, 10), bcx, H, cfg["ntaps"])
        h2 = gemv(1, out)
    x = orc.add(x, orc.rmsnorm(h2, m.tensor(0, 5)))
    gu = gemv(2, orc.rmsnorm(x, m.tensor(0, 6)))
    d = gemv(3, orc.silu_mul(gu[:F], gu[F:]))
    x = orc.add(x, orc.rmsnorm(d, m.tensor(0, 7)))
    h = orc.rmsnorm(x, m.tensor(-1, 1))
    if cfg.get("emb_bf16"):
        return orc.bf16_gemv(m.tensor(-1, 3), h)
    E, ES = m.tensor(-1, 0)
    return orc.q8r_gemm(E, ES.view(np.float16).astype(np.float32), h)


@pytest.mark.parametrize("kind", ["conv", "attn"])
@pytest.mark.parametrize("low", [(0, 0), (4, 0), (5, 1)], ids=["q8-table", "q4-table", "q5-bf16"])
def test_model_layer_composition(orc, kind, low):
    """The oracle's layer and head composition against a second restatement of
    layer_body built from the separately pinned primitives: which norm weight
    goes where, the residual adds, the per-tensor GEMV dispatch of a low-bit
    layer, the embedding row and tied head of a Q8 or bf16 table."""
    bits, emb16 = low
    cfg = dict(TINY, nlayers=1, attn_mask=1 if kind == "attn" else 0, numerics=1, lowbit=bits,
               lowbit_mask=1 if bits else 0, emb_bf16=emb16)
    m = orc.Model(**cfg)
    _, lg = m.feed(np.array([417], np.int32), True)
    assert np.array_equal(f32bits(_layer_by_hand(orc, m, cfg, 417)), f32bits(lg))
    m.close()
