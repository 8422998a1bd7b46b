"""The fused decode kernels equal the unfused op sequences bit for bit (and hence
the oracle): every GEMV prologue kind, the LM head's argmax partials, the
one-launch attention mixer, and the engine's fused decode path."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
SEED = 4242


def _t16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


def _u16(t):
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return t.cpu().numpy().view(np.uint16)


def _w(orc, pq, dev, N, K, seed):
    W, S = orc.q8_weights(seed, N, K)
    return W, S, pq.Q8Weight(torch.from_numpy(W).to(dev), torch.from_numpy(S.view(np.int16)).to(dev))


def _ref_gemv(orc, W, S, xb):
    qx, dx = orc.q8_quant_bf16(xb)
    return orc.f2bf(orc.q8_gemv(W, S, qx, dx))


@pytest.mark.parametrize("N", [3104, 6144, 16384, 2048, 65536])
def test_resnorm_prologue(orc, pq, dev, N):
    H = 2048
    W, S, w = _w(orc, pq, dev, N, H, SEED + N)
    x = orc.f2bf(orc.gen_normal(SEED + 1, H) * 5)
    h = orc.f2bf(orc.gen_normal(SEED + 2, H) * 40)
    w0 = orc.gen_affine(SEED + 3, H, 4.0, 0.4)
    w1 = orc.gen_affine(SEED + 4, H, 1.0, 0.1)
    xn = orc.add(x, orc.rmsnorm(h, w0))
    y_in = orc.rmsnorm(xn, w1)
    xo = torch.zeros(H, dtype=torch.int16, device=dev)
    dt = pq.DT_F32 if N == 65536 else pq.DT_BF16
    parts = torch.empty(2 * pq.lib().pq_q8_gemv_parts(N, H), dtype=torch.float32, device=dev) if N == 65536 else None
    y = pq.gemv_fused(w, pq.PRO_RESNORM, out_dtype=dt, parts=parts, h=_t16(h, dev), x_in=_t16(x, dev), x_out=xo,
                      w0=torch.from_numpy(w0).to(dev), w1=torch.from_numpy(w1).to(dev))
    assert np.array_equal(_u16(xo), xn)
    qx, dx = orc.q8_quant_bf16(y_in)
    yr = orc.q8_gemv(W, S, qx, dx)
    if dt == pq.DT_F32:
        assert np.array_equal(y.cpu().numpy().view(np.uint32), yr.view(np.uint32))
        nparts = pq.lib().pq_q8_gemv_parts(N, H)
        assert int(pq.argmax_parts(parts, nparts).item()) == orc.argmax(yr)
    else:
        assert np.array_equal(_u16(y), orc.f2bf(yr))


def test_norm_and_embed_prologues(orc, pq, dev):
    H, N, vocab = 2048, 6144, 3000
    W, S, w = _w(orc, pq, dev, N, H, SEED + 10)
    E, ES, emb = _w(orc, pq, dev, vocab, H, SEED + 11)
    w0 = orc.gen_affine(SEED + 12, H, 1.0, 0.1)
    x = orc.f2bf(orc.gen_normal(SEED + 13, H) * 3)
    y = pq.gemv_fused(w, pq.PRO_NORM, x_in=_t16(x, dev), w0=torch.from_numpy(w0).to(dev))
    assert np.array_equal(_u16(y), _ref_gemv(orc, W, S, orc.rmsnorm(x, w0)))
    for tok in (0, 2999, 64, 1234):
        xo = torch.zeros(H, dtype=torch.int16, device=dev)
        y = pq.gemv_fused(w, pq.PRO_EMBED, tok=torch.tensor([tok], dtype=torch.int32, device=dev), emb=emb,
                          vocab=vocab, x_out=xo, w0=torch.from_numpy(w0).to(dev))
        e = orc.embed_row(E, ES, tok)
        assert np.array_equal(_u16(xo), e)
        assert np.array_equal(_u16(y), _ref_gemv(orc, W, S, orc.rmsnorm(e, w0)))


def test_silu_prologue(orc, pq, dev):
    F, N = 8192, 2048
    W, S, w = _w(orc, pq, dev, N, F, SEED + 20)
    gu = orc.f2bf(orc.gen_normal(SEED + 21, 2 * F) * 30)
    y = pq.gemv_fused(w, pq.PRO_SILU, gu=_t16(gu, dev))
    assert np.array_equal(_u16(y), _ref_gemv(orc, W, S, orc.silu_mul(gu[:F], gu[F:])))


@pytest.mark.parametrize("nt", [3, 7])
def test_conv_prologue(orc, pq, dev, nt):
    H, N = 2048, 2048
    W, S, w = _w(orc, pq, dev, N, H, SEED + 30)
    taps = orc.gen_affine(SEED + 31, H * nt, 0.0, 0.5)
    ring = orc.f2bf(orc.gen_normal(SEED + 32, nt * H) * 3)
    bcx = orc.f2bf(orc.gen_normal(SEED + 33, 3 * H) * 10)
    o, ring_new = orc.conv_step(ring, taps, bcx, H, nt)
    rin, rout = _t16(ring, dev), torch.zeros(nt * H, dtype=torch.int16, device=dev)
    y = pq.gemv_fused(w, pq.PRO_CONV, bcx=_t16(bcx, dev), ring_in=rin, ring_out=rout,
                      taps=torch.from_numpy(taps).to(dev), ntaps=nt)
    assert np.array_equal(_u16(rout), ring_new)
    assert np.array_equal(_u16(rin), ring)
    assert np.array_equal(_u16(y), _ref_gemv(orc, W, S, o))


@pytest.mark.parametrize("N,K", [(3072, 2048), (65536, 2048), (2048, 8192), (130, 1024)])
def test_f32_prologue(orc, pq, dev, N, K):
    W, S, w = _w(orc, pq, dev, N, K, SEED + 70 + N)
    x = orc.gen_normal(SEED + 71 + K, K)
    qx, dx = orc.q8_quant(x)
    yr = orc.q8_gemv(W, S, qx, dx)
    y = pq.gemv_fused(w, pq.PRO_F32, out_dtype=pq.DT_F32, xf=torch.from_numpy(x).to(dev))
    assert np.array_equal(y.cpu().numpy().view(np.uint32), yr.view(np.uint32))


# k_argmax's tie order through the argmax partials of the fused GEMVs: rows 1,
# 2, 33, 64 and 300 hold the same codes and scales and give the largest
# outputs, so they tie; k_argmax picks row 2 (lane 2 outranks lane 1, warp 0
# outranks warps 1 and 2; the oracle's transcription agrees), where the lowest
# index would be row 1.
TIED = [1, 2, 33, 64, 300]


def test_argmax_parts_tie_order(orc, pq, dev):
    N, K = 3072, 2048
    W, S = orc.q8_weights(SEED + 91, N, K)
    W[TIED] = 127
    S[TIED] = np.float16(0.01).view(np.uint16)
    x = (np.abs(orc.gen_normal(SEED + 90, K)) + 0.5).astype(np.float32)
    qx, dx = orc.q8_quant(x)
    yr = orc.q8_gemv(W, S, qx, dx)
    assert (yr[TIED] == yr.max()).all() and orc.argmax(yr) == 2
    w = pq.Q8Weight(torch.from_numpy(W).to(dev), torch.from_numpy(S.view(np.int16)).to(dev))
    nparts = pq.lib().pq_q8_gemv_parts(N, K)
    parts = torch.empty(2 * nparts, dtype=torch.float32, device=dev)
    y = pq.gemv_fused(w, pq.PRO_F32, out_dtype=pq.DT_F32, parts=parts, xf=torch.from_numpy(x).to(dev))
    assert np.array_equal(y.cpu().numpy().view(np.uint32), yr.view(np.uint32))
    assert int(pq.argmax_parts(parts, nparts).item()) == 2
    assert int(pq.argmax(y).item()) == 2
    # the reference-numerics GEMV's pairs (row-major codes, fp32 scales)
    codes = torch.from_numpy(W).to(dev)
    scales = torch.from_numpy(S.view(np.float16).astype(np.float32)).to(dev)
    w0 = torch.ones(K, device=dev)
    xb = torch.from_numpy(orc.f2bf(x).view(np.int16)).to(dev)
    nparts = pq.lib().pq_q8r_gemv_parts(N)
    parts = torch.empty(2 * nparts, dtype=torch.float32, device=dev)
    y2 = pq.q8r_gemv_fused(codes, scales, pq.PRO_NORM, out_dtype=pq.DT_F32, parts=parts, x_in=xb, w0=w0)
    y2h = y2.cpu().numpy()
    assert (y2h[TIED] == y2h.max()).all() and orc.argmax(y2h) == 2
    assert int(pq.argmax_parts(parts, nparts).item()) == 2


@pytest.mark.parametrize("nt", [3, 7])
def test_conv_prologue_closed_forms(orc, pq, dev, nt):
    """The CONV prologue on the hand-built channels of tests/conv_cases.py (ascending
    unfused tap sum, bx and cy rounded to bf16): the shifted ring it writes, and the
    GEMV of its conv output, equal the closed forms."""
    import conv_cases as cc
    H = N = 2048
    W, S, w = _w(orc, pq, dev, N, H, SEED + 35)
    rb, taps, bcx, _ = cc.build(H, nt)
    want_out, want_ring = cc.expected(H, nt)
    rout = torch.zeros(nt * H, dtype=torch.int16, device=dev)
    y = pq.gemv_fused(w, pq.PRO_CONV, bcx=_t16(bcx, dev), ring_in=_t16(rb.reshape(-1), dev), ring_out=rout,
                      taps=torch.from_numpy(taps.reshape(-1)).to(dev), ntaps=nt)
    assert np.array_equal(_u16(rout).reshape(nt, H), want_ring)
    assert np.array_equal(_u16(y), _ref_gemv(orc, W, S, want_out))


def test_f32_prologue_quant_ties(orc, pq, dev):
    """The F32 prologue's quantizer (and pq_q8_quant) on blocks of exact halves
    (tests/quant_cases.py): codes rounded half to even, as lrintf in the
    reference's quant_row, then the GEMV over them."""
    import quant_cases as qc
    K, N = 2048, 2048
    x = qc.tie_blocks(seed=31, reps=10)[:K]
    qx_r, dx_r = orc.q8_quant(x)
    assert np.array_equal(qx_r, qc.rne_codes(x))
    qx, dx = pq.q8_quant(torch.from_numpy(x).to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(qx.cpu().numpy().reshape(-1), qx_r)
    assert np.array_equal(dx.cpu().numpy().reshape(-1).view(np.uint32), dx_r.view(np.uint32))
    W, S, w = _w(orc, pq, dev, N, K, SEED + 36)
    y = pq.gemv_fused(w, pq.PRO_F32, out_dtype=pq.DT_F32, xf=torch.from_numpy(x).to(dev))
    assert np.array_equal(y.cpu().numpy().view(np.uint32), orc.q8_gemv(W, S, qx_r, dx_r).view(np.uint32))


def _bench_shapes():
    import bench
    return bench.SHAPES


@pytest.mark.parametrize("name,N,K,o", _bench_shapes(), ids=[s[0] for s in _bench_shapes()])
def test_f32_prologue_bench_step(orc, pq, dev, name, N, K, o):
    """The launch bench.py times, in the form it times it: q8_gemv_fused_kernel with
    the F32 prologue on each GEMV of its step, with the output dtype it writes
    (bf16 for the layer GEMVs, fp32 logits for the LM head), twice in a row into
    the same output, against the oracle's R1 GEMV."""
    W, S, w = _w(orc, pq, dev, N, K, SEED + 170 + N + K)
    dt = pq.DT_F32 if o == "f32" else pq.DT_BF16
    out = torch.empty(N, dtype=torch.float32 if o == "f32" else torch.bfloat16, device=dev)
    for rep in range(2):
        x = orc.gen_normal(SEED + 171 + rep + K, K)
        qx, dx = orc.q8_quant(x)
        yr = orc.q8_gemv(W, S, qx, dx)
        y = pq.gemv_fused(w, pq.PRO_F32, out_dtype=dt, out=out, xf=torch.from_numpy(x).to(dev))
        torch.cuda.synchronize()
        if o == "f32":
            assert np.array_equal(y.cpu().numpy().view(np.uint32), yr.view(np.uint32)), (name, rep)
        else:
            assert np.array_equal(_u16(y), orc.f2bf(yr)), (name, rep)


def test_q8_prologue(orc, pq, dev):
    N, K = 2048, 2048
    W, S, w = _w(orc, pq, dev, N, K, SEED + 40)
    x = orc.gen_normal(SEED + 41, K)
    qx, dx = pq.q8_quant(torch.from_numpy(x).to(dev))
    y = pq.gemv_fused(w, pq.PRO_Q8, qx=qx, dx=dx)
    assert torch.equal(y.view(torch.int16), pq.q8_gemv(w, qx, dx, out_dtype=pq.DT_BF16).view(torch.int16))


# (pos, hd, nh, nkv, rot, theta, win): head_dim 64 full attention (the K/V-through-LDS
# mixer), then head_dim 128 full / sliding and head_dim 64 sliding (the generic mixer)
MIXER_CASES = [(0, 64, 32, 8, 32, 1e6, 0), (63, 64, 32, 8, 32, 1e6, 0), (64, 64, 32, 8, 32, 1e6, 0),
               (300, 64, 32, 8, 32, 1e6, 0), (2047, 64, 32, 8, 32, 1e6, 0), (4500, 64, 32, 8, 32, 1e6, 0),
               (0, 128, 16, 4, 64, 1e6, 0), (300, 128, 16, 4, 64, 1e6, 0), (2047, 128, 16, 4, 64, 1e6, 0),
               (300, 128, 16, 4, 128, 1e4, 256), (256, 128, 16, 4, 128, 1e4, 256), (1000, 128, 16, 4, 128, 1e4, 256),
               (130, 64, 32, 8, 32, 1e6, 100), (40, 128, 16, 4, 128, 1e4, 1)]


# quant: o_proj's Q8_0 input as well as the bf16 output, or the bf16 output
# alone (the reference-numerics engine's o_proj reads bf16); the small-head
# cases (4 q / 2 kv heads) are the tiny test model's shapes
@pytest.mark.parametrize("quant", [True, False], ids=["q8", "bf16"])
@pytest.mark.parametrize("pos,hd,nh,nkv,rot,theta,win", MIXER_CASES + [(37, 64, 4, 2, 32, 1e6, 0),
                                                                     (37, 128, 4, 2, 64, 1e6, 0)])
def test_attn_layer_decode(orc, pq, dev, pos, hd, nh, nkv, rot, theta, win, quant):
    print(f"mixer pos={pos} hd={hd} nh={nh} win={win} quant={quant}", flush=True)
    ctx = max(2048, pos + 1)
    nin = nh * hd + 2 * nkv * hd + nh
    kvd = nkv * hd
    row = orc.f2bf(orc.gen_normal(SEED + pos, nin) * 30)
    qn = orc.gen_affine(SEED + 50, hd, 1.0, 0.1)
    kn = orc.gen_affine(SEED + 51, hd, 1.0, 0.1)
    cs = orc.rope_table(ctx, hd, rot, theta)
    kc0 = np.zeros((ctx, kvd), np.float16)
    vc0 = np.zeros((ctx, kvd), np.float16)
    kc0[:pos] = orc.gen_normal(SEED + 52, pos * kvd).reshape(pos, kvd) * 2
    vc0[:pos] = orc.gen_normal(SEED + 53, pos * kvd).reshape(pos, kvd) * 5
    args = [torch.from_numpy(qn).to(dev), torch.from_numpy(kn).to(dev), torch.from_numpy(cs).to(dev)]
    # unfused: qk_prep then attn_decode
    r1 = _t16(row, dev)
    kc1, vc1 = _t16(kc0.view(np.uint16), dev), _t16(vc0.view(np.uint16), dev)
    pq.qk_prep(r1, nin, *args, kc1, vc1, pos, nh, nkv, hd, rot, 1)
    out1 = torch.empty(nh * hd, dtype=torch.int16, device=dev)
    qx1 = torch.empty(nh * hd, dtype=torch.int8, device=dev)
    dx1 = torch.empty(nh * hd // 32, dtype=torch.float32, device=dev)
    pq.attn_decode(r1, nin, kc1, vc1, pos, nh, nkv, hd, 1, 0.125, gate=r1[nh * hd + 2 * kvd:], gate_stride=nin,
                   out=out1, out_stride=nh * hd, qx=qx1, dx=dx1, win=win)
    # fused
    r2 = _t16(row, dev)
    kc2, vc2 = _t16(kc0.view(np.uint16), dev), _t16(vc0.view(np.uint16), dev)
    out2 = torch.empty(nh * hd, dtype=torch.int16, device=dev)
    qx2, dx2 = pq.attn_layer_decode(r2, *args, kc2, vc2, pos, nh, nkv, hd, rot, 0.125, out=out2, win=win, quant=quant)
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    assert torch.equal(out1, out2)
    if quant:
        assert torch.equal(qx1, qx2) and torch.equal(dx1.view(torch.int32), dx2.view(torch.int32))


# the synthetic backbone's layer shapes (head_dim 64, 3 taps: the one-launch
# attention mixer), and the real LFM3 widths (head_dim 128, FFN 7680, 7 taps,
# a full and a sliding-window attention layer with the window cut to 40: the
# q/k prep + split-K attention pair, the 7-tap CONV prologue and the plain
# Q8_0 GEMV for the K = 7680 down projection)
FUSED_CFGS = {
    "synth": dict(hidden=2048, ffn=8192, vocab=65536, nlayers=3, nh=32, nkv=8, hd=64, rot=32, ntaps=3, ctx=512,
                  eps=1e-5, theta=1e6, seed=77, attn_mask=0b010),
    "lfm3": dict(hidden=2048, ffn=7680, vocab=128000, nlayers=4, nh=16, nkv=4, hd=128, rot=64, ntaps=7, ctx=256,
                 eps=1e-5, theta=1e6, seed=78, attn_mask=0b1010, slide_mask=0b1000, slide_win=40, slide_rot=128,
                 slide_theta=1e4),
}


@pytest.mark.parametrize("numerics", [0, 1], ids=["q8", "ref"])
@pytest.mark.parametrize("which", list(FUSED_CFGS))
def test_engine_fused_equals_unfused(orc, pq, dev, which, numerics):
    """Fused steps replayed as captured graphs, fused steps launched one by one,
    and the unfused op sequence give the oracle's ids and the same final
    residual, under both GEMV numerics; graph replays are split into several
    decode calls with eager work (state reads, a non-graph step) between them."""
    from pulsar_amd.engine import Engine
    cfg = dict(FUSED_CFGS[which], numerics=numerics)
    prompt = orc.gen_tokens(9, 70, cfg["vocab"])
    m = orc.Model(**{k: v for k, v in cfg.items()})
    ref = m.greedy(prompt, 12)
    m.close()
    resid = []
    for fused, graph in ((True, True), (True, False), (False, False)):
        e = Engine(**cfg)
        e.load_synthetic()
        e.set_fused(fused)
        e.set_graph(graph)
        ids = e.greedy(prompt, 12)
        resid.append(e.hidden())
        e.close()
        assert np.array_equal(ids, ref), (fused, graph)
    assert np.array_equal(resid[0], resid[2]) and np.array_equal(resid[1], resid[2])
    e = Engine(**cfg)
    e.load_synthetic()
    assert e.feed(prompt) == ref[0]
    out = []
    for k, graph in ((3, True), (1, False), (4, True), (2, True)):
        e.set_graph(graph)
        out.extend(e.decode(k).tolist())
        e.hidden()
    e.close()
    assert np.array_equal(np.array(out), ref[1:11]), (out, ref[1:11].tolist())


def test_gate_up_interleave_and_swiglu(orc, pq, dev):
    """Interleaved gate/up packing: the GEMV returns the rows in 32-row groups,
    silu_mul over that order equals the plain one, and the fused SwiGLU
    epilogue gives the Q8_0 row of silu(gate)*up bit for bit."""
    H, F = 2048, 8192
    W, S = orc.q8_weights(SEED + 60, 2 * F, H)
    w = pq.Q8Weight(torch.from_numpy(W).to(dev), torch.from_numpy(S.view(np.int16)).to(dev), gate_up=True)
    x = orc.f2bf(orc.gen_normal(SEED + 61, H) * 5)
    h = orc.f2bf(orc.gen_normal(SEED + 62, H) * 40)
    w0 = orc.gen_affine(SEED + 63, H, 4.0, 0.4)
    w1 = orc.gen_affine(SEED + 64, H, 1.0, 0.1)
    xin = orc.rmsnorm(orc.add(x, orc.rmsnorm(h, w0)), w1)
    qx, dx = orc.q8_quant_bf16(xin)
    gu = orc.f2bf(orc.q8_gemv(W, S, qx, dx))                       # [gate | up], bf16
    act = orc.silu_mul(gu[:F], gu[F:])
    qa, da = orc.q8_quant_bf16(act)
    # the GEMV over the interleaved packing
    y = pq.q8_gemv(w, torch.from_numpy(qx).to(dev), torch.from_numpy(dx).to(dev), out_dtype=pq.DT_BF16)
    yi = _u16(y).reshape(F // 32, 2, 32)
    assert np.array_equal(yi[:, 0, :].reshape(-1), gu[:F]) and np.array_equal(yi[:, 1, :].reshape(-1), gu[F:])
    # silu over the interleaved row
    ys, q1, d1 = pq.silu_mul(y.view(torch.bfloat16), F, 1, out=True, quant=True, interleaved=True)
    assert np.array_equal(_u16(ys).reshape(-1), act)
    assert np.array_equal(q1.cpu().numpy().reshape(-1), qa) and np.array_equal(d1.cpu().numpy().reshape(-1), da)
    # RESNORM prologue + SwiGLU epilogue in one launch
    xo = torch.zeros(H, dtype=torch.int16, device=dev)
    q2, d2 = pq.gemv_fused_swiglu(w, pq.PRO_RESNORM, h=_t16(h, dev), x_in=_t16(x, dev), x_out=xo,
                                  w0=torch.from_numpy(w0).to(dev), w1=torch.from_numpy(w1).to(dev))
    assert np.array_equal(q2.cpu().numpy(), qa)
    assert np.array_equal(d2.cpu().numpy().view(np.uint32), da.view(np.uint32))
