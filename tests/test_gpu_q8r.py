"""GPU parity: the reference-numerics GEMV (pq_q8r_gemv, the reference's own
order: bf16 x, fp32 weight scales, fmaf block dots, 32-leaf shfl_down tree,
2048-wide chunks) against the oracle's restatement, bit for bit."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SEED = 20261203


def _case(orc, N, K, T, seed, signed_scales=False):
    W, S16 = orc.q8_weights(seed, N, K)
    S = S16.view(np.float16).astype(np.float32)
    if signed_scales:
        S = S * np.where(orc.gen_codes(seed + 5, N * (K // 32)).reshape(S.shape) < 0, -1.0, 1.0).astype(np.float32)
    xb = orc.f2bf(orc.gen_normal(seed + 3, T * K) * 3.0).reshape(T, K)
    return W, S, xb


def _run(pq, dev, W, S, xb, dt):
    x = torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16)
    y = pq.q8r_gemv(torch.from_numpy(W).to(dev), torch.from_numpy(S).to(dev), x, out_dtype=dt)
    torch.cuda.synchronize()
    return y


# T > 1 runs the T-wide form (up to 32 positions per workgroup, x staged up to
# 8 positions at a time): T = 40 and 33 cross both boundaries, K = 8192 and
# 12288 fold several 2048-wide chunks, K = 7680 and 2560 are one chunk of 240
# and 80 blocks (leaves with several blocks, codes widened per use); at T = 1
# rows of 2..8 chunks on few workgroups split their chunks over half-waves
# (K = 4096, 6144: two per row; 8192, 12288, 16384: four); K = 5120, 7680
# and 8160 are one chunk of 5..8 blocks per lane
@pytest.mark.parametrize("N,K,T", [(8192, 2048, 1), (3072, 2048, 1), (2048, 8192, 1), (97, 7680, 2),
                                   (61, 512, 1), (37, 1024, 3), (13, 32, 1), (65, 12288, 1), (45, 2560, 2),
                                   (2048, 2048, 4), (300, 2048, 40), (77, 8192, 33), (97, 7680, 9),
                                   (64, 12288, 5), (45, 2560, 17), (300, 4096, 1), (33, 16384, 1),
                                   (7, 6144, 1), (2048, 7680, 1), (131, 5120, 1), (40, 8160, 1)])
def test_q8r_gemv_bitexact(orc, pq, dev, N, K, T):
    print(f"q8r N={N} K={K} T={T}", flush=True)
    W, S, xb = _case(orc, N, K, T, SEED + N + K, signed_scales=(N % 2 == 1))
    want = orc.q8r_gemm(W, S, xb)
    y = _run(pq, dev, W, S, xb, pq.DT_F32).cpu().numpy()
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
    yb = _run(pq, dev, W, S, xb, pq.DT_BF16).cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(yb, orc.f2bf(want))


def test_q8r_zero_and_one_hot(orc, pq, dev):
    """x = 0 gives exact zeros; a one-hot x picks column k times the block scale."""
    N, K = 40, 2048
    W, S, _ = _case(orc, N, K, 1, SEED + 9)
    xb = np.zeros((2, K), np.uint16)
    k = 1234
    xb[1, k] = 0x3f80   # 1.0
    y = _run(pq, dev, W, S, xb, pq.DT_F32).cpu().numpy()
    assert np.all(y[0].view(np.uint32) == 0)
    assert np.array_equal(y[1], (W[:, k].astype(np.float32) * S[:, k // 32]).astype(np.float32))
    assert np.array_equal(y.view(np.uint32), orc.q8r_gemm(W, S, xb).view(np.uint32))


def test_q8r_rejects_bad_args(pq, dev):
    K = 8992   # above 8192 and not a multiple of 2048
    W = torch.zeros((8, K), dtype=torch.int8, device=dev)
    S = torch.zeros((8, K // 32), dtype=torch.float32, device=dev)
    x = torch.zeros(K, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError):
        pq.q8r_gemv(W, S, x)


# The T = 1 reference-numerics GEMV with x from a prologue equals the unfused
# op (pq_rmsnorm / pq_silu_mul / pq_conv, each pinned to the oracle elsewhere)
# followed by pq_q8r_gemv, bit for bit, with the vectors the prologue writes
# once (the residual, the shifted conv ring) equal too.
@pytest.mark.parametrize("kind,N,K", [("resnorm", 3104, 2048), ("resnorm", 65536, 2048), ("resnorm", 300, 4096),
                                      ("norm", 6144, 2048), ("norm", 77, 1024), ("silu", 2048, 8192),
                                      ("silu", 2048, 4096), ("silu", 130, 2048), ("conv3", 2048, 2048),
                                      ("conv7", 2048, 2048), ("conv3", 1000, 4096), ("conv7", 1000, 4096),
                                      ("resnorm", 2052, 8192), ("norm", 4100, 8192), ("silu", 513, 1024),
                                      ("resnorm", 7, 1024)])
def test_q8r_gemv_fused(pq, dev, kind, N, K):
    print(f"q8r fused {kind} N={N} K={K}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(N * 7 + K)
    codes = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
    scales = torch.rand((N, K // 32), device=dev, generator=g) * 0.02
    bf = lambda *shape, s=1.0: (torch.randn(shape, device=dev, generator=g) * s).to(torch.bfloat16)
    out_dt = pq.DT_F32 if N == 65536 else pq.DT_BF16
    if kind == "resnorm":
        h, x = bf(K, s=30.0), bf(K, s=4.0)
        w0, w1 = torch.rand(K, device=dev, generator=g) + 0.5, torch.rand(K, device=dev, generator=g) + 0.5
        x1 = x.clone()
        xin, _, _ = pq.rmsnorm(x1, w0, h=h, w1=w1)
        want = pq.q8r_gemv(codes, scales, xin, out_dtype=out_dt)
        xo = torch.empty(K, dtype=torch.int16, device=dev)
        nparts = pq.lib().pq_q8r_gemv_parts(N)
        parts = torch.empty(2 * nparts, dtype=torch.float32, device=dev)
        y = pq.q8r_gemv_fused(codes, scales, pq.PRO_RESNORM, out_dtype=out_dt, parts=parts, h=h.view(torch.int16),
                              x_in=x.view(torch.int16), x_out=xo, w0=w0, w1=w1)
        assert torch.equal(xo, x1.view(torch.int16))
        if out_dt == pq.DT_F32:   # the per-workgroup pairs give pq_argmax's id over the fp32 outputs
            assert int(pq.argmax_parts(parts, nparts).item()) == int(pq.argmax(want).item())
    elif kind == "norm":
        x = bf(K, s=3.0)
        w0 = torch.rand(K, device=dev, generator=g) + 0.5
        xin, _, _ = pq.rmsnorm(x.clone(), w0)
        want = pq.q8r_gemv(codes, scales, xin, out_dtype=out_dt)
        y = pq.q8r_gemv_fused(codes, scales, pq.PRO_NORM, out_dtype=out_dt, x_in=x.view(torch.int16), w0=w0)
    elif kind == "silu":
        gu = bf(2 * K, s=3.0)
        xin, _, _ = pq.silu_mul(gu, K, 1)
        want = pq.q8r_gemv(codes, scales, xin.reshape(K), out_dtype=out_dt)
        y = pq.q8r_gemv_fused(codes, scales, pq.PRO_SILU, out_dtype=out_dt, gu=gu.view(torch.int16))
    else:
        nt = 7 if kind == "conv7" else 3
        bcx, ring = bf(3 * K, s=2.0), bf(nt * K, s=2.0)
        taps = torch.randn(K, nt, device=dev, generator=g) * 0.5
        ring1 = ring.clone()
        xin = torch.empty(K, dtype=torch.bfloat16, device=dev)
        pq.conv(ring1, taps, bcx, xin, K, 1, nt)
        want = pq.q8r_gemv(codes, scales, xin, out_dtype=out_dt)
        ring_out = torch.empty_like(ring)
        y = pq.q8r_gemv_fused(codes, scales, pq.PRO_CONV, out_dtype=out_dt, bcx=bcx.view(torch.int16),
                              ring_in=ring.view(torch.int16), ring_out=ring_out.view(torch.int16), taps=taps,
                              ntaps=nt)
        assert torch.equal(ring_out.view(torch.int16), ring1.view(torch.int16))
    torch.cuda.synchronize()
    if out_dt == pq.DT_F32:
        assert torch.equal(y.view(torch.int32), want.view(torch.int32))
    else:
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))


# The gate/up GEMV with the SwiGLU epilogue equals the unfused gate/up GEMV
# (bf16 out) followed by pq_silu_mul, bit for bit; F = 4 exercises a single
# tile, 8192 the tile walk over many row tiles per workgroup.
@pytest.mark.parametrize("kind,F,K", [("resnorm", 8192, 2048), ("resnorm", 7680, 2048), ("norm", 4, 2048),
                                      ("resnorm", 2052, 1024), ("resnorm", 2048, 8192), ("norm", 1000, 4096)])
def test_q8r_gemv_fused_swiglu(pq, dev, kind, F, K):
    print(f"q8r fused swiglu {kind} F={F} K={K}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(F * 3 + K)
    codes = torch.randint(-127, 128, (2 * F, K), dtype=torch.int8, device=dev, generator=g)
    scales = torch.rand((2 * F, K // 32), device=dev, generator=g) * 0.02
    bf = lambda n, s: (torch.randn(n, device=dev, generator=g) * s).to(torch.bfloat16)
    w0, w1 = torch.rand(K, device=dev, generator=g) + 0.5, torch.rand(K, device=dev, generator=g) + 0.5
    x = bf(K, 4.0)
    if kind == "resnorm":
        h = bf(K, 30.0)
        x1 = x.clone()
        xin, _, _ = pq.rmsnorm(x1, w0, h=h, w1=w1)
        xo = torch.empty(K, dtype=torch.int16, device=dev)
        y = pq.q8r_gemv_fused_swiglu(codes, scales, pq.PRO_RESNORM, h=h, x_in=x, x_out=xo, w0=w0, w1=w1)
    else:
        xin, _, _ = pq.rmsnorm(x.clone(), w0)
        y = pq.q8r_gemv_fused_swiglu(codes, scales, pq.PRO_NORM, x_in=x, w0=w0)
    gu = pq.q8r_gemv(codes, scales, xin)
    Fp = (F + 255) // 256 * 256   # pq_silu_mul takes F a multiple of 256: zero-pad gate and up
    gup = torch.zeros(2 * Fp, dtype=torch.bfloat16, device=dev)
    gup[:F], gup[Fp:Fp + F] = gu[:F], gu[F:]
    want, _, _ = pq.silu_mul(gup, Fp, 1)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), want.reshape(Fp)[:F].view(torch.int16))
    if kind == "resnorm":
        assert torch.equal(xo, x1.view(torch.int16))


# The EMBED prologue on the row-major table (the R2 decode step's layer 0):
# x_out = pq_embed_rows' row of *tok (zeros for an id outside the table) and the
# GEMV of its RMSNorm, bit for bit against pq_embed_rows + pq_rmsnorm + pq_q8r_gemv.
@pytest.mark.parametrize("K", [2048, 1024, 4096, 8192])
def test_q8r_gemv_fused_embed(pq, dev, K):
    import ctypes as C
    g = torch.Generator(device=dev)
    g.manual_seed(K + 5)
    N, vocab = 3000, 1000
    codes = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
    scales = torch.rand((N, K // 32), device=dev, generator=g) * 0.02
    ec = torch.randint(-127, 128, (vocab, K), dtype=torch.int8, device=dev, generator=g)
    es = torch.rand((vocab, K // 32), device=dev, generator=g) * 0.05
    w0 = torch.rand(K, device=dev, generator=g) + 0.5
    for tok in (0, vocab - 1, 123, -1, vocab):
        print(f"q8r fused embed K={K} tok={tok}", flush=True)
        t = torch.tensor([tok], dtype=torch.int32, device=dev)
        row = torch.empty(K, dtype=torch.int16, device=dev)
        pq.check(pq.lib().pq_embed_rows(C.c_void_p(ec.data_ptr()), C.c_void_p(es.data_ptr()), C.c_void_p(t.data_ptr()),
                                        C.c_void_p(row.data_ptr()), K, vocab, 1, C.c_void_p(pq.stream_ptr())),
                 "pq_embed_rows")
        xin, _, _ = pq.rmsnorm(row.view(torch.bfloat16).clone(), w0)
        want = pq.q8r_gemv(codes, scales, xin)
        xo = torch.full((K,), 0x7fff, dtype=torch.int16, device=dev)
        y = pq.q8r_gemv_fused(codes, scales, pq.PRO_EMBED, tok=t, emb_rows=(ec, es), x_out=xo, w0=w0, vocab=vocab)
        torch.cuda.synchronize()
        assert torch.equal(xo, row), tok
        assert torch.equal(y.view(torch.int16), want.view(torch.int16)), tok
