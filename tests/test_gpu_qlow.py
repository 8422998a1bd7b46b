"""GPU parity: the Q4 / Q5 low-bit GEMV (pq_qlow_gemv, the reference's order)
against the oracle's restatement, bit for bit, and the packed payload against
the tiled layout lfm3_qlow.cuh:5-13 describes (written here in numpy)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(orc, N, K, bits, seed):
    rng = np.random.default_rng(seed)
    Q = rng.integers(0, 2 ** bits, (N, K)).astype(np.uint8)
    d = (np.abs(rng.standard_normal((N, K // 32))) * 0.02 * 128).astype(np.float16)
    mn = (-rng.random((N, K // 32)) * 0.3).astype(np.float16)
    S = np.stack([d.view(np.uint16), mn.view(np.uint16)], -1)
    xb = orc.f2bf(orc.gen_normal(seed + 1, K) * 2.0)
    return Q, S, xb


def _ref_layout(Q, S, bits):
    from qlow_layout import pack
    return pack(Q, S, bits)


@pytest.mark.parametrize("bits,N,K", [(4, 2048, 2048), (5, 2048, 2048), (4, 2048, 8192), (5, 4096, 4096),
                                      (4, 96, 256), (5, 64, 16384), (4, 16384, 2048)])
def test_qlow_gemv_bitexact(orc, pq, dev, bits, N, K):
    print(f"qlow bits={bits} N={N} K={K}", flush=True)
    Q, S, xb = _case(orc, N, K, bits, 900 + N + K + bits)
    w = pq.QlowWeight(torch.from_numpy(Q).to(dev), torch.from_numpy(S.view(np.int16)).to(dev), bits)
    x = torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16)
    want = orc.qlow_gemv(Q, S, xb)
    y = pq.qlow_gemv(w, x, out_dtype=pq.DT_F32)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
    yb = pq.qlow_gemv(w, x).cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(yb, orc.f2bf(want))
    # without a workspace (every K slice in one workgroup) the same bits: a
    # whole row's staging (x, group sums, 8 rows' partials and scales: 49
    # floats per 32-group) fits LDS up to the largest K, 16384
    y1 = pq.qlow_gemv(w, x, out_dtype=pq.DT_F32, split=False)
    assert np.array_equal(y1.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bits", [4, 5])
def test_qlow_layout_is_the_references(orc, pq, dev, bits):
    """pq_qlow_pack writes the documented tiled payload byte for byte, and the
    GEMV reads a payload laid out that way independently of the pack."""
    N, K = 64, 512
    Q, S, xb = _case(orc, N, K, bits, 77 + bits)
    codes, sc = _ref_layout(Q, S, bits)
    w = pq.QlowWeight(torch.from_numpy(Q).to(dev), torch.from_numpy(S.view(np.int16)).to(dev), bits)
    assert np.array_equal(w.pcodes.cpu().numpy(), codes)
    assert np.array_equal(w.pscales.cpu().numpy().view(np.uint16), sc)
    w.pcodes = torch.from_numpy(codes).to(dev)
    w.pscales = torch.from_numpy(sc.view(np.int16)).to(dev)
    x = torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16)
    y = pq.qlow_gemv(w, x, out_dtype=pq.DT_F32).cpu().numpy()
    assert np.array_equal(y.view(np.uint32), orc.qlow_gemv(Q, S, xb).view(np.uint32))


def test_qlow_rejects_bad_shapes(pq, dev):
    with pytest.raises(ValueError):
        pq.QlowWeight(torch.zeros((40, 256), dtype=torch.uint8, device=dev),
                      torch.zeros((40, 8, 2), dtype=torch.int16, device=dev), 4)


# The Q4 / Q5 GEMV with x from a prologue equals the unfused op (pq_rmsnorm /
# pq_silu_mul / pq_conv, each pinned to the oracle elsewhere) followed by
# pq_qlow_gemv, bit for bit, with the vectors the prologue writes once (the
# residual, the shifted conv ring) equal too. The shapes cover the three
# per-thread widths (K = 2048, 4096, 8192) and the three rows-per-workgroup
# slices (N = 16384, 3072, 2048).
@pytest.mark.parametrize("kind,bits,N,K", [("resnorm", 4, 3072, 2048), ("resnorm", 5, 16384, 2048),
                                           ("resnorm", 4, 2048, 8192), ("norm", 5, 2048, 2048),
                                           ("norm", 4, 4096, 4096), ("silu", 4, 2048, 8192),
                                           ("silu", 5, 3072, 4096), ("conv3", 4, 2048, 2048),
                                           ("conv7", 5, 2048, 2048), ("conv3", 5, 1024, 4096),
                                           ("conv7", 4, 3072, 4096)])
def test_qlow_gemv_fused(orc, pq, dev, kind, bits, N, K):
    print(f"qlow fused {kind} bits={bits} N={N} K={K}", flush=True)
    Q, S, _ = _case(orc, N, K, bits, 31 * N + K + bits)
    w = pq.QlowWeight(torch.from_numpy(Q).to(dev), torch.from_numpy(S.view(np.int16)).to(dev), bits)
    g = torch.Generator(device=dev)
    g.manual_seed(N + 3 * K + bits)
    bf = lambda *shape, s=1.0: (torch.randn(shape, device=dev, generator=g) * s).to(torch.bfloat16)
    out_dt = pq.DT_F32 if N == 16384 else pq.DT_BF16
    if kind == "resnorm":
        h, x = bf(K, s=30.0), bf(K, s=4.0)
        w0, w1 = torch.rand(K, device=dev, generator=g) + 0.5, torch.rand(K, device=dev, generator=g) + 0.5
        x1 = x.clone()
        xin, _, _ = pq.rmsnorm(x1, w0, h=h, w1=w1)
        want = pq.qlow_gemv(w, xin, out_dtype=out_dt)
        xo = torch.empty(K, dtype=torch.int16, device=dev)
        y = pq.qlow_gemv_fused(w, pq.PRO_RESNORM, out_dtype=out_dt, h=h.view(torch.int16), x_in=x.view(torch.int16),
                               x_out=xo, w0=w0, w1=w1)
        torch.cuda.synchronize()
        assert torch.equal(xo, x1.view(torch.int16))
    elif kind == "norm":
        x = bf(K, s=3.0)
        w0 = torch.rand(K, device=dev, generator=g) + 0.5
        xin, _, _ = pq.rmsnorm(x.clone(), w0)
        want = pq.qlow_gemv(w, xin, out_dtype=out_dt)
        y = pq.qlow_gemv_fused(w, pq.PRO_NORM, out_dtype=out_dt, x_in=x.view(torch.int16), w0=w0)
    elif kind == "silu":
        gu = bf(2 * K, s=3.0)
        xin, _, _ = pq.silu_mul(gu, K, 1)
        want = pq.qlow_gemv(w, xin.reshape(K), out_dtype=out_dt)
        y = pq.qlow_gemv_fused(w, pq.PRO_SILU, out_dtype=out_dt, gu=gu.view(torch.int16))
    else:
        nt = 7 if kind == "conv7" else 3
        bcx, ring = bf(3 * K, s=2.0), bf(nt * K, s=2.0)
        taps = torch.randn(K, nt, device=dev, generator=g) * 0.5
        ring1 = ring.clone()
        xin = torch.empty(K, dtype=torch.bfloat16, device=dev)
        pq.conv(ring1, taps, bcx, xin, K, 1, nt)
        want = pq.qlow_gemv(w, xin, out_dtype=out_dt)
        ring_out = torch.empty_like(ring)
        y = pq.qlow_gemv_fused(w, pq.PRO_CONV, out_dtype=out_dt, bcx=bcx.view(torch.int16),
                               ring_in=ring.view(torch.int16), ring_out=ring_out.view(torch.int16), taps=taps,
                               ntaps=nt)
        torch.cuda.synchronize()
        assert torch.equal(ring_out.view(torch.int16), ring1.view(torch.int16))
    torch.cuda.synchronize()
    if out_dt == pq.DT_F32:
        assert torch.equal(y.view(torch.int32), want.view(torch.int32))
    else:
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))


# The gate/up GEMV with the SwiGLU epilogue equals pq_rmsnorm, pq_qlow_gemv of
# the 2F rows (bf16) and pq_silu_mul, bit for bit. F covers the three rows per
# half (8: F=1024 and 1056, 16: F=3072, 32: F=8192 and 16384 at K=2048, halved
# to 16 at K=4096), a tile count that is not a multiple of 8 (F=1056), both K
# slice counts and the three per-thread prologue widths.
@pytest.mark.parametrize("kind,bits,F,K", [("resnorm", 4, 8192, 2048), ("resnorm", 5, 1024, 4096),
                                           ("norm", 4, 3072, 8192), ("norm", 5, 16384, 2048),
                                           ("resnorm", 4, 16384, 4096), ("norm", 4, 1056, 2048)])
def test_qlow_gemv_fused_swiglu(orc, pq, dev, kind, bits, F, K):
    print(f"qlow swiglu {kind} bits={bits} F={F} K={K}", flush=True)
    Q, S, _ = _case(orc, 2 * F, K, bits, 7 * F + K + bits)
    w = pq.QlowWeight(torch.from_numpy(Q).to(dev), torch.from_numpy(S.view(np.int16)).to(dev), bits)
    g = torch.Generator(device=dev)
    g.manual_seed(F + 5 * K + bits)
    bf = lambda *shape, s=1.0: (torch.randn(shape, device=dev, generator=g) * s).to(torch.bfloat16)
    x = bf(K, s=4.0)
    w0, w1 = torch.rand(K, device=dev, generator=g) + 0.5, torch.rand(K, device=dev, generator=g) + 0.5
    if kind == "resnorm":
        h = bf(K, s=30.0)
        x1 = x.clone()
        xin, _, _ = pq.rmsnorm(x1, w0, h=h, w1=w1)
        xo = torch.empty(K, dtype=torch.int16, device=dev)
        y = pq.qlow_gemv_fused_swiglu(w, pq.PRO_RESNORM, h=h.view(torch.int16), x_in=x.view(torch.int16), x_out=xo,
                                      w0=w0, w1=w1)
        torch.cuda.synchronize()
        assert torch.equal(xo, x1.view(torch.int16))
    else:
        xin, _, _ = pq.rmsnorm(x.clone(), w0)
        y = pq.qlow_gemv_fused_swiglu(w, pq.PRO_NORM, x_in=x.view(torch.int16), w0=w0)
    gu = pq.qlow_gemv(w, xin, out_dtype=pq.DT_BF16)
    # pq_silu_mul takes F a multiple of 256: gate and up each padded with zeros
    # (an elementwise op; the first F outputs are the ones wanted)
    Fp = -(-F // 256) * 256
    gp = torch.zeros(2 * Fp, dtype=torch.bfloat16, device=dev)
    gp[:F], gp[Fp:Fp + F] = gu[:F], gu[F:]
    want, _, _ = pq.silu_mul(gp, Fp, 1)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), want.reshape(Fp)[:F].view(torch.int16))


def test_qlow_gemv_fused_rejects(pq, dev):
    """Shapes and kinds the fused form does not take fail with an error."""
    w = pq.QlowWeight(torch.zeros((64, 1024), dtype=torch.uint8, device=dev),
                      torch.zeros((64, 32, 2), dtype=torch.int16, device=dev), 4)
    x = torch.zeros(1024, dtype=torch.int16, device=dev)
    w0 = torch.ones(1024, device=dev)
    with pytest.raises(pq.PQError, match="K 2048, 4096 or 8192"):
        pq.qlow_gemv_fused(w, pq.PRO_NORM, x_in=x, w0=w0)
    w2 = pq.QlowWeight(torch.zeros((64, 2048), dtype=torch.uint8, device=dev),
                       torch.zeros((64, 64, 2), dtype=torch.int16, device=dev), 4)
    with pytest.raises(pq.PQError, match="prologue kind"):
        pq.qlow_gemv_fused(w2, pq.PRO_F32, xf=torch.zeros(2048, device=dev))
    with pytest.raises(pq.PQError, match="RESNORM or NORM"):
        pq.qlow_gemv_fused_swiglu(w2, pq.PRO_SILU, gu=torch.zeros(4096, dtype=torch.int16, device=dev))


# T positions in one launch equal the per-position GEMV row by row, bit for
# bit: every position-block size (T = 1, 3, 8, 33, 100) and the three K forms
# (2048: 8 positions per workgroup, 4096: 4, 8192: 2), with the outputs
# written at a row stride wider than N.
@pytest.mark.parametrize("bits,N,K,T", [(4, 3072, 2048, 33), (5, 16384, 2048, 8), (4, 2048, 8192, 100),
                                        (5, 2048, 4096, 3), (4, 96, 256, 40), (5, 2048, 2048, 1),
                                        (4, 64, 16384, 5)])
def test_qlow_gemm_equals_gemv(orc, pq, dev, bits, N, K, T):
    print(f"qlow gemm bits={bits} N={N} K={K} T={T}", flush=True)
    Q, S, _ = _case(orc, N, K, bits, 5 * N + K + T + bits)
    w = pq.QlowWeight(torch.from_numpy(Q).to(dev), torch.from_numpy(S.view(np.int16)).to(dev), bits)
    g = torch.Generator(device=dev)
    g.manual_seed(N + K + T)
    X = (torch.randn((T, K), device=dev, generator=g) * 2.0).to(torch.bfloat16)
    X[T // 2] = 0.0                                   # a zero row
    wide = torch.full((T, N + 40), float("nan"), dtype=torch.float32, device=dev)
    y = pq.qlow_gemm(w, X, out_dtype=pq.DT_F32, out=wide[:, :N])
    yb = pq.qlow_gemm(w, X)
    torch.cuda.synchronize()
    for t in range(T):
        want = pq.qlow_gemv(w, X[t], out_dtype=pq.DT_F32)
        assert torch.equal(y[t].view(torch.int32), want.view(torch.int32)), t
        assert torch.equal(yb[t].view(torch.int16), pq.qlow_gemv(w, X[t]).view(torch.int16)), t
    assert torch.isnan(wide[:, N:]).all()            # nothing written past N in a row
    if T <= 8:   # the oracle on the first rows
        for t in range(T):
            xb = X[t].view(torch.int16).cpu().numpy().view(np.uint16)
            assert np.array_equal(y[t].cpu().numpy().view(np.uint32), orc.qlow_gemv(Q, S, xb).view(np.uint32))
