"""GPU parity: Q8_0 quantizer, packed decode GEMV and MFMA prefill GEMM vs the oracle.

Integer work (codes, isum) and every fp32/bf16 output are compared bit for bit
(the R1 order is shared by the kernels and the oracle).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SEED = 20261201


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a.view(np.uint16)


def _weights(orc, pq, dev, N, K, seed):
    W, S = orc.q8_weights(seed, N, K)
    w = pq.Q8Weight(torch.from_numpy(W).to(dev), torch.from_numpy(S.view(np.int16)).to(dev))
    return W, S, w


@pytest.mark.parametrize("T,K", [(1, 2048), (3, 96), (16, 8192), (5, 32)])
def test_quant_f32(orc, pq, dev, T, K):
    print(f"quant_f32 T={T} K={K}", flush=True)
    x = orc.gen_normal(SEED + K + T, T * K).reshape(T, K)
    x[0, :32] = 0.0                            # all-zero block -> d = 0, q = 0
    if K >= 64:
        x[0, 32:64] *= 1e-30                   # subnormal-range block
    qx_r, dx_r = orc.q8_quant(x)
    qx, dx = pq.q8_quant(torch.from_numpy(x).to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(qx.cpu().numpy(), qx_r)
    assert np.array_equal(_bits(dx.cpu().numpy()), _bits(dx_r))


def test_quant_bf16(orc, pq, dev):
    T, K = 4, 2048
    x = orc.gen_normal(SEED + 7, T * K).reshape(T, K) * 30.0
    xb = orc.f2bf(x)
    qx_r, dx_r = orc.q8_quant_bf16(xb)
    qx, dx = pq.q8_quant(torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16))
    torch.cuda.synchronize()
    assert np.array_equal(qx.cpu().numpy(), qx_r)
    assert np.array_equal(_bits(dx.cpu().numpy()), _bits(dx_r))


GEMV_SHAPES = [
    (64, 2048), (97, 96), (1, 32), (130, 288),      # odd rows, partial tiles, partial chunks
    (8192, 2048),                                    # single Q8_0 GEMV workload
    (3104, 2048), (2048, 2048), (16384, 2048),       # fused q|k|v|gate, o_proj, gate+up
    (2048, 8192),                                    # down projection (split-K across workgroups)
    (6144, 2048),                                    # conv in_proj
    # the reference's own K set (q8_gemv_neon_test.c:152-157: N = 256 for K <= 128, else 97)
    (256, 32), (256, 64), (256, 96), (256, 128), (97, 2048), (97, 4096), (97, 7680),
]


@pytest.mark.parametrize("N,K", GEMV_SHAPES)
@pytest.mark.parametrize("bf16", [False, True])
def test_gemv_bitexact(orc, pq, dev, N, K, bf16):
    print(f"gemv N={N} K={K} bf16={bf16}", flush=True)
    W, S, w = _weights(orc, pq, dev, N, K, SEED + N + K)
    x = orc.gen_normal(SEED + 3 * N + K, K)
    qx_r, dx_r = orc.q8_quant(x)
    y_r = orc.q8_gemv(W, S, qx_r, dx_r)
    qx, dx = pq.q8_quant(torch.from_numpy(x).to(dev))
    y = pq.q8_gemv(w, qx, dx, out_dtype=pq.DT_BF16 if bf16 else pq.DT_F32)
    torch.cuda.synchronize()
    if bf16:
        got = y.view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got, orc.f2bf(y_r))
    else:
        got = y.cpu().numpy()
        bad = np.nonzero(_bits(got) != _bits(y_r))[0]
        assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}: {got[bad[:5]]} vs {y_r[bad[:5]]}"


def test_gemv_lm_head(orc, pq, dev):
    N, K = 65536, 2048
    print(f"gemv lm head N={N} K={K}", flush=True)
    W, S, w = _weights(orc, pq, dev, N, K, SEED + 99)
    x = orc.gen_normal(SEED + 98, K)
    qx_r, dx_r = orc.q8_quant(x)
    y_r = orc.q8_gemv(W, S, qx_r, dx_r)
    qx, dx = pq.q8_quant(torch.from_numpy(x).to(dev))
    y = pq.q8_gemv(w, qx, dx).cpu().numpy()
    assert np.array_equal(_bits(y), _bits(y_r))
    assert orc.argmax(y) == orc.argmax(y_r)


def test_gemv_repeat_and_inplace(orc, pq, dev):
    """Repeat calls agree and y may overwrite the buffer x was quantized from."""
    N, K = 2048, 8192
    W, S, w = _weights(orc, pq, dev, N, K, SEED + 5)
    x = orc.gen_normal(SEED + 6, K)
    qx_r, dx_r = orc.q8_quant(x)
    y_r = orc.q8_gemv(W, S, qx_r, dx_r)
    xt = torch.from_numpy(x).to(dev)
    for _ in range(3):
        qx, dx = pq.q8_quant(xt)
        y = pq.q8_gemv(w, qx, dx)
        assert np.array_equal(_bits(y.cpu().numpy()), _bits(y_r))
    # in place: the output buffer is the activation buffer it was quantized from
    buf = torch.zeros(K, dtype=torch.float32, device=dev)
    buf.copy_(xt)
    qx, dx = pq.q8_quant(buf)
    pq.q8_gemv(w, qx, dx, out=buf[:N])
    assert np.array_equal(_bits(buf[:N].cpu().numpy()), _bits(y_r))


@pytest.mark.parametrize("N,K,T", [(64, 2048, 1), (97, 96, 5), (130, 288, 33), (3104, 2048, 32),
                                   (2048, 8192, 32), (16384, 2048, 64), (2048, 2048, 77),
                                   (16384, 2048, 100), (16416, 2048, 40), (16384, 4096, 48),
                                   (16384, 2048, 512), (65536, 2048, 96),
                                   # the LFM3 shapes: FFN 7680 (gate+up 15360 rows, down K = 7680),
                                   # q|k|v|gate 3088 rows, vocab 128000
                                   (15360, 2048, 32), (2048, 7680, 32), (2048, 7680, 256), (3088, 2048, 100),
                                   (128000, 2048, 32)])
def test_gemm_bitexact(orc, pq, dev, N, K, T):
    print(f"gemm N={N} K={K} T={T}", flush=True)
    W, S, w = _weights(orc, pq, dev, N, K, SEED + 11 * N + K)
    x = orc.gen_normal(SEED + 13 * T + K, T * K).reshape(T, K)
    qx_r, dx_r = orc.q8_quant(x)
    y_r = orc.q8_gemm(W, S, qx_r, dx_r)
    qx, dx = pq.q8_quant(torch.from_numpy(x).to(dev))
    y = pq.q8_gemm(w, qx, dx).cpu().numpy()
    bad = np.argwhere(_bits(y) != _bits(y_r))
    assert bad.shape[0] == 0, f"{bad.shape[0]} cells differ, first {bad[:5].tolist()}"
    # without a workspace (no K split) the same bits
    y_ns = pq.q8_gemm(w, qx, dx, split=False).cpu().numpy()
    assert np.array_equal(_bits(y_ns), _bits(y_r))
    # batched == per-position T=1 GEMVs (prefill_chunk_test's invariant)
    yb = pq.q8_gemm(w, qx, dx, out_dtype=pq.DT_BF16)
    for t in range(0, T, max(1, T // 4)):
        y1 = pq.q8_gemv(w, qx[t], dx[t], out_dtype=pq.DT_BF16)
        assert torch.equal(y1.view(torch.int16), yb[t].view(torch.int16))
