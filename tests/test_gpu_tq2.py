"""GPU parity of the ternary PQ2_0 x Q8_K path: Q8_K quantizer and GEMV bit for bit
against the oracle (itself bit-equal to the reference's pq2_gemv_cpu)."""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("K,T", [(4096, 1), (12288, 1), (256, 3)])
def test_q8k_quant(orc, pq, dev, K, T):
    x = orc.gen_normal(K + T, T * K).reshape(T, K) * 3
    x[0, :256] = 0.0                              # all-zero block
    if K >= 512:
        x[0, 300] = x[0, 301] = -50.0             # ties for max|x|: the first index wins
    want = np.stack([orc.q8k_quant(x[t]) for t in range(T)])
    got = pq.q8k_quant(torch.from_numpy(x).to(dev)).cpu().numpy()
    assert np.array_equal(got, want)


# config-5 shapes, then the reference's parity set (bonsai2 pq1t_parity.c:71-74:
# 151669 x 2560 is the LM head, 1001 x 2560 an odd row count), then small ones
TQ2_SHAPES = [(12288, 4096), (4096, 12288),
              (6144, 2560), (2560, 4096), (19456, 2560), (2560, 9728), (151669, 2560), (1001, 2560), (37, 9728),
              (61, 2560), (3, 256)]


@pytest.mark.parametrize("N,K", TQ2_SHAPES)
def test_tq2_gemv(orc, pq, dev, N, K):
    print(f"tq2 N={N} K={K}", flush=True)
    codes = orc.gen_ternary(N + K, N * K // 4).reshape(N, K // 4)
    S = orc.gen_scales(N + K + 1, N * K // 128).reshape(N, K // 128)
    x = orc.gen_normal(N + K + 2, K)
    xq = orc.q8k_quant(x)
    want = orc.tq2_gemv(codes, S, xq, N, K)
    xqd = pq.q8k_quant(torch.from_numpy(x).to(dev))
    y = pq.tq2_gemv(torch.from_numpy(codes).to(dev), torch.from_numpy(S.view(np.int16)).to(dev), xqd, K, N)
    got = y.cpu().numpy()
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:4]}"


def test_tq2_golden(pq, dev):
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "kernels.npz"))
    N, K = d["t_y"].size, d["t_x"].size
    y = pq.tq2_gemv(torch.from_numpy(d["t_codes"]).to(dev), torch.from_numpy(d["t_S"].view(np.int16)).to(dev),
                    torch.from_numpy(d["t_xq"]).to(dev), K, N)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), d["t_y"].view(np.uint32))


@pytest.mark.parametrize("N,K", [(12288, 4096), (4096, 12288)])
def test_tq2_reference_call_order(orc, pq, dev, N, K):
    """The entry point called as pq2_parity.c:79 calls pq2_gemv_sm53_launch:
    (w_codes, w_scales_h, xq, y, K, rows, stream), returning 0."""
    import ctypes
    codes = orc.gen_ternary(7 * N + K, N * K // 4).reshape(N, K // 4)
    S = orc.gen_scales(7 * N + K + 1, N * K // 128).reshape(N, K // 128)
    x = orc.gen_normal(7 * N + K + 2, K)
    xq = orc.q8k_quant(x)
    d_cd, d_sc = torch.from_numpy(codes).to(dev), torch.from_numpy(S.view(np.int16)).to(dev)
    d_xq = torch.from_numpy(xq).to(dev)
    d_y = torch.zeros(N, dtype=torch.float32, device=dev)
    rows = N
    rc = pq.lib().pq_tq2_gemv(ctypes.c_void_p(d_cd.data_ptr()), ctypes.c_void_p(d_sc.data_ptr()),
                              ctypes.c_void_p(d_xq.data_ptr()), ctypes.c_void_p(d_y.data_ptr()), K, rows, None)
    torch.cuda.synchronize()
    assert rc == 0
    assert np.array_equal(d_y.cpu().numpy().view(np.uint32), orc.tq2_gemv(codes, S, xq, N, K).view(np.uint32))
    # K that is not a multiple of 256 is refused with a negative status
    assert pq.lib().pq_tq2_gemv(ctypes.c_void_p(d_cd.data_ptr()), ctypes.c_void_p(d_sc.data_ptr()),
                                ctypes.c_void_p(d_xq.data_ptr()), ctypes.c_void_p(d_y.data_ptr()), 100, rows, None) < 0


# one launch over several tensors of one K: each tensor's rows give the oracle's
# bits (row counts that do and do not fill whole workgroups, one to three
# tensors; tensors of equal row count share workgroups, the others do not)
@pytest.mark.parametrize("rows,K", [((12288, 12288), 4096), ((2048, 512, 512), 4096), ((61, 1001, 37), 2560),
                                    ((4096,), 12288), ((3, 5), 256), ((1000, 1000, 1000), 4096),
                                    ((77, 77), 12288), ((33, 33), 256), ((500, 500, 500), 2560)])
def test_tq2_gemv_batch(orc, pq, dev, rows, K):
    print(f"tq2 batch rows={rows} K={K}", flush=True)
    x = orc.gen_normal(K + 7, K)
    xq = orc.q8k_quant(x)
    xqd = pq.q8k_quant(torch.from_numpy(x).to(dev))
    host, dev_t = [], []
    for i, N in enumerate(rows):
        codes = orc.gen_ternary(N + K + 11 * i, N * K // 4).reshape(N, K // 4)
        S = orc.gen_scales(N + K + 11 * i + 1, N * K // 128).reshape(N, K // 128)
        host.append((codes, S, N))
        dev_t.append((torch.from_numpy(codes).to(dev), torch.from_numpy(S.view(np.int16)).to(dev)))
    ys = pq.tq2_gemv_batch(dev_t, xqd, K)
    torch.cuda.synchronize()
    for (codes, S, N), y in zip(host, ys):
        want = orc.tq2_gemv(codes, S, xq, N, K)
        assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32)), N
