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


@pytest.mark.parametrize("N,K", [(12288, 4096), (4096, 12288), (37, 9728), (61, 2560), (3, 256)])
def test_tq2_gemv(orc, pq, dev, N, K):
    codes = orc.gen_ternary(N + K, N * K // 4).reshape(N, K // 4)
    S = orc.gen_scales(N + K + 1, N * K // 128).reshape(N, K // 128)
    x = orc.gen_normal(N + K + 2, K)
    xq = orc.q8k_quant(x)
    want = orc.tq2_gemv(codes, S, xq, N, K)
    xqd = pq.q8k_quant(torch.from_numpy(x).to(dev))
    y = pq.tq2_gemv(torch.from_numpy(codes).to(dev), torch.from_numpy(S.view(np.int16)).to(dev), xqd, N, K)
    got = y.cpu().numpy()
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:4]}"


def test_tq2_golden(pq, dev):
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "kernels.npz"))
    N, K = d["t_y"].size, d["t_x"].size
    y = pq.tq2_gemv(torch.from_numpy(d["t_codes"]).to(dev), torch.from_numpy(d["t_S"].view(np.int16)).to(dev),
                    torch.from_numpy(d["t_xq"]).to(dev), N, K)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), d["t_y"].view(np.uint32))
