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
# and 80 blocks (leaves with several blocks, codes widened per use)
@pytest.mark.parametrize("N,K,T", [(8192, 2048, 1), (3072, 2048, 1), (2048, 8192, 1), (97, 7680, 2),
                                   (61, 512, 1), (37, 1024, 3), (13, 32, 1), (65, 12288, 1), (45, 2560, 2),
                                   (2048, 2048, 4), (300, 2048, 40), (77, 8192, 33), (97, 7680, 9),
                                   (64, 12288, 5), (45, 2560, 17)])
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
