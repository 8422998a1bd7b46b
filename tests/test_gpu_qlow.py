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
