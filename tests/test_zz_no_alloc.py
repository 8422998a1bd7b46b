"""The allocation-free GEMM (pq_q8_gemm_noalloc) against pq_q8_gemm_ws with a
caller workspace: the same bits, through the C ABI, on two calls in a row (the
second smaller, so it runs on the first call's leftover scratch contents)."""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

PQ_ERR_WORKSPACE = -3


def _case(orc, pq, dev, N, K, T, seed):
    W, S = orc.q8_weights(seed, N, K)
    w = pq.Q8Weight(torch.from_numpy(W).to(dev), torch.from_numpy(S.view(np.int16)).to(dev))
    x = orc.gen_normal(seed + 1, T * K).reshape(T, K)
    qx, dx = pq.q8_quant(torch.from_numpy(x).to(dev))
    return w, qx, dx


def _ptr(t):
    return C.c_void_p(t.data_ptr())


def _noalloc(pq, w, qx, dx, N, K, T):
    y = torch.full((T, N), float("nan"), dtype=torch.float32, device=qx.device)
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = pq.lib().pq_q8_gemm_noalloc(_ptr(w.pcodes), _ptr(w.pscales), _ptr(qx), _ptr(dx), _ptr(y), pq.DT_F32, N, K, T, stream)
    return rc, y


def _with_ws(pq, w, qx, dx, N, K, T):
    L = pq.lib()
    nbytes = L.pq_q8_gemm_workspace_bytes(N, K, T)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=qx.device)
    y = torch.full((T, N), float("nan"), dtype=torch.float32, device=qx.device)
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.pq_q8_gemm_ws(_ptr(w.pcodes), _ptr(w.pscales), _ptr(qx), _ptr(dx), _ptr(y), pq.DT_F32, N, K, T, _ptr(ws), nbytes,
                         stream)
    assert rc == 0, L.pq_last_error()
    return nbytes, y


def test_noalloc_matches_workspace_form(orc, pq, dev):
    L = pq.lib()
    cap = L.pq_q8_gemm_scratch_bytes()
    assert cap == 16 << 20
    # down projection at a 32-position chunk (K split over 32 chunks: 8 MiB of
    # partials), then a smaller split shape, then one that needs no split
    for N, K, T, seed in ((2048, 8192, 32, 11), (2048, 4096, 8, 12), (1024, 1024, 3, 13)):
        print(f"noalloc N={N} K={K} T={T}", flush=True)
        w, qx, dx = _case(orc, pq, dev, N, K, T, seed)
        need, y_ref = _with_ws(pq, w, qx, dx, N, K, T)
        assert need <= cap
        rc, y = _noalloc(pq, w, qx, dx, N, K, T)
        torch.cuda.synchronize()
        assert rc == 0, L.pq_last_error()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), y_ref.cpu().numpy().view(np.uint32))
        if T <= 8:   # and the oracle, on the smaller cases
            W, S = orc.q8_weights(seed, N, K)
            x = orc.gen_normal(seed + 1, T * K).reshape(T, K)
            want = orc.q8_gemm(W, S, *orc.q8_quant(x))
            assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_noalloc_refuses_what_does_not_fit(orc, pq, dev):
    L = pq.lib()
    N, K, T = 4096, 16384, 32          # 64 chunks x 32 positions x 4096 rows x 4 B = 32 MiB of partials
    assert L.pq_q8_gemm_workspace_bytes(N, K, T) > L.pq_q8_gemm_scratch_bytes()
    dummy = torch.zeros(64, dtype=torch.uint8, device=dev)
    p = _ptr(dummy)
    rc = L.pq_q8_gemm_noalloc(p, p, p, p, p, pq.DT_F32, N, K, T, None)
    assert rc == PQ_ERR_WORKSPACE
    assert b"scratch" in L.pq_last_error()


def test_noalloc_under_graph_capture(orc, pq, dev):
    """Calls captured into a HIP graph after one eager call on the device (which
    looks up the scratch array's address): two split shapes back to back in one
    graph, replayed three times with eager work between the replays, each replay
    bit-equal to pq_q8_gemm_ws."""
    L = pq.lib()
    cases = [(2048, 8192, 32, 31), (2048, 4096, 8, 32)]
    data = [_case(orc, pq, dev, N, K, T, seed) for (N, K, T, seed) in cases]
    refs = [_with_ws(pq, w, qx, dx, N, K, T)[1] for (w, qx, dx), (N, K, T, _) in zip(data, cases)]
    rc, _ = _noalloc(pq, *data[0], *cases[0][:3])   # outside capture: resolves the address
    assert rc == 0, L.pq_last_error()
    ys = [torch.full((T, N), float("nan"), dtype=torch.float32, device=dev) for (N, K, T, _) in cases]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    rcs = []
    with torch.cuda.graph(g):
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        for (w, qx, dx), (N, K, T, _), y in zip(data, cases, ys):
            rcs.append(L.pq_q8_gemm_noalloc(_ptr(w.pcodes), _ptr(w.pscales), _ptr(qx), _ptr(dx), _ptr(y), pq.DT_F32,
                                            N, K, T, stream))
    assert rcs == [0, 0], L.pq_last_error()
    for rep in range(3):
        print(f"noalloc graph replay {rep}", flush=True)
        for y in ys:
            y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for y, r in zip(ys, refs):
            assert np.array_equal(y.cpu().numpy().view(np.uint32), r.cpu().numpy().view(np.uint32)), rep
        # eager work between replays, on the same scratch array
        rc, _ = _noalloc(pq, *data[1], *cases[1][:3])
        assert rc == 0, L.pq_last_error()
        torch.cuda.synchronize()
