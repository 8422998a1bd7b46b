"""GPU parity of the layer kernels (norms, q/k prep, attention, conv, silu, argmax,
embedding) against the oracle: bf16 / fp16 / int8 outputs compared bit for bit."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SEED = 777


def _t16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


def _u16(t):
    return t.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("H,T", [(2048, 1), (2048, 5), (256, 3), (8192, 2)])
def test_rmsnorm_plain_and_quant(orc, pq, dev, H, T):
    x = orc.f2bf(orc.gen_normal(SEED + H, T * H).reshape(T, H) * 7)
    w = orc.gen_affine(SEED + 1, H, 1.0, 0.1)
    want = orc.rmsnorm(x, w)
    qx_r, dx_r = orc.q8_quant_bf16(want)
    y, qx, dx = pq.rmsnorm(_t16(x, dev), torch.from_numpy(w).to(dev), quant=True)
    assert np.array_equal(_u16(y), want)
    assert np.array_equal(qx.cpu().numpy(), qx_r)
    assert np.array_equal(dx.cpu().numpy().view(np.uint32), dx_r.view(np.uint32))


def test_rmsnorm_residual(orc, pq, dev):
    H, T = 2048, 3
    x = orc.f2bf(orc.gen_normal(SEED + 2, T * H).reshape(T, H) * 5)
    h = orc.f2bf(orc.gen_normal(SEED + 3, T * H).reshape(T, H) * 40)
    w0 = orc.gen_affine(SEED + 4, H, 4.0, 0.4)
    w1 = orc.gen_affine(SEED + 5, H, 1.0, 0.1)
    h3 = orc.rmsnorm(h, w0)
    xn = orc.add(x, h3)
    want = orc.rmsnorm(xn, w1)
    xd = _t16(x, dev)
    y, qx, dx = pq.rmsnorm(xd, torch.from_numpy(w0).to(dev), h=_t16(h, dev), w1=torch.from_numpy(w1).to(dev),
                           quant=True)
    assert np.array_equal(_u16(xd), xn)
    assert np.array_equal(_u16(y), want)
    assert np.array_equal(qx.cpu().numpy(), orc.q8_quant_bf16(want)[0])


def _qkv_case(orc, nh, nkv, hd, T, ctx, seed):
    nin = nh * hd + 2 * nkv * hd + nh
    rows = orc.f2bf(orc.gen_normal(seed, T * nin).reshape(T, nin) * 30)
    qn = orc.gen_affine(seed + 1, hd, 1.0, 0.1)
    kn = orc.gen_affine(seed + 2, hd, 1.0, 0.1)
    cs = orc.rope_table(ctx, hd, 32, 1e6)
    return nin, rows, qn, kn, cs


@pytest.mark.parametrize("pos0,T,hd,rot,theta", [(0, 1, 64, 32, 1e6), (77, 1, 64, 32, 1e6), (100, 9, 64, 32, 1e6),
                                                  (2000, 3, 64, 32, 1e6),
                                                  # head_dim 128: full attention (half rotated, theta 1e6)
                                                  # and sliding attention (all rotated, theta 1e4)
                                                  (0, 1, 128, 64, 1e6), (300, 5, 128, 64, 1e6),
                                                  (257, 3, 128, 128, 1e4), (4000, 2, 128, 128, 1e4)])
def test_qk_prep(orc, pq, dev, pos0, T, hd, rot, theta):
    nh, nkv, ctx = (32, 8, 2048) if hd == 64 else (16, 4, 4096)
    nin, rows, qn, kn, _ = _qkv_case(orc, nh, nkv, hd, T, 2, SEED + pos0)
    cs = orc.rope_table(ctx, hd, rot, theta)
    kvd = nkv * hd
    want_rows = rows.copy()
    kc_r = np.zeros((ctx, kvd), np.uint16)
    vc_r = np.zeros((ctx, kvd), np.uint16)
    for t in range(T):
        r = want_rows[t]
        q = orc.headnorm(r[:nh * hd], qn, nh, hd)
        k = orc.headnorm(r[nh * hd:nh * hd + kvd], kn, nkv, hd)
        q = orc.rope(q, cs, pos0 + t, nh, hd, rot)
        k = orc.rope(k, cs, pos0 + t, nkv, hd, rot)
        r[:nh * hd] = q
        kc_r[pos0 + t] = orc.bf2f(k).astype(np.float16).view(np.uint16)
        vc_r[pos0 + t] = orc.bf2f(r[nh * hd + kvd:nh * hd + 2 * kvd]).astype(np.float16).view(np.uint16)
    qkv = _t16(rows, dev)
    kc = torch.zeros((ctx, kvd), dtype=torch.int16, device=dev)
    vc = torch.zeros((ctx, kvd), dtype=torch.int16, device=dev)
    pq.qk_prep(qkv, nin, torch.from_numpy(qn).to(dev), torch.from_numpy(kn).to(dev), torch.from_numpy(cs).to(dev),
               kc, vc, pos0, nh, nkv, hd, rot, T)
    got = _u16(qkv)
    assert np.array_equal(got[:, :nh * hd], want_rows[:, :nh * hd])
    assert np.array_equal(_u16(kc), kc_r) and np.array_equal(_u16(vc), vc_r)


@pytest.mark.parametrize("npos_last,T,nh,nkv,hd,win", [
    (1, 1, 32, 8, 64, 0), (64, 1, 32, 8, 64, 0), (65, 1, 32, 8, 64, 0), (300, 1, 32, 8, 64, 0),
    (2048, 1, 32, 8, 64, 0), (40, 33, 32, 8, 64, 0), (130, 7, 8, 8, 64, 0), (70, 2, 16, 2, 64, 0),
    # head_dim 128 (16 q / 4 kv heads), full and sliding-window (256) layers
    (1, 1, 16, 4, 128, 0), (300, 1, 16, 4, 128, 0), (129, 40, 16, 4, 128, 0),
    (300, 1, 16, 4, 128, 256), (257, 1, 16, 4, 128, 256), (2000, 1, 16, 4, 128, 256),
    (330, 90, 16, 4, 128, 256), (200, 20, 8, 8, 64, 100), (90, 5, 16, 4, 128, 1)])
def test_attention(orc, pq, dev, npos_last, T, nh, nkv, hd, win):
    pos0 = npos_last - T
    kvd = nkv * hd
    q = orc.f2bf(orc.gen_normal(SEED + 9 * npos_last, T * nh * hd).reshape(T, nh * hd) * 2)
    gate = orc.f2bf(orc.gen_normal(SEED + 9 * npos_last + 1, T * nh).reshape(T, nh) * 3)
    kc = (orc.gen_normal(SEED + 9 * npos_last + 2, npos_last * kvd) * 2).astype(np.float16).view(np.uint16)
    vc = (orc.gen_normal(SEED + 9 * npos_last + 3, npos_last * kvd) * 5).astype(np.float16).view(np.uint16)
    scale = 0.125
    want = np.stack([orc.sigmoid_gate(gate[t], orc.attn(q[t], kc, vc, pos0 + t + 1, nh, nkv, hd, scale, win), nh, hd)
                     for t in range(T)])
    out = torch.zeros((T, nh * hd), dtype=torch.int16, device=dev)
    qx = torch.empty((T, nh * hd), dtype=torch.int8, device=dev)
    dx = torch.empty((T, nh * hd // 32), dtype=torch.float32, device=dev)
    pq.attn_decode(_t16(q, dev), nh * hd, _t16(kc, dev), _t16(vc, dev), pos0, nh, nkv, hd, T, scale,
                   gate=_t16(gate, dev), gate_stride=nh, out=out, out_stride=nh * hd, qx=qx, dx=dx, win=win)
    got = _u16(out)
    bad = np.argwhere(got != want)
    assert bad.shape[0] == 0, f"{bad.shape[0]} differ, first {bad[:4].tolist()}"
    assert np.array_equal(qx.cpu().numpy(), orc.q8_quant_bf16(want)[0])


def test_qk_prep_ref_bf16_cache(orc, pq, dev):
    """pq_qk_prep_ref: q as pq_qk_prep leaves it, and the cache rows the bf16 k
    (normed, rotated) and v as they are (k_kv_write's copy)."""
    nh, nkv, hd, ctx, pos0, T, rot = 16, 4, 128, 512, 300, 5, 64
    nin, rows, qn, kn, _ = _qkv_case(orc, nh, nkv, hd, T, 2, SEED + 77)
    cs = orc.rope_table(ctx, hd, rot, 1e6)
    kvd = nkv * hd
    want = rows.copy()
    kc_r = np.zeros((ctx, kvd), np.uint16)
    vc_r = np.zeros((ctx, kvd), np.uint16)
    for t in range(T):
        r = want[t]
        r[:nh * hd] = orc.rope(orc.headnorm(r[:nh * hd], qn, nh, hd), cs, pos0 + t, nh, hd, rot)
        kc_r[pos0 + t] = orc.rope(orc.headnorm(r[nh * hd:nh * hd + kvd], kn, nkv, hd), cs, pos0 + t, nkv, hd, rot)
        vc_r[pos0 + t] = r[nh * hd + kvd:nh * hd + 2 * kvd]
    qkv = _t16(rows, dev)
    kc = torch.zeros((ctx, kvd), dtype=torch.int16, device=dev)
    vc = torch.zeros((ctx, kvd), dtype=torch.int16, device=dev)
    pq.qk_prep_ref(qkv, nin, torch.from_numpy(qn).to(dev), torch.from_numpy(kn).to(dev),
                   torch.from_numpy(cs).to(dev), kc, vc, pos0, nh, nkv, hd, rot, T)
    assert np.array_equal(_u16(qkv)[:, :nh * hd], want[:, :nh * hd])
    assert np.array_equal(_u16(kc), kc_r) and np.array_equal(_u16(vc), vc_r)


# pq_attn_ref (k_attn_head's order over the bf16 cache) against the oracle's
# orc_attn_ref + sigmoid gate, bit for bit: one key, one and several rounds of
# the 256 threads' softmax sums, 2048 and 4500 keys, chunks of T queries,
# head_dim 64 and 128, GQA groups 1, 4 and 8, windows 256, 100 and 1.
@pytest.mark.parametrize("npos_last,T,nh,nkv,hd,win", [
    (1, 1, 32, 8, 64, 0), (300, 1, 32, 8, 64, 0), (2048, 1, 32, 8, 64, 0), (40, 33, 32, 8, 64, 0),
    (1, 1, 16, 4, 128, 0), (600, 1, 16, 4, 128, 0), (129, 40, 16, 4, 128, 0), (4500, 2, 16, 4, 128, 0),
    (300, 1, 16, 4, 128, 256), (2000, 1, 16, 4, 128, 256), (330, 90, 16, 4, 128, 256),
    (200, 20, 8, 8, 64, 100), (90, 5, 16, 4, 128, 1)])
def test_attention_ref(orc, pq, dev, npos_last, T, nh, nkv, hd, win):
    pos0 = npos_last - T
    kvd = nkv * hd
    q = orc.f2bf(orc.gen_normal(SEED + 7 * npos_last, T * nh * hd).reshape(T, nh * hd) * 2)
    gate = orc.f2bf(orc.gen_normal(SEED + 7 * npos_last + 1, T * nh).reshape(T, nh) * 3)
    kc = orc.f2bf(orc.gen_normal(SEED + 7 * npos_last + 2, npos_last * kvd) * 2)
    vc = orc.f2bf(orc.gen_normal(SEED + 7 * npos_last + 3, npos_last * kvd) * 5)
    scale = 0.125
    want = np.stack([orc.sigmoid_gate(gate[t], orc.attn_ref(q[t], kc, vc, pos0 + t + 1, nh, nkv, hd, scale, win),
                                      nh, hd) for t in range(T)])
    out = torch.zeros((T, nh * hd), dtype=torch.int16, device=dev)
    pq.attn_ref(_t16(q, dev), nh * hd, _t16(kc, dev), _t16(vc, dev), pos0, nh, nkv, hd, T, scale, out, nh * hd,
                gate=_t16(gate, dev), gate_stride=nh, win=win)
    got = _u16(out)
    bad = np.argwhere(got != want)
    assert bad.shape[0] == 0, f"{bad.shape[0]} differ, first {bad[:4].tolist()}"


def test_attention_ref_segment_order(orc, pq, dev):
    """The value segments add pairwise (the oracle's hand-derived case: 0x3f81
    where a sequential sum gives 0x3f80), and no gate leaves the output as is."""
    nh, nkv, hd = 4, 2, 128
    bf = lambda a: orc.f2bf(np.asarray(a, np.float32))
    v = np.zeros((16, nkv, hd), np.float32)
    v[0], v[8], v[1:8] = 16.0, 2.0 ** -4, 2.0 ** -20
    out = torch.zeros(nh * hd, dtype=torch.int16, device=dev)
    pq.attn_ref(_t16(bf(np.zeros(nh * hd)), dev), nh * hd, _t16(bf(np.ones(16 * nkv * hd)), dev), _t16(bf(v), dev),
                15, nh, nkv, hd, 1, 0.125, out, nh * hd)
    assert (_u16(out) == 0x3F81).all()


# pq_attn_decode_ref (one decode token's q/k prep inside its attention launch)
# against the oracle's head norm + RoPE + cache write, then orc_attn_ref and
# the gate, bit for bit -- output and both cache rows, the projected row left
# as it was -- and against the unfused pair pq_qk_prep_ref + pq_attn_ref.
# The position's own key is the last of its score warp (32 warps) and of its
# value segment (8): positions 0, 1, 31, 32, 63, 64, 256 and 289 put it in
# the first or the last warp and segment, in a half-active wave (256: warp 0
# has a round more than warp 1); GQA groups 1, 4 and 8, head_dim 64 and 128,
# partial and full RoPE, windows 256, 100 and 1.
@pytest.mark.parametrize("pos,nh,nkv,hd,rot,win", [
    (0, 32, 8, 64, 32, 0), (1, 32, 8, 64, 32, 0), (31, 32, 8, 64, 32, 0), (32, 32, 8, 64, 32, 0),
    (256, 32, 8, 64, 32, 0), (2047, 32, 8, 64, 32, 0),
    (0, 16, 4, 128, 64, 0), (63, 16, 4, 128, 64, 0), (64, 16, 4, 128, 64, 0), (289, 16, 4, 128, 64, 0),
    (1999, 16, 4, 128, 128, 256), (300, 16, 4, 128, 128, 256), (150, 8, 8, 64, 64, 100), (90, 16, 4, 128, 128, 1),
    (700, 8, 1, 128, 64, 0)])
def test_attention_decode_ref(orc, pq, dev, pos, nh, nkv, hd, rot, win):
    ctx = pos + 3
    kvd = nkv * hd
    nin, rows, qn, kn, _ = _qkv_case(orc, nh, nkv, hd, 1, ctx, SEED + 31 * pos + hd)
    cs = orc.rope_table(ctx, hd, rot, 1e6 if rot < hd else 1e4)
    kc0 = np.zeros((ctx, kvd), np.uint16)
    vc0 = np.zeros((ctx, kvd), np.uint16)
    kc0[:pos] = orc.f2bf(orc.gen_normal(SEED + 5 * pos, pos * kvd).reshape(pos, kvd) * 2)
    vc0[:pos] = orc.f2bf(orc.gen_normal(SEED + 5 * pos + 1, pos * kvd).reshape(pos, kvd) * 5)
    r = rows[0]
    qr = orc.rope(orc.headnorm(r[:nh * hd], qn, nh, hd), cs, pos, nh, hd, rot)
    kc_r, vc_r = kc0.copy(), vc0.copy()
    kc_r[pos] = orc.rope(orc.headnorm(r[nh * hd:nh * hd + kvd], kn, nkv, hd), cs, pos, nkv, hd, rot)
    vc_r[pos] = r[nh * hd + kvd:nh * hd + 2 * kvd]
    gate = r[nh * hd + 2 * kvd:]
    scale = 1.0 / np.sqrt(hd)
    want = orc.sigmoid_gate(gate, orc.attn_ref(qr, kc_r, vc_r, pos + 1, nh, nkv, hd, scale, win), nh, hd)
    qkv = _t16(rows, dev)
    qnd, knd, csd = (torch.from_numpy(a).to(dev) for a in (qn, kn, cs))
    kc, vc = _t16(kc0, dev), _t16(vc0, dev)
    out = torch.zeros(nh * hd, dtype=torch.int16, device=dev)
    gd = qkv[0, nh * hd + 2 * kvd:]
    pq.attn_decode_ref(qkv, qnd, knd, csd, kc, vc, pos, nh, nkv, hd, rot, scale, out, gate=gd, win=win)
    got = _u16(out)
    bad = np.argwhere(got != want)
    assert bad.shape[0] == 0, f"{bad.shape[0]} differ, first {bad[:4].tolist()}"
    assert np.array_equal(_u16(kc), kc_r) and np.array_equal(_u16(vc), vc_r)
    assert np.array_equal(_u16(qkv), rows)
    # the unfused pair on the same inputs
    qkv2, kc2, vc2 = _t16(rows, dev), _t16(kc0, dev), _t16(vc0, dev)
    out2 = torch.zeros(nh * hd, dtype=torch.int16, device=dev)
    pq.qk_prep_ref(qkv2, nin, qnd, knd, csd, kc2, vc2, pos, nh, nkv, hd, rot, 1)
    pq.attn_ref(qkv2, nin, kc2, vc2, pos, nh, nkv, hd, 1, scale, out2, nh * hd, gate=qkv2[:, nh * hd + 2 * kvd:],
                gate_stride=nin, win=win)
    assert np.array_equal(_u16(out2), got)
    assert np.array_equal(_u16(kc2), kc_r) and np.array_equal(_u16(vc2), vc_r)


# pq_attn_decode_ref_q8gate: each head's gate formed in the attention launch
# from Q8 rows on rmsnorm(x, w) equals the separate reference-numerics GEMV of
# those rows (pq_q8r_gemv_fused, NORM prologue, bf16 out, itself pinned to
# pq_rmsnorm + pq_q8r_gemv and the oracle) followed by pq_attn_decode_ref with
# that gate, bit for bit, output and cache rows; head_dim 64 and 128, windows,
# positions 0, 31 and 290.
@pytest.mark.parametrize("pos,nh,nkv,hd,rot,win", [(0, 32, 8, 64, 32, 0), (290, 32, 8, 64, 32, 0),
                                                   (31, 16, 4, 128, 64, 0), (300, 16, 4, 128, 128, 256)])
def test_attention_decode_ref_q8gate(orc, pq, dev, pos, nh, nkv, hd, rot, win):
    H = 2048
    ctx = pos + 3
    kvd = nkv * hd
    nin, rows, qn, kn, _ = _qkv_case(orc, nh, nkv, hd, 1, ctx, SEED + 17 * pos + hd)
    cs = orc.rope_table(ctx, hd, rot, 1e6 if rot < hd else 1e4)
    kc0 = np.zeros((ctx, kvd), np.uint16)
    vc0 = np.zeros((ctx, kvd), np.uint16)
    kc0[:pos] = orc.f2bf(orc.gen_normal(SEED + 3 * pos, pos * kvd).reshape(pos, kvd) * 2)
    vc0[:pos] = orc.f2bf(orc.gen_normal(SEED + 3 * pos + 1, pos * kvd).reshape(pos, kvd) * 5)
    g = torch.Generator(device=dev)
    g.manual_seed(pos + hd)
    codes = torch.randint(-127, 128, (nh, H), dtype=torch.int8, device=dev, generator=g)
    scales = torch.rand((nh, H // 32), device=dev, generator=g) * 0.002
    x = (torch.randn(H, device=dev, generator=g) * 3).to(torch.bfloat16)
    w = torch.rand(H, device=dev, generator=g) + 0.5
    scale = 1.0 / np.sqrt(hd)
    qnd, knd, csd = (torch.from_numpy(a).to(dev) for a in (qn, kn, cs))
    # the separate gate GEMV, its bf16 gates, then the attention on them
    gate = pq.q8r_gemv_fused(codes, scales, pq.PRO_NORM, out_dtype=pq.DT_BF16, x_in=x.view(torch.int16), w0=w)
    kc_a, vc_a = _t16(kc0, dev), _t16(vc0, dev)
    want = torch.zeros(nh * hd, dtype=torch.int16, device=dev)
    pq.attn_decode_ref(_t16(rows, dev), qnd, knd, csd, kc_a, vc_a, pos, nh, nkv, hd, rot, scale, want,
                       gate=gate.view(torch.int16), win=win)
    # the one launch
    kc_b, vc_b = _t16(kc0, dev), _t16(vc0, dev)
    got = torch.zeros(nh * hd, dtype=torch.int16, device=dev)
    pq.attn_decode_ref_q8gate(_t16(rows, dev), qnd, knd, csd, kc_b, vc_b, codes, scales, x.view(torch.int16), w,
                              pos, nh, nkv, hd, rot, scale, got, win=win)
    bad = np.argwhere(_u16(got) != _u16(want))
    assert bad.shape[0] == 0, f"{bad.shape[0]} differ, first {bad[:4].tolist()}"
    assert torch.equal(kc_a, kc_b) and torch.equal(vc_a, vc_b)
    # the gates matter: a zero gate row would leave the output at half
    assert len(set(_u16(gate.view(torch.int16)).tolist())) > nh // 2


def test_attention_decode_ref_rejects(pq, dev):
    """Bad shapes fail on the host with an error, before any launch."""
    z16 = torch.zeros(4096, dtype=torch.int16, device=dev)
    zf = torch.zeros(4096, dtype=torch.float32, device=dev)
    for pos, hd, rot in [(-1, 64, 32), (5, 96, 32), (5, 64, 33), (5, 64, 66)]:
        with pytest.raises(RuntimeError):
            pq.attn_decode_ref(z16, zf, zf, zf, z16, z16, pos, 4, 2, hd, rot, 0.125, z16)


# T past one 32-position tile (33, 100, 256: the tile at 0 alone reads and then
# rewrites the ring), T below the tap count (7, 3), a channel count that is not
# a multiple of 64
@pytest.mark.parametrize("ntaps,T,H", [(3, 1, 2048), (3, 32, 2048), (7, 5, 2048), (3, 33, 2048), (3, 100, 2048),
                                       (7, 256, 2048), (7, 3, 2048), (7, 70, 1000)])
def test_conv(orc, pq, dev, ntaps, T, H):
    taps = orc.gen_affine(SEED + 20, H * ntaps, 0.0, 0.5)
    ring0 = orc.f2bf(orc.gen_normal(SEED + 21, ntaps * H) * 3)
    bcx = orc.f2bf(orc.gen_normal(SEED + 22, T * 3 * H).reshape(T, 3 * H) * 10)
    ring = ring0.copy()
    want = []
    for t in range(T):
        o, ring = orc.conv_step(ring, taps, bcx[t], H, ntaps)
        want.append(o)
    rd = _t16(ring0, dev)
    out = torch.empty((T, H), dtype=torch.int16, device=dev)
    pq.conv(rd, torch.from_numpy(taps).to(dev), _t16(bcx, dev), out, H, T, ntaps)
    assert np.array_equal(_u16(out), np.stack(want))
    assert np.array_equal(_u16(rd), ring)


@pytest.mark.parametrize("F,T", [(8192, 1), (8192, 4), (512, 2), (7680, 3), (768, 2)])
def test_silu_mul(orc, pq, dev, F, T):
    gu = orc.f2bf(orc.gen_normal(SEED + F + T, T * 2 * F).reshape(T, 2 * F) * 20)
    want = np.stack([orc.silu_mul(gu[t, :F], gu[t, F:]) for t in range(T)])
    y, qx, dx = pq.silu_mul(_t16(gu, dev), F, T, quant=True)
    assert np.array_equal(_u16(y), want)
    assert np.array_equal(qx.cpu().numpy(), orc.q8_quant_bf16(want)[0])


def test_argmax_and_ties(orc, pq, dev):
    v = orc.gen_normal(SEED + 30, 65536)
    assert int(pq.argmax(torch.from_numpy(v).to(dev)).item()) == orc.argmax(v)
    v2 = np.zeros(65536, np.float32)
    v2[[7, 300, 65535]] = 5.0
    assert int(pq.argmax(torch.from_numpy(v2).to(dev)).item()) == 7
    # k_argmax's tie order (the oracle's transcription of its trees) where many
    # values tie: rows 1 and 2 give 2, nothing above -1e30 gives -1
    v3 = np.zeros(300, np.float32)
    v3[[1, 2]] = 1.0
    assert int(pq.argmax(torch.from_numpy(v3).to(dev)).item()) == 2
    assert int(pq.argmax(torch.full((100,), -float("inf"), device=dev)).item()) == -1
    rng = np.random.default_rng(SEED + 31)
    for n in (5, 256, 300, 4099, 65536, 128000):
        v4 = rng.integers(0, 3, n).astype(np.float32)
        assert int(pq.argmax(torch.from_numpy(v4).to(dev)).item()) == orc.argmax(v4), n


def test_embed(orc, pq, dev):
    vocab, H = 1000, 2048
    W, S = orc.q8_weights(SEED + 40, vocab, H)
    w = pq.Q8Weight(torch.from_numpy(W).to(dev), torch.from_numpy(S.view(np.int16)).to(dev))
    toks = np.array([0, 999, 64, 513, -1, 1000], np.int32)
    got = pq.embed(w, torch.from_numpy(toks).to(dev), H, vocab).cpu().numpy().view(np.uint16)
    for i, t in enumerate(toks[:4]):
        assert np.array_equal(got[i], orc.embed_row(W, S, int(t)))
    assert not got[4:].any()


def test_expf_on_device_matches_host(orc, pq, dev):
    """silu over a sweep of inputs exercises the device e^x against the host one."""
    x = np.concatenate([np.linspace(-100, 100, 8192 - 6), [0.0, -0.0, 88.0, -88.0, 1e-30, -1e-30]]).astype(np.float32)
    a = orc.f2bf(x)
    b = orc.f2bf(np.ones_like(x))
    gu = np.concatenate([a, b])[None, :]
    y, _, _ = pq.silu_mul(_t16(gu, dev), 8192, 1)
    assert np.array_equal(_u16(y)[0], orc.silu_mul(a, b))


@pytest.mark.parametrize("nt", [3, 7])
def test_conv_closed_forms(orc, pq, dev, nt):
    """The conv kernel on the hand-built channels of tests/conv_cases.py: the
    ascending unfused tap sum, bx = bf16(B*x) and cy = bf16(acc) before C, each
    of which a departure would change (the oracle's closed-form test shows which)."""
    import conv_cases as cc
    H = 256
    rb, taps, bcx, _ = cc.build(H, nt)
    want_out, want_ring = cc.expected(H, nt)
    rd = _t16(rb.reshape(-1), dev)
    out = torch.empty((1, H), dtype=torch.int16, device=dev)
    pq.conv(rd, torch.from_numpy(taps.reshape(-1)).to(dev), _t16(bcx, dev), out, H, 1, nt)
    torch.cuda.synchronize()
    assert np.array_equal(_u16(out)[0], want_out)
    assert np.array_equal(_u16(rd).reshape(nt, H), want_ring)
