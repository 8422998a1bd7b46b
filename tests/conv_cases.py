"""Closed-form channels for one step of the gated short conv (k_shift_in +
k_conv7 / k_conv_chunk, lfm3_nanode.cu:892-941).

Per channel the step forms bx = bf16(B*x), shifts it into the ring as the newest
slot, sums acc = (((0 + fl(t_0 r_0)) + fl(t_1 r_1)) + ...) over the taps in
ascending order with each product rounded before the add (__fmul_rn then
__fadd_rn), rounds cy = bf16(acc) and writes bf16(C * cy). Each channel below is
built so that one plausible departure from that changes its output:

  order   products 2^24, 1, 0.., -2^24: ascending gives 0, the descending (or a
          pairwise) sum gives 1
  fused   products -2^-8 and t*bx with fl(t*bx) = 2^-8 but t*bx != 2^-8: the
          unfused sum is 0, an fma chain leaves the nonzero residue
  bx      B = x = 1 + 9*2^-7: B*x = 1 + 18.6328*2^-7, whose RNE bf16 is
          1 + 19*2^-7 (truncation 1 + 18*2^-7); a first product of 2^-8 puts the
          rounded value on a bf16 tie (ties to even: 1 + 20*2^-7), the unrounded
          value above it (1 + 19*2^-7), the truncated one on another tie
          (1 + 18*2^-7)
  cy      acc = 1 + 2^-8 - 2^-20 rounds to cy = 1 before C = 1 + 2^-7 multiplies
          it (1 + 2^-7); C * acc unrounded crosses the tie (1 + 2^-6)

Every channel is repeated to fill H. The expected outputs are worked by hand
(in the comments above) and re-derived exactly with fractions here.
"""
from fractions import Fraction

import numpy as np

ORDER, FUSED, BX, CY = range(4)
KINDS = ("order", "fused", "bx", "cy")


def _bf16_bits(v):
    """bf16 bits of a float exactly representable in bf16."""
    b = np.array([v], np.float32).view(np.uint32)[0]
    assert b & 0xFFFF == 0, v
    return int(b >> 16)


def _fused_tap(bx):
    """An fp32 t with fl(t * bx) == 2^-8 while the exact product differs."""
    t = np.float32(2.0 ** -8 / bx)
    for _ in range(64):
        exact = Fraction(float(t)) * Fraction(bx)
        if exact != Fraction(1, 256) and _rne_f32(exact) == Fraction(1, 256):
            return float(t)
        t = np.nextafter(t, np.float32(1.0))
    raise AssertionError("no fused tap")


def build(H, nt):
    """(ring_old bits [nt][H], taps f32 [H][nt], bcx bits [3H], kinds [H]) for one step."""
    ring_new = np.zeros((nt, H), np.float64)
    taps = np.zeros((H, nt), np.float64)
    B = np.ones(H)
    C = np.ones(H)
    X = np.ones(H)
    kinds = np.arange(H) % 4
    fused_bx = 1.0 + 2.0 ** -7
    tf = _fused_tap(fused_bx)
    for i in range(H):
        k = kinds[i]
        ring_new[:, i] = 1.0
        if k == ORDER:
            taps[i, 0], taps[i, 1], taps[i, nt - 1] = 2.0 ** 24, 1.0, -(2.0 ** 24)
        elif k == FUSED:
            taps[i, 0], taps[i, nt - 1] = -(2.0 ** -8), tf
            B[i] = fused_bx
        elif k == BX:
            taps[i, 0], taps[i, nt - 1] = 2.0 ** -8, 1.0
            B[i] = X[i] = 1.0 + 9 * 2.0 ** -7
        else:
            taps[i, 0] = 1.0 + 2.0 ** -8 - 2.0 ** -20
            C[i] = 1.0 + 2.0 ** -7
    # the step shifts ring_old[k+1] into slot k: ring_old[0] is dropped, so set it
    # to a value that would show up if it were not
    ring_old = np.zeros((nt, H), np.float64)
    ring_old[1:] = ring_new[:nt - 1]
    ring_old[0] = 3.0
    rb = np.vectorize(_bf16_bits)(ring_old).astype(np.uint16)
    bcx = np.concatenate([np.vectorize(_bf16_bits)(v).astype(np.uint16) for v in (B, C, X)])
    return rb, taps.astype(np.float32), bcx, kinds


def expected(H, nt):
    """(out bits [H], ring_new bits [nt][H]) of the step, from the closed forms."""
    rb, _, bcx, kinds = build(H, nt)
    want_out = {ORDER: 0x0000, FUSED: 0x0000,
                BX: _bf16_bits(1.0 + 20 * 2.0 ** -7), CY: _bf16_bits(1.0 + 2.0 ** -7)}
    out = np.array([want_out[k] for k in kinds], np.uint16)
    bx = {ORDER: _bf16_bits(1.0), FUSED: _bf16_bits(1.0 + 2.0 ** -7),
          BX: _bf16_bits(1.0 + 19 * 2.0 ** -7), CY: _bf16_bits(1.0)}
    ring = np.empty((nt, H), np.uint16)
    ring[:nt - 1] = rb[1:]
    ring[nt - 1] = [bx[k] for k in kinds]
    return out, ring


def departures(H, nt):
    """The outputs a plausible departure gives, per kind, to show the channels
    separate them: {name: out bits [H]} from exact-rational restatements."""
    rb, taps, bcx, kinds = build(H, nt)

    def step(order, fused, round_bx, round_cy):
        outs = []
        for i in range(H):
            B = Fraction(float(np.uint32(int(bcx[i]) << 16).view(np.float32)))
            Cv = Fraction(float(np.uint32(int(bcx[H + i]) << 16).view(np.float32)))
            X = Fraction(float(np.uint32(int(bcx[2 * H + i]) << 16).view(np.float32)))
            bxe = B * X
            bxv = _rne_bf16(bxe) if round_bx else bxe
            r = [Fraction(float(np.uint32(int(rb[k + 1, i]) << 16).view(np.float32))) for k in range(nt - 1)] + [bxv]
            t = [Fraction(float(taps[i, k])) for k in range(nt)]
            ks = range(nt) if order == "asc" else range(nt - 1, -1, -1)
            acc = Fraction(0)
            for k in ks:
                p = t[k] * r[k]
                acc = _rne_f32(acc + p) if fused else _rne_f32(acc + _rne_f32(p))
            cy = _rne_bf16(acc) if round_cy else acc
            outs.append(_bits_of(_rne_bf16(Cv * cy)))
        return np.array(outs, np.uint16)

    return {"reference": step("asc", False, True, True), "descending": step("desc", False, True, True),
            "fused": step("asc", True, True, True), "bx unrounded": step("asc", False, False, True),
            "cy unrounded": step("asc", False, True, False)}


def _rne(v, mant_bits):
    """Round the exact rational v to mant_bits significant bits, ties to even (normal range)."""
    if v == 0:
        return Fraction(0)
    s = -1 if v < 0 else 1
    a = abs(v)
    e = 0
    while a >= 2:
        a /= 2
        e += 1
    while a < 1:
        a *= 2
        e -= 1
    scaled = a * (1 << (mant_bits - 1))
    n = scaled.numerator // scaled.denominator
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return s * Fraction(n, 1 << (mant_bits - 1)) * Fraction(2) ** e


def _rne_f32(v):
    return _rne(v, 24)


def _rne_bf16(v):
    return _rne(v, 8)


def _bits_of(v):
    return _bf16_bits(float(v)) if v != 0 else 0
