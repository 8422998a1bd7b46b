"""GPU self-checks of the arithmetic shortcuts the kernels take.

The hardware f32 -> bf16 conversion every kernel uses
(v_cvt_pk_bf16_f32, single and packed) against the reference's rounding
(round to nearest even, inf/nan passed through; lfm3_nanode.cu:114-121) on
all 2^32 float bit patterns: they agree everywhere except on signaling NaNs,
which the hardware quiets. The kernels convert only results of arithmetic,
which are never signaling NaNs (IEEE 754-2008 6.2), so on every value they
convert the two are the same."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_bf16_conversion_exhaustive(pq, dev):
    counts = torch.zeros(65536, dtype=torch.int32, device=dev)
    first = torch.zeros(65536, dtype=torch.int32, device=dev)
    pq.check(pq.lib().pq_check_bf16_cvt(counts.data_ptr(), first.data_ptr(), pq.stream_ptr()), "pq_check_bf16_cvt")
    torch.cuda.synchronize()
    c = counts.cpu().numpy().view(np.uint32)
    f = first.cpu().numpy().view(np.uint32)
    # the signaling NaNs: exponent all ones, quiet bit clear, payload != 0,
    # both signs -- 2 * (2^22 - 1) patterns, lowest 0x7f800001
    assert int(c.sum()) == 2 * ((1 << 22) - 1)
    bad = np.nonzero(c)[0]
    assert int(f[bad].min()) == 0x7F800001
    # every mismatching block lies in the NaN ranges 0x7f80..0x7fff, 0xff80..0xffff
    # (block b holds patterns b << 16) and holds only signaling NaNs: 2^16 - 2^15
    # per block above the quiet bit's half, minus the infinity in the first
    assert set((bad >> 7).tolist()) <= {0x7F80 >> 7, 0xFF80 >> 7}
    for b in bad:
        sub = (b & 0x7F)
        want = 0 if sub >= 0x40 else (1 << 16) - (1 if sub == 0 else 0)
        assert int(c[b]) == want, (hex(int(b)), int(c[b]), want)


@pytest.mark.parametrize("seed", [1, 20261201])
def test_quant_shared_divisor_matches_division(pq, dev, seed):
    """The quantizers' shared-divisor quotient (one refined reciprocal per
    block, two fma corrections per value) gives the Q8_0 codes of x / d, and
    the same quotient bits wherever |x| >= 2^-20 |d|: 2^24 random blocks x 64
    values, ties and their 2-ulp neighbours included."""
    counts = torch.zeros(65536, dtype=torch.int32, device=dev)
    first = torch.zeros(65536, dtype=torch.int32, device=dev)
    pq.check(pq.lib().pq_check_quant_div(counts.data_ptr(), first.data_ptr(), seed, pq.stream_ptr()),
             "pq_check_quant_div")
    torch.cuda.synchronize()
    c = counts.cpu().numpy().view(np.uint32)
    f = first.cpu().numpy().view(np.uint32)
    assert int(c.sum()) == 0, f"{int(c.sum())} mismatches; first threads {[int(x) for x in f[c > 0][:8]]}"


def test_clock_probe(pq, dev):
    """pq_clock_mhz reports a shader clock in MI355X's range (its boost clock is 2.4 GHz)."""
    out = torch.zeros(2, dtype=torch.float32, device=dev)
    pq.check(pq.lib().pq_clock_mhz(out.data_ptr(), pq.stream_ptr()), "pq_clock_mhz")
    torch.cuda.synchronize()
    assert 500.0 < float(out[0]) < 3000.0


def test_stream_read(pq, dev):
    """pq_stream_read (the bench's read ceiling) runs over a buffer and a tail
    shorter than one grid step, and leaves its sink alone for real data."""
    buf = torch.ones(3 << 20, dtype=torch.uint8, device=dev)
    sink = torch.full((1,), 5.0, dtype=torch.float32, device=dev)
    for nb in (buf.numel(), 16, 4096 + 16):
        pq.check(pq.lib().pq_stream_read(buf.data_ptr(), nb, sink.data_ptr(), pq.stream_ptr()), "pq_stream_read")
    torch.cuda.synchronize()
    assert float(sink[0]) == 5.0
