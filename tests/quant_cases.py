"""Q8_0 blocks full of exact ties for the activation quantizer (d = amax/127,
q = rne(x/d), clamp +-127; the rounding of q8_gemv_cpu.c:63-81's lrintf).

Each block has amax = 127*m*2^k with m an fp16 significand, so amax/127 = m*2^k
exactly (in fp32 and in fp16: the reference's fp16 scale and the fp32 scale
coincide), and its other elements are n*d + d/2: every x/d is an exact half,
which ties to even settle (ties away from zero and truncation differ).
"""
import numpy as np

SCALES = [(1.0, 0), (1.0, -6), (1.5, -3), (1.25, 4), (1.0009765625, -10), (1.998046875, 2), (1.0, -14)]


def tie_blocks(seed=29, reps=1):
    rng = np.random.default_rng(seed)
    blocks = []
    for _ in range(reps):
        for m, k in SCALES:
            d = np.float32(m * 2.0 ** k)
            n = rng.integers(-126, 126, 32)
            xb = ((n + 0.5) * np.float64(d)).astype(np.float32)
            xb[rng.integers(0, 32)] = np.float32(127.0) * d * (1 if rng.random() < 0.5 else -1)
            xb[rng.integers(0, 32)] = np.float32(0.5) * d     # 0.5 -> 0 under ties to even
            xb[rng.integers(0, 32)] = np.float32(-1.5) * d    # -1.5 -> -2
            xb[rng.integers(0, 32)] = np.float32(2.5) * d     # 2.5 -> 2
            blocks.append(xb)
    return np.concatenate(blocks)


def rne_codes(x):
    """The codes by numpy's round-half-to-even on the exact quotients (d = amax/127 is exact here)."""
    xb = x.reshape(-1, 32).astype(np.float64)
    d = np.abs(xb).max(1, keepdims=True) / 127.0
    return np.clip(np.round(xb / d), -127, 127).astype(np.int8).reshape(-1)


def away_codes(x):
    xb = x.reshape(-1, 32).astype(np.float64)
    d = np.abs(xb).max(1, keepdims=True) / 127.0
    q = xb / d
    return np.clip(np.sign(q) * np.floor(np.abs(q) + 0.5), -127, 127).astype(np.int8).reshape(-1)
