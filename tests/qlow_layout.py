"""The reference's tiled Q4 / Q5 payload (lfm3_qlow.cuh:5-13; the dtype 6 / 7
tensors .auto/lfm3/export_qlow.py writes), restated in numpy for the tests:
the layout pq_qlow_pack is checked against, and the payload the test blobs carry."""
import numpy as np


def pack(Q, S, bits):
    """The reference's tiled payload: per (32-row tile, group) 32 x 16 bytes of
    nibbles (byte b of word i: weight 8i+b low, 8i+4+b high), for Q5 then
    32 x uint32 planes (bit 8b+p = bit 4 of weight 4p+b); scales per (tile,
    group) 32 x (d', mn)."""
    N, K = Q.shape
    G, T = K // 32, N // 32
    q = Q.reshape(T, 32, G, 32).transpose(0, 2, 1, 3).astype(np.uint32)    # [tile][g][row][k]
    words = np.zeros((T, G, 32, 4), np.uint32)
    for i in range(4):
        for b in range(4):
            words[..., i] |= ((q[..., 8 * i + b] & 15) | ((q[..., 8 * i + 4 + b] & 15) << 4)) << (8 * b)
    parts = [words.view(np.uint8).reshape(T, G, 512)]
    if bits == 5:
        plane = np.zeros((T, G, 32), np.uint32)
        for p in range(8):
            for b in range(4):
                plane |= ((q[..., 4 * p + b] >> 4) & 1) << (8 * b + p)
        parts.append(plane.view(np.uint8).reshape(T, G, 128))
    codes = np.concatenate(parts, -1).reshape(-1)
    sc = S.reshape(T, 32, G, 2).transpose(0, 2, 1, 3).reshape(-1)
    return codes, sc
