"""The C++ engine end to end on the GPU against the oracle backbone.

Bit-exact logits and residuals on small models computed live by the oracle,
prefill-chunk invariance, and the 64 greedy ids of the full synthetic 24-layer
backbone against the committed golden fixture."""
import json
import os
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TINY = dict(hidden=256, ffn=512, vocab=1000, nlayers=4, nh=4, nkv=2, hd=64, rot=32, ntaps=3, ctx=256,
            eps=1e-5, theta=1e6, seed=20261201, attn_mask=0b1010)
# full-width layers, two of them: one gated conv, one attention
WIDE2 = dict(hidden=2048, ffn=8192, vocab=65536, nlayers=2, nh=32, nkv=8, hd=64, rot=32, ntaps=3, ctx=512,
             eps=1e-5, theta=1e6, seed=99, attn_mask=0b10)


def _engine(pq, cfg, chunk=32):
    from pulsar_amd.engine import Engine
    e = Engine(**cfg, prefill_chunk=chunk)
    e.load_synthetic()
    return e


def test_tiny_matches_oracle(orc, pq, dev):
    g = json.load(open(os.path.join(GOLDEN, "tiny_greedy.json")))
    e = _engine(pq, TINY)
    ids = e.greedy(np.array(g["prompt"], np.int32), len(g["ids"]))
    assert ids.tolist() == g["ids"]
    m = orc.Model(**TINY)
    prompt = np.array(g["prompt"], np.int32)
    e.reset()
    r_e, lg_e = e.feed(prompt, True)
    r_o, lg_o = m.feed(prompt, True)
    assert r_e == r_o
    assert np.array_equal(lg_e.view(np.uint32), lg_o.view(np.uint32))
    assert np.array_equal(e.hidden(), m.hidden())
    for step in range(3):
        r_e, lg_e = e.feed(np.array([r_e], np.int32), True)
        r_o, lg_o = m.feed(np.array([r_o], np.int32), True)
        assert r_e == r_o and np.array_equal(lg_e.view(np.uint32), lg_o.view(np.uint32)), step
    e.close()
    m.close()


def test_wide_layers_match_oracle(orc, pq, dev):
    e = _engine(pq, WIDE2)
    m = orc.Model(**WIDE2)
    prompt = orc.gen_tokens(5, 40, WIDE2["vocab"])       # chunks of 32 + 8
    r_e, lg_e = e.feed(prompt, True)
    r_o, lg_o = m.feed(prompt, True)
    assert np.array_equal(e.hidden(), m.hidden())
    assert r_e == r_o and np.array_equal(lg_e.view(np.uint32), lg_o.view(np.uint32))
    for step in range(4):
        r_e, lg_e = e.feed(np.array([r_e], np.int32), True)
        r_o, lg_o = m.feed(np.array([r_o], np.int32), True)
        assert np.array_equal(e.hidden(), m.hidden()), step
        assert r_e == r_o and np.array_equal(lg_e.view(np.uint32), lg_o.view(np.uint32)), step
    e.close()
    m.close()


def test_prefill_chunk_invariance(orc, pq, dev):
    """Chunked prefill (MFMA GEMM, T-wide attention/conv) == one position at a time."""
    prompt = orc.gen_tokens(7, 45, TINY["vocab"])
    a = _engine(pq, TINY, chunk=32)
    b = _engine(pq, TINY, chunk=1)
    ra, la = a.feed(prompt, True)
    rb, lb = b.feed(prompt, True)
    assert ra == rb and np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    assert np.array_equal(a.greedy(prompt, 8), b.greedy(prompt, 8))
    a.close()
    b.close()


def test_lfm3_synth_greedy_64(orc, pq, dev):
    """The synthetic 24-layer LFM3-style backbone: 256-token prompt, 64 greedy ids
    identical to the oracle's (tests/golden/lfm3_synth_greedy.json)."""
    g = json.load(open(os.path.join(GOLDEN, "lfm3_synth_greedy.json")))
    cfg = dict(g["cfg"])
    t0 = time.time()
    e = _engine(pq, cfg)
    t1 = time.time()
    prompt = np.array(g["prompt"], np.int32)
    assert np.array_equal(prompt, orc.gen_tokens(g["prompt_seed"], g["n_prompt"], cfg["vocab"]))
    ids = e.greedy(prompt, 64)
    t2 = time.time()
    print(f"load {t1 - t0:.1f}s, prompt + 64 steps {t2 - t1:.2f}s")
    assert ids.tolist() == g["ids"], f"first mismatch at step {int(np.argmax(ids != np.array(g['ids'])))}"
    e.reset()
    _, lg = e.feed(prompt, True)
    import hashlib
    assert hashlib.sha256(lg.tobytes()).hexdigest() == g["prompt_logits_sha256"]
    e.close()
