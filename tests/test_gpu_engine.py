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
    e = _engine(pq, cfg, chunk=256)       # the 256-token prompt as one layer-major chunk
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
    e.set_chunk(32)                       # eight 32-position chunks per layer: the same bits
    e.reset()
    _, lg = e.feed(prompt, True)
    assert hashlib.sha256(lg.tobytes()).hexdigest() == g["prompt_logits_sha256"]
    e.close()


def _model_blob(orc, cfg, path):
    from model_blob import model_blob
    model_blob(orc, cfg, path)


def test_blob_load_matches_synthetic(orc, pq, dev, tmp_path):
    """The tiny model through an .lfm3q8 file: same greedy ids as the golden
    and the same residual as the synthetic load."""
    from pulsar_amd.engine import Engine
    p = tmp_path / "tiny.lfm3q8"
    _model_blob(orc, TINY, p)
    g = json.load(open(os.path.join(GOLDEN, "tiny_greedy.json")))
    e = Engine(**TINY)
    e.load_blob(p)
    ids = e.greedy(np.array(g["prompt"], np.int32), len(g["ids"]))
    assert ids.tolist() == g["ids"]
    ref = _engine(pq, TINY)
    ref.greedy(np.array(g["prompt"], np.int32), len(g["ids"]))
    assert np.array_equal(e.hidden(), ref.hidden())
    e.close()
    ref.close()
    # a blob whose shapes do not fit the configuration is refused
    bad = dict(TINY, ffn=768)
    e = Engine(**bad)
    with pytest.raises(pq.PQError, match="feed_forward"):
        e.load_blob(p)
    e.close()


def test_feed_past_context_is_refused_whole(orc, pq, dev):
    """A prompt longer than the room left in the context is refused before the
    first chunk: the position, KV cache and conv rings stay as they were."""
    cfg = dict(TINY, ctx=64)
    e = _engine(pq, cfg)
    ref = _engine(pq, cfg)
    first = orc.gen_tokens(11, 40, cfg["vocab"])
    e.feed(first)
    ref.feed(first)
    with pytest.raises(pq.PQError, match="exceed the context"):
        e.feed(orc.gen_tokens(12, 25, cfg["vocab"]))      # 40 + 25 > 64
    assert e.position() == 40
    more = orc.gen_tokens(13, 24, cfg["vocab"])            # 40 + 24 == 64 still fits
    r_e, lg_e = e.feed(more, True)
    r_r, lg_r = ref.feed(more, True)
    assert r_e == r_r and np.array_equal(lg_e.view(np.uint32), lg_r.view(np.uint32))
    e.close()
    ref.close()


# ------------------------------------------------ the reference's GEMV numerics
@pytest.mark.parametrize("cfg", [TINY, WIDE2], ids=["tiny", "wide2"])
def test_ref_numerics_matches_oracle(orc, pq, dev, cfg):
    """numerics = 1 (PQ_NUMERICS_REF): every GEMV through pq_q8r_gemv on bf16
    activations and fp32 scales, bit for bit against the oracle backbone in the
    same mode, over a 40-token prompt (layer-major, chunks of 32) and 4 steps."""
    cfg = dict(cfg, numerics=1)
    e = _engine(pq, cfg)
    m = orc.Model(**cfg)
    prompt = orc.gen_tokens(5, 40, cfg["vocab"])
    r_e, lg_e = e.feed(prompt, True)
    r_o, lg_o = m.feed(prompt, True)
    assert np.array_equal(e.hidden(), m.hidden())
    assert r_e == r_o and np.array_equal(lg_e.view(np.uint32), lg_o.view(np.uint32))
    for step in range(4):
        r_e, lg_e = e.feed(np.array([r_e], np.int32), True)
        r_o, lg_o = m.feed(np.array([r_o], np.int32), True)
        assert r_e == r_o and np.array_equal(lg_e.view(np.uint32), lg_o.view(np.uint32)), step
    e.close()
    m.close()


def test_ref_numerics_greedy_64(orc, pq, dev):
    """The synthetic 24-layer backbone under the reference's GEMV order: the
    64 greedy ids of tests/golden/lfm3_synth_greedy_ref.json."""
    g = json.load(open(os.path.join(GOLDEN, "lfm3_synth_greedy_ref.json")))
    cfg = dict(g["cfg"])
    assert cfg["numerics"] == 1
    e = _engine(pq, cfg, chunk=256)
    ids = e.greedy(np.array(g["prompt"], np.int32), 64)
    assert ids.tolist() == g["ids"], f"first mismatch at step {int(np.argmax(ids != np.array(g['ids'])))}"
    e.reset()
    _, lg = e.feed(np.array(g["prompt"], np.int32), True)
    import hashlib
    assert hashlib.sha256(lg.tobytes()).hexdigest() == g["prompt_logits_sha256"]
    e.close()


def test_blob_scales_fp16_or_ref_numerics(orc, pq, dev, tmp_path):
    """A blob whose fp32 scales fp16 cannot hold: the Q8 engine refuses it with
    a count (nothing rounded silently); the reference-numerics engine loads it
    with its fp32 scales. An exact blob loads in both modes and matches the
    synthetic engines."""
    from pulsar_amd.blob import Blob, write_blob
    from pulsar_amd.engine import Engine
    p = tmp_path / "tiny.lfm3q8"
    _model_blob(orc, TINY, p)
    ref_cfg = dict(TINY, numerics=1)
    g = json.load(open(os.path.join(GOLDEN, "tiny_greedy.json")))
    prompt = np.array(g["prompt"], np.int32)
    e = Engine(**ref_cfg)
    e.load_blob(p)
    syn = _engine(pq, ref_cfg)
    assert np.array_equal(e.greedy(prompt, 8), syn.greedy(prompt, 8))
    assert np.array_equal(e.hidden(), syn.hidden())
    e.close()
    syn.close()
    # nudge one tensor's scales off the fp16 grid
    b = Blob(p)
    ts = []
    for i in range(len(b)):
        info = b.info(i)
        v = b.read(i)
        if info["name"] == "lfm.model.layers.1.self_attn.o_proj.weight":
            c, s = v
            s = s.copy()
            s[::3] *= np.float32(1 + 2 ** -20)
            v = (c, s)
        elif info["dtype"] == 3:
            v = ("bf16", v)
        ts.append((info["name"], v))
    cfg_json = b.config()
    b.close()
    q = tmp_path / "nudged.lfm3q8"
    write_blob(q, cfg_json, ts)
    e = Engine(**TINY)
    with pytest.raises(pq.PQError, match="o_proj.*not fp16 values"):
        e.load_blob(q)
    e.close()
    e = Engine(**ref_cfg)
    e.load_blob(q)                        # kept as fp32: loads
    ids = e.greedy(prompt, 4)
    assert len(ids) == 4
    e.close()


# ------------------------------------------------- the real LFM3 backbone's shapes
# hidden 2048, FFN 7680, vocab 128000, 16 q / 4 kv heads of dim 128, 7-tap conv,
# full attention (theta 1e6, 64 of 128 dims rotated) and sliding-window
# attention (theta 1e4, all dims rotated); four layers, the window cut to 40 so
# a 100-token prompt crosses it inside and across 32-position chunks
REAL4 = dict(hidden=2048, ffn=7680, vocab=128000, nlayers=4, nh=16, nkv=4, hd=128, rot=64, ntaps=7, ctx=256,
             eps=1e-5, theta=1e6, seed=77, attn_mask=0b1010, slide_mask=0b1000, slide_win=40, slide_rot=128,
             slide_theta=1e4)


@pytest.mark.parametrize("numerics", [0, 1])
def test_real_widths_match_oracle(orc, pq, dev, numerics):
    cfg = dict(REAL4, numerics=numerics)
    e = _engine(pq, cfg)
    m = orc.Model(**cfg)
    prompt = orc.gen_tokens(8, 100, cfg["vocab"])
    r_e, lg_e = e.feed(prompt, True)
    r_o, lg_o = m.feed(prompt, True)
    assert np.array_equal(e.hidden(), m.hidden())
    assert r_e == r_o and np.array_equal(lg_e.view(np.uint32), lg_o.view(np.uint32))
    for step in range(4):
        r_e, lg_e = e.feed(np.array([r_e], np.int32), True)
        r_o, lg_o = m.feed(np.array([r_o], np.int32), True)
        assert r_e == r_o and np.array_equal(lg_e.view(np.uint32), lg_o.view(np.uint32)), step
    e.close()
    m.close()


def test_real_lfm3_blob_greedy_64(orc, pq, dev, tmp_path):
    """The real LFM3 backbone's shapes and layer pattern (13 conv, 6 full and 5
    sliding-window attention layers, interleaved as the reference's model):
    the oracle's synthetic model written as an .lfm3q8 file under the
    reference's tensor names and layer_types, loaded through
    pq_engine_load_blob; a 256-token prompt and 64 greedy ids (positions past
    the 256-key window) equal to tests/golden/lfm3_real_shapes_greedy.json."""
    from pulsar_amd.engine import Engine
    g = json.load(open(os.path.join(GOLDEN, "lfm3_real_shapes_greedy.json")))
    cfg = dict(g["cfg"])
    p = tmp_path / "lfm3_real_shapes.lfm3q8"
    t0 = time.time()
    _model_blob(orc, cfg, p)
    t1 = time.time()
    e = Engine(**cfg, prefill_chunk=256)
    e.load_blob(p)
    t2 = time.time()
    prompt = np.array(g["prompt"], np.int32)
    ids = e.greedy(prompt, 64)
    print(f"blob write {t1 - t0:.1f}s ({os.path.getsize(p) / 1e9:.2f} GB), load {t2 - t1:.1f}s")
    assert ids.tolist() == g["ids"], f"first mismatch at step {int(np.argmax(ids != np.array(g['ids'])))}"
    e.reset()
    _, lg = e.feed(prompt, True)
    import hashlib
    assert hashlib.sha256(lg.tobytes()).hexdigest() == g["prompt_logits_sha256"]
    e.close()
    os.remove(p)
