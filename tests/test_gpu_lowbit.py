"""The low-bit backbone and the bf16 embedding table on the GPU.

pq_bf16_gemv / pq_embed_bf16 against the oracle (k_gemv_bf16's order, the row
copy), and the engine loading .lfm3q8 files with Q4 / Q5 tensors (dtype 6 / 7)
and a bf16 table (dtype 3) under the reference numerics: logits and residuals
bit for bit against the oracle backbone over a prompt and decode steps, the
fused decode step (graph and eager) against the unfused one, and the 64 greedy
ids of the 24-layer synthetic backbone with Q4 linears against its golden."""
import ctypes as C
import json
import os
import time

import numpy as np
import pytest
import torch

from model_blob import engine_cfg, model_blob

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")

TINY = dict(hidden=256, ffn=512, vocab=1000, nlayers=4, nh=4, nkv=2, hd=64, rot=32, ntaps=3, ctx=256,
            eps=1e-5, theta=1e6, seed=20261201, attn_mask=0b1010, numerics=1)
# full width (the fused decode kernels): layer 0 gated conv, layer 1 attention
WIDE2 = dict(hidden=2048, ffn=8192, vocab=65536, nlayers=2, nh=32, nkv=8, hd=64, rot=32, ntaps=3, ctx=512,
             eps=1e-5, theta=1e6, seed=99, attn_mask=0b10, numerics=1)


def _p(t):
    return C.c_void_p(t.data_ptr())


@pytest.mark.parametrize("N,K", [(65536, 2048), (1000, 256), (77, 4096), (130, 5120), (33, 96)])
def test_bf16_gemv(orc, pq, dev, N, K):
    print(f"bf16_gemv N={N} K={K}", flush=True)
    rng = np.random.default_rng(N + K)
    W = orc.f2bf(rng.standard_normal(N * K).astype(np.float32)).reshape(N, K)
    x = orc.f2bf(rng.standard_normal(K).astype(np.float32) * 2)
    W[N // 3, :] = W[N // 5, :]            # two equal rows
    want = orc.bf16_gemv(W, x)
    Wd = torch.from_numpy(W.view(np.int16)).to(dev)
    xd = torch.from_numpy(x.view(np.int16)).to(dev)
    y = torch.empty(N, dtype=torch.float32, device=dev)
    nparts = pq.lib().pq_bf16_gemv_parts(N)
    parts = torch.empty(2 * nparts, dtype=torch.float32, device=dev)
    pq.check(pq.lib().pq_bf16_gemv(_p(Wd), _p(xd), _p(y), N, K, _p(parts), C.c_void_p(pq.stream_ptr())),
             "pq_bf16_gemv")
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
    assert int(pq.argmax_parts(parts, nparts).item()) == orc.argmax(want)


def test_bf16_gemv_tie_order(orc, pq, dev):
    """Rows 1, 2, 33, 64 and 300 equal and largest: the argmax pairs give
    k_argmax's pick, row 2 (the lowest index would be row 1)."""
    N, K = 3000, 512
    rng = np.random.default_rng(17)
    W = orc.f2bf(rng.standard_normal(N * K).astype(np.float32) * 0.01).reshape(N, K)
    W[[1, 2, 33, 64, 300]] = orc.f2bf(np.ones(K, np.float32))
    x = orc.f2bf(np.ones(K, np.float32))
    want = orc.bf16_gemv(W, x)
    assert orc.argmax(want) == 2
    Wd = torch.from_numpy(W.view(np.int16)).to(dev)
    xd = torch.from_numpy(x.view(np.int16)).to(dev)
    y = torch.empty(N, dtype=torch.float32, device=dev)
    nparts = pq.lib().pq_bf16_gemv_parts(N)
    parts = torch.empty(2 * nparts, dtype=torch.float32, device=dev)
    pq.check(pq.lib().pq_bf16_gemv(_p(Wd), _p(xd), _p(y), N, K, _p(parts), C.c_void_p(pq.stream_ptr())),
             "pq_bf16_gemv")
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
    assert int(pq.argmax_parts(parts, nparts).item()) == 2


def test_embed_bf16(orc, pq, dev):
    rng = np.random.default_rng(5)
    vocab, H = 300, 2048
    table = rng.integers(0, 65536, (vocab, H)).astype(np.uint16)
    toks = np.array([0, 299, 17, -1, 300, 5], np.int32)
    td = torch.from_numpy(table.view(np.int16)).to(dev)
    kd = torch.from_numpy(toks).to(dev)
    out = torch.full((len(toks), H), 0x7fff, dtype=torch.int16, device=dev)
    pq.check(pq.lib().pq_embed_bf16(_p(td), _p(kd), _p(out), H, vocab, len(toks), C.c_void_p(pq.stream_ptr())),
             "pq_embed_bf16")
    got = out.cpu().numpy().view(np.uint16)
    for i, t in enumerate(toks):
        want = table[t] if 0 <= t < vocab else np.zeros(H, np.uint16)
        assert np.array_equal(got[i], want), t


def _engine_from_blob(orc, pq, cfg, path, chunk=32):
    from pulsar_amd.engine import Engine
    model_blob(orc, cfg, path)
    e = Engine(**engine_cfg(cfg), prefill_chunk=chunk)
    e.load_blob(path)
    return e


# (bits, lowbit_mask, emb_bf16): Q4 layers 1-2 with the Q8 table, Q5 layers 0-1
# with the bf16 table, the bf16 table alone
TINY_CASES = [(4, 0b0110, 0), (5, 0b0011, 1), (0, 0, 1)]


@pytest.mark.parametrize("bits,mask,emb16", TINY_CASES, ids=["q4", "q5-bf16", "bf16"])
def test_lowbit_blob_matches_oracle(orc, pq, dev, tmp_path, bits, mask, emb16):
    """A 40-token prompt (chunks of 32 and 8: the parts' T-wide staging) and 4
    single-position feeds, logits and residual bit for bit against the oracle."""
    cfg = dict(TINY, lowbit=bits, lowbit_mask=mask, emb_bf16=emb16)
    e = _engine_from_blob(orc, pq, cfg, tmp_path / "t.lfm3q8")
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
    # greedy decode through pq_engine_decode's step (TINY: the unfused sequence)
    ids = e.greedy(prompt, 6)
    assert np.array_equal(ids, m.greedy(prompt, 6))
    e.close()
    m.close()


WIDE_CASES = [(4, 0b11, 1), (5, 0b10, 0), (0, 0, 1)]


@pytest.mark.parametrize("bits,mask,emb16", WIDE_CASES, ids=["q4-all-bf16", "q5-attn", "bf16"])
def test_lowbit_fused_step(orc, pq, dev, tmp_path, bits, mask, emb16):
    """Full-width layers: the fused decode step with split slots (a layer's
    low-bit parts run their own GEMVs, the conv ring copied for the ping-pong),
    replayed from graphs and launched eagerly, and the unfused sequence, give the
    oracle's greedy ids and the same final residual; graph replays split into
    decode calls with eager work between them."""
    cfg = dict(WIDE2, lowbit=bits, lowbit_mask=mask, emb_bf16=emb16)
    path = tmp_path / "w.lfm3q8"
    model_blob(orc, cfg, path)
    m = orc.Model(**cfg)
    prompt = orc.gen_tokens(9, 70, cfg["vocab"])
    ref = m.greedy(prompt, 12)
    m.close()
    from pulsar_amd.engine import Engine
    resid = []
    for fused, graph in ((True, True), (True, False), (False, False)):
        print(f"lowbit fused={fused} graph={graph}", flush=True)
        e = Engine(**engine_cfg(cfg))
        e.load_blob(path)
        e.set_fused(fused)
        e.set_graph(graph)
        ids = e.greedy(prompt, 12)
        resid.append(e.hidden())
        e.close()
        assert np.array_equal(ids, ref), (fused, graph, ids.tolist(), ref.tolist())
    assert np.array_equal(resid[0], resid[2]) and np.array_equal(resid[1], resid[2])
    e = Engine(**engine_cfg(cfg))
    e.load_blob(path)
    assert e.feed(prompt) == ref[0]
    out = []
    for k, graph in ((3, True), (1, False), (4, True), (2, True)):
        e.set_graph(graph)
        out.extend(e.decode(k).tolist())
        e.hidden()
    e.close()
    assert np.array_equal(np.array(out), ref[1:11]), (out, ref[1:11].tolist())


def test_lowbit_needs_reference_numerics(orc, pq, dev, tmp_path):
    """A Q4 tensor or a bf16 table in a Q8_0-numerics engine is refused with a
    message naming the tensor and the mode that runs it; a reload of a plain Q8
    blob into a low-bit engine drops the parts (the same ids as a Q8 engine)."""
    from pulsar_amd.engine import Engine
    p = tmp_path / "q4.lfm3q8"
    model_blob(orc, dict(TINY, lowbit=4, lowbit_mask=0b0001), p)
    e = Engine(**engine_cfg(dict(TINY, numerics=0)))
    with pytest.raises(pq.PQError, match="layers.0.*Q4 / Q5.*PQ_NUMERICS_REF"):
        e.load_blob(p)
    e.close()
    b = tmp_path / "bf.lfm3q8"
    model_blob(orc, dict(TINY, emb_bf16=1), b)
    e = Engine(**engine_cfg(dict(TINY, numerics=0)))
    with pytest.raises(pq.PQError, match="embed_tokens.*bf16 table.*PQ_NUMERICS_REF"):
        e.load_blob(b)
    e.close()
    q8 = tmp_path / "q8.lfm3q8"
    model_blob(orc, TINY, q8)
    prompt = orc.gen_tokens(6, 20, TINY["vocab"])
    e = Engine(**engine_cfg(TINY))
    e.load_blob(p)
    e.load_blob(q8)
    a = e.greedy(prompt, 5)
    e.close()
    m = orc.Model(**TINY)
    assert np.array_equal(a, m.greedy(prompt, 5))
    m.close()


def test_lfm3_synth_q4_greedy_64(orc, pq, dev, tmp_path):
    """The synthetic 24-layer backbone with every layer's linears Q4 (the
    attention gate_proj Q8) as an .lfm3q8 file: a 256-token prompt and 64
    greedy ids through the fused step equal to tests/golden/lfm3_synth_q4_greedy.json."""
    g = json.load(open(os.path.join(GOLDEN, "lfm3_synth_q4_greedy.json")))
    cfg = dict(g["cfg"])
    t0 = time.time()
    e = _engine_from_blob(orc, pq, cfg, tmp_path / "q4.lfm3q8", chunk=256)
    t1 = time.time()
    prompt = np.array(g["prompt"], np.int32)
    assert np.array_equal(prompt, orc.gen_tokens(g["prompt_seed"], g["n_prompt"], cfg["vocab"]))
    ids = e.greedy(prompt, 64)
    print(f"blob + load {t1 - t0:.1f}s, prompt + 64 steps {time.time() - t1:.2f}s", flush=True)
    assert ids.tolist() == g["ids"], f"first mismatch at step {int(np.argmax(ids != np.array(g['ids'])))}"
    e.reset()
    _, lg = e.feed(prompt, True)
    import hashlib
    assert hashlib.sha256(lg.tobytes()).hexdigest() == g["prompt_logits_sha256"]
    e.close()
