"""Writes the golden fixtures of tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py [kernels] [tiny] [full] [full_ref] [real]

lfm3_synth_greedy.json  the synthetic 24-layer LFM3-style backbone (hidden 2048,
                        FFN 8192, vocab 65536, layers 0-15 gated conv, 16-23 GQA
                        attention 32/8 x 64, RoPE theta 1e6 on 32 dims): a 256-token
                        prompt and the 64 greedy ids the oracle decodes from it
lfm3_synth_greedy_ref.json  the same model and prompt with every GEMV in the
                        reference's own order (numerics = 1: bf16 x, fp32 scales)
lfm3_synth_q4_greedy.json  the same model, prompt and GEMV order with every layer's
                        linears Q4 (all but the attention gate_proj, which stays Q8;
                        the exporter's dtype 6 tensors, .auto/lfm3/export_qlow.py)
lfm3_real_shapes_greedy.json  the real LFM3 backbone's shapes and layer pattern (13 conv,
                        6 full and 5 sliding-window attention layers, head_dim 128,
                        FFN 7680, vocab 128000, 7-tap conv) with synthetic weights
tiny_greedy.json        a 4-layer, hidden-256 model: prompt, ids, last logits digest
kernels.npz             small kernel vectors (Q8_0 GEMV / GEMM, ternary GEMV,
                        attention) with their oracle outputs
Inputs come from the documented splitmix64 generator, so the fixtures are
data only (inputs and expected outputs).
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import pyoracle as orc  # noqa: E402

FULL = dict(hidden=2048, ffn=8192, vocab=65536, nlayers=24, nh=32, nkv=8, hd=64, rot=32, ntaps=3, ctx=2048,
            eps=1e-5, theta=1e6, seed=20261201, attn_mask=0xFF0000)
TINY = dict(hidden=256, ffn=512, vocab=1000, nlayers=4, nh=4, nkv=2, hd=64, rot=32, ntaps=3, ctx=256,
            eps=1e-5, theta=1e6, seed=20261201, attn_mask=0b1010)
# The real LFM3 backbone's shapes and layer pattern (the reference's model:
# hidden 2048, FFN 7680, vocab 128000, 16 q / 4 kv heads of dim 128, 7-tap
# conv; layers 0, 1, 3, 5, ..., 23 conv, 2, 6, ..., 22 full attention (theta 1e6,
# half the dims rotated), 4, 8, ..., 20 sliding-window attention (window 256,
# theta 1e4, all dims rotated)), with synthetic weights.
REAL_ATTN = sum(1 << l for l in range(2, 24, 2))
REAL_SLIDE = sum(1 << l for l in range(4, 24, 4))
REAL = dict(hidden=2048, ffn=7680, vocab=128000, nlayers=24, nh=16, nkv=4, hd=128, rot=64, ntaps=7, ctx=2048,
            eps=1e-5, theta=1e6, seed=20261201, attn_mask=REAL_ATTN, slide_mask=REAL_SLIDE, slide_win=256,
            slide_rot=128, slide_theta=1e4)
PROMPT_SEED = 20261201 + 4 * 5000


def greedy_fixture(cfg, n_prompt, n_steps, path):
    t0 = time.time()
    m = orc.Model(**cfg)
    prompt = orc.gen_tokens(PROMPT_SEED, n_prompt, cfg["vocab"])
    ids = m.greedy(prompt, n_steps)
    m.reset()
    _, lg = m.feed(prompt, True)
    m.close()
    out = {"cfg": cfg, "prompt_seed": PROMPT_SEED, "n_prompt": n_prompt, "prompt": prompt.tolist(),
           "ids": ids.tolist(), "prompt_logits_sha256": hashlib.sha256(lg.tobytes()).hexdigest(),
           "prompt_logits_head": [float(v) for v in lg[:8]]}
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(path, f"{time.time() - t0:.1f}s", ids[:8].tolist())


def kernel_fixture(path):
    d = {}
    for tag, (N, K) in {"g1": (97, 96), "g2": (64, 2048), "g3": (130, 288)}.items():
        W, S = orc.q8_weights(1000 + N + K, N, K)
        x = orc.gen_normal(2000 + N + K, 3 * K).reshape(3, K)
        qx, dx = orc.q8_quant(x)
        d[f"{tag}_W"], d[f"{tag}_S"], d[f"{tag}_x"] = W, S, x
        d[f"{tag}_qx"], d[f"{tag}_dx"], d[f"{tag}_y"] = qx, dx, orc.q8_gemm(W, S, qx, dx)
    N, K = 37, 1024
    codes = orc.gen_ternary(3000, N * K // 4)
    S = orc.gen_scales(3001, N * K // 128)
    x = orc.gen_normal(3002, K)
    xq = orc.q8k_quant(x)
    d.update(t_codes=codes, t_S=S, t_x=x, t_xq=xq, t_y=orc.tq2_gemv(codes, S, xq, N, K))
    nh, nkv, hd, npos = 8, 2, 64, 130
    q = orc.f2bf(orc.gen_normal(4000, nh * hd))
    kc = orc.gen_normal(4001, npos * nkv * hd).astype(np.float16).view(np.uint16)
    vc = orc.gen_normal(4002, npos * nkv * hd).astype(np.float16).view(np.uint16)
    d.update(a_q=q, a_k=kc, a_v=vc, a_out=orc.attn(q, kc, vc, npos, nh, nkv, hd, 0.125))
    np.savez_compressed(path, **d)
    print(path)


if __name__ == "__main__":
    which = sys.argv[1:] or ["kernels", "tiny", "full", "full_ref", "real", "full_q4"]
    if "kernels" in which:
        kernel_fixture(os.path.join(HERE, "kernels.npz"))
    if "tiny" in which:
        greedy_fixture(TINY, 40, 16, os.path.join(HERE, "tiny_greedy.json"))
    if "full" in which:
        greedy_fixture(FULL, 256, 64, os.path.join(HERE, "lfm3_synth_greedy.json"))
    if "real" in which:
        greedy_fixture(REAL, 256, 64, os.path.join(HERE, "lfm3_real_shapes_greedy.json"))
    if "full_ref" in which:
        greedy_fixture(dict(FULL, numerics=1), 256, 64, os.path.join(HERE, "lfm3_synth_greedy_ref.json"))
    if "full_q4" in which:
        greedy_fixture(dict(FULL, numerics=1, lowbit=4, lowbit_mask=0xFFFFFF), 256, 64,
                       os.path.join(HERE, "lfm3_synth_q4_greedy.json"))
