"""The oracle's synthetic model written as an .lfm3q8 file under the reference's
tensor names (export_lfm3_q8.py; .auto/lfm3/export_qlow.py for the Q4 / Q5
tensors): Q8 tensors with their fp16 scales widened to fp32 (exact), low-bit
tensors in the exporter's tiled payload, the tied table as Q8 or bf16."""
import numpy as np

from qlow_layout import pack

# the engine's configuration keys (the oracle's extra keys describe the weights)
ORACLE_ONLY = ("emb_bf16", "lowbit", "lowbit_mask")


def engine_cfg(cfg):
    return {k: v for k, v in cfg.items() if k not in ORACLE_ONLY}


def model_blob(orc, cfg, path):
    from pulsar_amd.blob import write_blob
    m = orc.Model(**cfg)
    H, F = cfg["hidden"], cfg["ffn"]

    def sources(layer, slot, names):
        """The slot's source tensors as the blob lists them, Q8 or low-bit."""
        w, s = m.tensor(layer, slot)
        s32 = np.array(s).view(np.float16).astype(np.float32)
        low = m.lowbit(layer, slot)
        out = []
        for (r0, n, bits), nm in zip(m.parts(layer, slot), names):
            if bits == 8:
                out.append((nm, (np.array(w[r0:r0 + n]), s32[r0:r0 + n])))
            else:
                pc, ps = pack(low[0][r0:r0 + n], low[1][r0:r0 + n], bits)
                out.append((nm, ("qlow", bits, n, w.shape[1], pc, ps)))
        return out

    if cfg.get("emb_bf16"):
        ts = [("lfm.model.embed_tokens.weight", ("bf16", np.array(m.tensor(-1, 3))))]
    else:
        w, s = m.tensor(-1, 0)
        ts = [("lfm.model.embed_tokens.weight", (np.array(w), np.array(s).view(np.float16).astype(np.float32)))]
    for l in range(cfg["nlayers"]):
        P = f"lfm.model.layers.{l}."
        if (cfg["attn_mask"] >> l) & 1:
            ts += sources(l, 0, [P + f"self_attn.{nm}.weight" for nm in ("q_proj", "k_proj", "v_proj", "gate_proj")])
            ts += sources(l, 1, [P + "self_attn.o_proj.weight"])
            ts.append((P + "self_attn.q_norm.weight", np.array(m.tensor(l, 8))))
            ts.append((P + "self_attn.k_norm.weight", np.array(m.tensor(l, 9))))
        else:
            ts += sources(l, 0, [P + "conv.in_proj.weight"])
            ts += sources(l, 1, [P + "conv.out_proj.weight"])
            ts.append((P + "conv.conv.weight", np.array(m.tensor(l, 10)).reshape(H, 1, cfg["ntaps"])))
        ts += sources(l, 2, [P + "feed_forward.w1.weight", P + "feed_forward.w3.weight"])
        ts += sources(l, 3, [P + "feed_forward.w2.weight"])
        for slot, nm in ((4, "operator_norm"), (5, "post_operator_norm"), (6, "ffn_norm"), (7, "post_ffn_norm")):
            ts.append((P + nm + ".weight", np.array(m.tensor(l, slot))))
    ts.append(("lfm.model.embedding_norm.weight", np.array(m.tensor(-1, 1))))

    def kind(l):
        if not (cfg["attn_mask"] >> l) & 1:
            return "conv"
        return "sliding_attention" if (cfg.get("slide_mask", 0) >> l) & 1 else "full_attention"

    layer_types = [kind(l) for l in range(cfg["nlayers"])]
    write_blob(path, {"hidden_size": H, "vocab_size": cfg["vocab"], "layer_types": layer_types}, ts)
    m.close()
