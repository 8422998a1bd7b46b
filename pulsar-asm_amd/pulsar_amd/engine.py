"""Python handle on the C++ backbone engine (pq_engine_* in include/pulsar_amd.h)."""
import ctypes as C

import numpy as np

from . import PQError, check, lib
from ._abi import ModelCfg

# The synthetic 24-layer LFM3-style backbone: hidden 2048, FFN 8192, vocab 65536,
# 32 q / 8 kv heads of dim 64 (RoPE on the first 32 dims, theta 1e6), 3-tap
# gated short conv in layers 0-15 and GQA attention in layers 16-23.
LFM3_SYNTH = dict(hidden=2048, ffn=8192, vocab=65536, nlayers=24, nh=32, nkv=8, hd=64, rot=32, ntaps=3,
                  ctx=2048, eps=1e-5, theta=1e6, seed=20261201, attn_mask=0xFF0000, prefill_chunk=256)


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


class Engine:
    def __init__(self, **cfg):
        full = dict(LFM3_SYNTH)
        full.update(cfg)
        self.cfg = full
        self._c = ModelCfg(**full)
        self.h = lib().pq_engine_create(C.byref(self._c))
        if not self.h:
            raise PQError("pq_engine_create failed: " + lib().pq_last_error().decode())

    def close(self):
        if self.h:
            lib().pq_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def load_synthetic(self):
        check(lib().pq_engine_load_synthetic(self.h), "pq_engine_load_synthetic")

    def load_blob(self, path):
        """Every backbone tensor from an .lfm3q8 file (pq_engine_load_blob)."""
        check(lib().pq_engine_load_blob(self.h, str(path).encode()), "pq_engine_load_blob")

    def set_q8(self, layer, slot, codes, scales):
        codes = np.ascontiguousarray(codes, np.int8)
        scales = np.ascontiguousarray(scales, np.uint16)
        check(lib().pq_engine_set_q8(self.h, layer, slot, _p(codes), _p(scales)), "pq_engine_set_q8")

    def set_f32(self, layer, slot, v):
        v = np.ascontiguousarray(v, np.float32)
        check(lib().pq_engine_set_f32(self.h, layer, slot, _p(v), v.size), "pq_engine_set_f32")

    def mark_loaded(self):
        check(lib().pq_engine_mark_loaded(self.h), "pq_engine_mark_loaded")

    def reset(self):
        check(lib().pq_engine_reset(self.h), "pq_engine_reset")

    def feed(self, tokens, want_logits=False):
        tokens = np.ascontiguousarray(tokens, np.int32)
        nid = np.zeros(1, np.int32)
        lg = np.empty(self.cfg["vocab"], np.float32) if want_logits else None
        check(lib().pq_engine_feed(self.h, _p(tokens), tokens.size, _p(nid), _p(lg) if lg is not None else None),
              "pq_engine_feed")
        return (int(nid[0]), lg) if want_logits else int(nid[0])

    def greedy(self, prompt, n_steps):
        prompt = np.ascontiguousarray(prompt, np.int32)
        ids = np.empty(n_steps, np.int32)
        check(lib().pq_engine_greedy(self.h, _p(prompt), prompt.size, n_steps, _p(ids)), "pq_engine_greedy")
        return ids

    def decode(self, n_steps, want_ids=True):
        ids = np.empty(n_steps, np.int32) if want_ids else None
        check(lib().pq_engine_decode(self.h, n_steps, _p(ids) if ids is not None else None), "pq_engine_decode")
        return ids

    def set_fused(self, on):
        check(lib().pq_engine_set_fused(self.h, 1 if on else 0), "pq_engine_set_fused")

    def set_chunk(self, n):
        """Positions per prefill chunk (1 .. the prefill_chunk of the configuration)."""
        check(lib().pq_engine_set_chunk(self.h, n), "pq_engine_set_chunk")

    def set_graph(self, on):
        check(lib().pq_engine_set_graph(self.h, 1 if on else 0), "pq_engine_set_graph")

    def sync(self):
        check(lib().pq_engine_sync(self.h), "pq_engine_sync")

    def stream(self):
        return lib().pq_engine_stream(self.h)

    def position(self):
        return lib().pq_engine_position(self.h)

    def hidden(self):
        out = np.empty(self.cfg["hidden"], np.uint16)
        check(lib().pq_engine_hidden(self.h, _p(out)), "pq_engine_hidden")
        return out

    def weight_bytes(self):
        return lib().pq_engine_weight_bytes(self.h)


def synth_fill(kind, seed, n, a=0.0, b=0.0):
    dt = {0: np.int8, 1: np.float32, 2: np.uint16, 3: np.float32, 4: np.uint8, 5: np.int32}[kind]
    out = np.empty(n, dt)
    check(lib().pq_synth_fill(kind, seed, _p(out), n, a, b), "pq_synth_fill")
    return out
