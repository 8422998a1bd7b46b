"""ctypes view of the oracle library (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module. It loads oracle/_build/liboracle.so (and oracle/_ref/libref.so
when present) and wraps the C restatement with numpy arrays.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

QBLK = 32
CHUNK = 8
ATT_SPLIT = 64
Q8K_BYTES = 292


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "_build", "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError("oracle not built: run python oracle/build.py")
        L = C.CDLL(path)
        L.orc_bf2f.restype = C.c_float
        L.orc_bf2f.argtypes = [C.c_uint16]
        L.orc_f2bf.restype = C.c_uint16
        L.orc_f2bf.argtypes = [C.c_float]
        L.orc_h2f.restype = C.c_float
        L.orc_h2f.argtypes = [C.c_uint16]
        L.orc_f2h.restype = C.c_uint16
        L.orc_f2h.argtypes = [C.c_float]
        L.orc_expf.restype = C.c_float
        L.orc_expf.argtypes = [C.c_float]
        L.orc_sm64_at.restype = C.c_uint64
        L.orc_sm64_at.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_argmax.restype = C.c_int
        L.orc_pairwise.restype = C.c_float
        L.orc_rms_sumsq.restype = C.c_float
        L.orc_head_sumsq.restype = C.c_float
        L.orc_model_create.restype = C.c_void_p
        L.orc_model_feed.restype = C.c_int
        L.orc_model_tensor.restype = C.c_int
        _LIB = L
    return _LIB


def ref():
    """The reference's own CPU routines (oracle/_ref), or None if not built."""
    global _REF
    if _REF is None:
        path = os.path.join(HERE, "_ref", "libref.so")
        if not os.path.exists(path):
            return None
        _REF = C.CDLL(path)
        _REF.pq2_h2f.restype = C.c_float
        _REF.pq2_h2f.argtypes = [C.c_uint16]
    return _REF


# ------------------------------------------------------------------ generator
def gen_codes(seed, n):
    out = np.empty(n, np.int8)
    lib().orc_gen_codes(C.c_uint64(seed), _p(out), C.c_size_t(n))
    return out


def gen_normal(seed, n):
    out = np.empty(n, np.float32)
    lib().orc_gen_normal(C.c_uint64(seed), _p(out), C.c_size_t(n))
    return out


def gen_scales(seed, n, mult=0.01):
    out = np.empty(n, np.uint16)
    lib().orc_gen_scales(C.c_uint64(seed), _p(out), C.c_size_t(n), C.c_float(mult))
    return out


def gen_affine(seed, n, a, b):
    out = np.empty(n, np.float32)
    lib().orc_gen_affine(C.c_uint64(seed), _p(out), C.c_size_t(n), C.c_float(a), C.c_float(b))
    return out


def gen_ternary(seed, nbytes):
    out = np.empty(nbytes, np.uint8)
    lib().orc_gen_ternary(C.c_uint64(seed), _p(out), C.c_size_t(nbytes))
    return out


def gen_tokens(seed, n, vocab):
    out = np.empty(n, np.int32)
    lib().orc_gen_tokens(C.c_uint64(seed), _p(out), C.c_int(n), C.c_int(vocab))
    return out


def q8_weights(seed, N, K):
    """Row-major int8 codes [N][K] and fp16 scale bits [N][K/32]."""
    w = gen_codes(seed, N * K).reshape(N, K)
    s = gen_scales(seed + 1, N * (K // QBLK)).reshape(N, K // QBLK)
    return w, s


# ----------------------------------------------------------------- quantizers
def q8_quant(x):
    x = np.ascontiguousarray(x, np.float32)
    T = x.shape[0] if x.ndim == 2 else 1
    K = x.shape[-1]
    qx = np.empty((T, K), np.int8)
    dx = np.empty((T, K // QBLK), np.float32)
    xr = x.reshape(T, K)
    for t in range(T):
        lib().orc_q8_quant(_p(xr[t]), C.c_int(K), _p(qx[t]), _p(dx[t]))
    if x.ndim == 1:
        return qx[0], dx[0]
    return qx, dx


def q8_quant_bf16(xb):
    xb = np.ascontiguousarray(xb, np.uint16)
    K = xb.shape[-1]
    T = xb.size // K
    qx = np.empty((T, K), np.int8)
    dx = np.empty((T, K // QBLK), np.float32)
    xr = xb.reshape(T, K)
    for t in range(T):
        lib().orc_q8_quant_bf16(_p(xr[t]), C.c_int(K), _p(qx[t]), _p(dx[t]))
    if xb.ndim == 1:
        return qx[0], dx[0]
    return qx, dx


def q8k_quant(x):
    x = np.ascontiguousarray(x, np.float32)
    K = x.size
    out = np.empty((K // 256) * Q8K_BYTES, np.uint8)
    lib().orc_q8k_quant(_p(x), C.c_int(K), _p(out))
    return out


# --------------------------------------------------------------------- GEMVs
def q8_gemv(W, S, qx, dx):
    N, K = W.shape
    y = np.empty(N, np.float32)
    lib().orc_q8_gemv(_p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(S)),
                      _p(np.ascontiguousarray(qx)), _p(np.ascontiguousarray(dx, np.float32)),
                      _p(y), C.c_int(N), C.c_int(K))
    return y


def q8_gemm(W, S, qx, dx):
    N, K = W.shape
    T = qx.shape[0]
    y = np.empty((T, N), np.float32)
    lib().orc_q8_gemm(_p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(S)),
                      _p(np.ascontiguousarray(qx)), _p(np.ascontiguousarray(dx, np.float32)),
                      _p(y), C.c_int(N), C.c_int(K), C.c_int(T))
    return y


def q8_gemv_a11(W, S32, x):
    N, K = W.shape
    y = np.empty(N, np.float32)
    lib().orc_q8_gemv_a11(_p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(S32, np.float32)),
                          _p(np.ascontiguousarray(x, np.float32)), _p(y), C.c_int(N), C.c_int(K))
    return y


def q8r_gemm(W, S32, xb):
    """R2 (the reference's GEMV order): codes [N][K], fp32 scales [N][K/32],
    x bf16 bits [T][K] (or [K]) -> y fp32 [T][N] (or [N])."""
    N, K = W.shape
    xb2 = np.ascontiguousarray(xb, np.uint16).reshape(-1, K)
    T = xb2.shape[0]
    y = np.empty((T, N), np.float32)
    lib().orc_q8r_gemm(_p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(S32, np.float32)), _p(xb2), _p(y),
                       C.c_int(N), C.c_int(K), C.c_int(T))
    return y if np.ndim(xb) == 2 else y[0]


def qlow_gemv(Q, S, xb):
    """Q4/Q5 (reference order): codes uint8 [N][K] (one per byte), S fp16 bits
    [N][K/32][2] (d' = 128 d, mn), x bf16 bits [K] -> y fp32 [N]."""
    N, K = Q.shape
    y = np.empty(N, np.float32)
    lib().orc_qlow_gemv(_p(np.ascontiguousarray(Q, np.uint8)), _p(np.ascontiguousarray(S, np.uint16)),
                        _p(np.ascontiguousarray(xb, np.uint16)), _p(y), C.c_int(N), C.c_int(K))
    return y


def bf16_gemv(W, xb):
    """The bf16-table LM head (k_gemv_bf16 order): W bf16 bits [N][K], x bf16
    bits [K] -> y fp32 [N]."""
    N, K = W.shape
    y = np.empty(N, np.float32)
    lib().orc_bf16_gemv(_p(np.ascontiguousarray(W, np.uint16)), _p(np.ascontiguousarray(xb, np.uint16)), _p(y),
                        C.c_int(N), C.c_int(K))
    return y


def q8_gemv_exact(W, S, qx, dx):
    N, K = W.shape
    y = np.empty(N, np.float64)
    lib().orc_q8_gemv_exact(_p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(S)),
                            _p(np.ascontiguousarray(qx)), _p(np.ascontiguousarray(dx, np.float32)),
                            _p(y), C.c_int(N), C.c_int(K))
    return y


def tq2_gemv(codes, S, xq, N, K):
    y = np.empty(N, np.float32)
    lib().orc_tq2_gemv(_p(np.ascontiguousarray(codes)), _p(np.ascontiguousarray(S)),
                       _p(np.ascontiguousarray(xq)), _p(y), C.c_int(N), C.c_int(K))
    return y


# ----------------------------------------------------------- layer primitives
def f2bf(x):
    x = np.ascontiguousarray(x, np.float32)
    return np.array([lib().orc_f2bf(float(v)) for v in x.ravel()], np.uint16).reshape(x.shape)


def bf2f(b):
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def expf(x):
    x = np.ascontiguousarray(x, np.float32)
    return np.array([lib().orc_expf(float(v)) for v in x.ravel()], np.float32).reshape(x.shape)


def rmsnorm(x, w, eps=1e-5):
    x = np.ascontiguousarray(x, np.uint16)
    n = x.shape[-1]
    y = np.empty_like(x)
    xr, yr = x.reshape(-1, n), y.reshape(-1, n)
    for t in range(xr.shape[0]):
        lib().orc_rmsnorm(_p(xr[t]), _p(np.ascontiguousarray(w, np.float32)), _p(yr[t]),
                          C.c_int(n), C.c_float(eps))
    return y


def rms_sumsq(x):
    """RMSNorm's sum of squares of bf16 x in rmsnorm_body's order."""
    x = np.ascontiguousarray(x, np.uint16)
    return np.float32(lib().orc_rms_sumsq(_p(x), C.c_int(x.size)))


def head_sumsq(x):
    """A head norm's sum of squares of bf16 x [hd] in k_headnorm's order."""
    x = np.ascontiguousarray(x, np.uint16)
    return np.float32(lib().orc_head_sumsq(_p(x), C.c_int(x.size)))


def headnorm(x, w, nheads, hd, eps=1e-5):
    x = np.array(x, np.uint16, copy=True)
    lib().orc_headnorm(_p(x), _p(np.ascontiguousarray(w, np.float32)), C.c_int(nheads), C.c_int(hd),
                       C.c_float(eps))
    return x


def rope_invf(hd, rot, theta):
    invf = np.empty(hd // 2, np.float32)
    lib().orc_rope_invf(_p(invf), C.c_int(hd), C.c_int(rot), C.c_float(theta))
    return invf


def rope_table(maxpos, hd, rot, theta):
    cs = np.empty(maxpos * (rot // 2) * 2 + 2, np.float32)
    lib().orc_rope_table(_p(cs), C.c_int(maxpos), C.c_int(hd), C.c_int(rot), C.c_float(theta))
    return cs[: maxpos * (rot // 2) * 2]


def rope(x, cs, pos, nheads, hd, rot):
    x = np.array(x, np.uint16, copy=True)
    lib().orc_rope(_p(x), _p(np.ascontiguousarray(cs, np.float32)), C.c_int(pos), C.c_int(nheads),
                   C.c_int(hd), C.c_int(rot))
    return x


def attn(q, Kc, Vc, npos, nh, nkv, hd, scale, win=0):
    out = np.empty(nh * hd, np.uint16)
    lib().orc_attn(_p(np.ascontiguousarray(q, np.uint16)), _p(np.ascontiguousarray(Kc, np.uint16)),
                   _p(np.ascontiguousarray(Vc, np.uint16)), _p(out), C.c_int(npos), C.c_int(nh),
                   C.c_int(nkv), C.c_int(hd), C.c_float(scale), C.c_int(win))
    return out


def attn_ref(q, Kc, Vc, npos, nh, nkv, hd, scale, win=0):
    """k_attn_head's order over a bf16 cache (orc_attn_ref); returns bf16 [nh*hd]."""
    out = np.empty(nh * hd, np.uint16)
    lib().orc_attn_ref(_p(np.ascontiguousarray(q, np.uint16)), _p(np.ascontiguousarray(Kc, np.uint16)),
                       _p(np.ascontiguousarray(Vc, np.uint16)), _p(out), C.c_int(npos), C.c_int(nh), C.c_int(nkv),
                       C.c_int(hd), C.c_float(scale), C.c_int(win))
    return out


def attn_twopass(q, Kc, Vc, npos, nh, nkv, hd, scale, win=0):
    out = np.empty(nh * hd, np.float32)
    lib().orc_attn_twopass(_p(np.ascontiguousarray(q, np.uint16)), _p(np.ascontiguousarray(Kc, np.uint16)),
                           _p(np.ascontiguousarray(Vc, np.uint16)), _p(out), C.c_int(npos), C.c_int(nh),
                           C.c_int(nkv), C.c_int(hd), C.c_float(scale), C.c_int(win))
    return out


def conv_step(ring, taps, bcx, H, ntaps):
    """Returns (out, new ring); ring is not modified."""
    ring = np.array(ring, np.uint16, copy=True)
    out = np.empty(H, np.uint16)
    lib().orc_conv_step(_p(ring), _p(np.ascontiguousarray(taps, np.float32)),
                        _p(np.ascontiguousarray(bcx, np.uint16)), _p(out), C.c_int(H), C.c_int(ntaps))
    return out, ring


def _ew(fn, a, b):
    a = np.ascontiguousarray(a, np.uint16)
    y = np.empty_like(a)
    fn(_p(a), _p(np.ascontiguousarray(b, np.uint16)), _p(y), C.c_int(a.size))
    return y


def add(a, b):
    return _ew(lib().orc_add, a, b)


def mul(a, b):
    return _ew(lib().orc_mul, a, b)


def silu_mul(a, b):
    return _ew(lib().orc_silu_mul, a, b)


def sigmoid_gate(g, a, nh, hd):
    a = np.array(a, np.uint16, copy=True)
    lib().orc_sigmoid_gate(_p(np.ascontiguousarray(g, np.uint16)), _p(a), C.c_int(nh), C.c_int(hd))
    return a


def argmax(v):
    v = np.ascontiguousarray(v, np.float32)
    return lib().orc_argmax(_p(v), C.c_int(v.size))


def embed_row(W, S, tok):
    K = W.shape[1]
    out = np.empty(K, np.uint16)
    lib().orc_embed_row(_p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(S)), C.c_int(tok),
                        C.c_int(K), _p(out))
    return out


# ------------------------------------------------------------------- backbone
class Cfg(C.Structure):
    _fields_ = [("hidden", C.c_int), ("ffn", C.c_int), ("vocab", C.c_int), ("nlayers", C.c_int),
                ("nh", C.c_int), ("nkv", C.c_int), ("hd", C.c_int), ("rot", C.c_int),
                ("ntaps", C.c_int), ("ctx", C.c_int), ("eps", C.c_float), ("theta", C.c_float),
                ("seed", C.c_uint64), ("attn_mask", C.c_uint32), ("numerics", C.c_int),
                ("slide_mask", C.c_uint32), ("slide_win", C.c_int), ("slide_rot", C.c_int),
                ("slide_theta", C.c_float), ("emb_bf16", C.c_int), ("lowbit", C.c_int),
                ("lowbit_mask", C.c_uint32)]


class Model:
    """The CPU backbone; cfg is a dict with the Cfg field names."""

    def __init__(self, **cfg):
        self.cfg = dict(cfg)
        self._c = Cfg(**cfg)
        self._h = lib().orc_model_create(C.byref(self._c))
        if not self._h:
            raise ValueError("orc_model_create refused the configuration")

    def close(self):
        if self._h:
            lib().orc_model_free(C.c_void_p(self._h))
            self._h = None

    def __del__(self):
        self.close()

    def reset(self):
        lib().orc_model_reset(C.c_void_p(self._h))

    def feed(self, toks, want_logits=False):
        toks = np.ascontiguousarray(toks, np.int32)
        lg = np.empty(self.cfg["vocab"], np.float32) if want_logits else None
        r = lib().orc_model_feed(C.c_void_p(self._h), _p(toks), C.c_int(toks.size),
                                 _p(lg) if lg is not None else None)
        if r < 0:
            raise RuntimeError("context overflow")
        return (r, lg) if want_logits else r

    def greedy(self, prompt, n_steps):
        prompt = np.ascontiguousarray(prompt, np.int32)
        ids = np.empty(n_steps, np.int32)
        lib().orc_model_greedy(C.c_void_p(self._h), _p(prompt), C.c_int(prompt.size),
                               C.c_int(n_steps), _p(ids))
        return ids

    def parts(self, layer, slot):
        """The slot's source tensors: [(row offset, rows, bits)], bits 8 = Q8, 4 / 5 = low-bit."""
        r0, n, b = (C.c_int * 4)(), (C.c_int * 4)(), (C.c_int * 4)()
        k = lib().orc_model_parts(C.c_void_p(self._h), C.c_int(layer), C.c_int(slot), r0, n, b)
        if k < 0:
            raise KeyError((layer, slot))
        return [(r0[i], n[i], b[i]) for i in range(k)]

    def lowbit(self, layer, slot):
        """The slot's low-bit codes uint8 [N][K] and scales fp16 bits [N][K/32][2], or None."""
        q, sc = C.c_void_p(), C.c_void_p()
        n, k = C.c_int(), C.c_int()
        if lib().orc_model_lowbit(C.c_void_p(self._h), C.c_int(layer), C.c_int(slot), C.byref(q), C.byref(sc),
                                  C.byref(n), C.byref(k)) != 0:
            return None
        N, K = n.value, k.value
        return (np.ctypeslib.as_array(C.cast(q, C.POINTER(C.c_uint8)), shape=(N, K)),
                np.ctypeslib.as_array(C.cast(sc, C.POINTER(C.c_uint16)), shape=(N, K // QBLK, 2)))

    def hidden(self):
        out = np.empty(self.cfg["hidden"], np.uint16)
        lib().orc_model_debug_hidden(C.c_void_p(self._h), _p(out))
        return out

    def tensor(self, layer, slot):
        p0, p1 = C.c_void_p(), C.c_void_p()
        n, k = C.c_int(), C.c_int()
        r = lib().orc_model_tensor(C.c_void_p(self._h), C.c_int(layer), C.c_int(slot), C.byref(p0),
                                   C.byref(p1), C.byref(n), C.byref(k))
        if r != 0:
            raise KeyError((layer, slot))
        N, K = n.value, k.value
        if p1.value:
            w = np.ctypeslib.as_array(C.cast(p0, C.POINTER(C.c_int8)), shape=(N, K))
            s = np.ctypeslib.as_array(C.cast(p1, C.POINTER(C.c_uint16)), shape=(N, K // QBLK))
            return w, s
        if layer == -1 and slot == 2:
            return np.ctypeslib.as_array(C.cast(p0, C.POINTER(C.c_float)), shape=(N * (K // 2) * 2,))
        if layer == -1 and slot == 3:   # the bf16 table
            return np.ctypeslib.as_array(C.cast(p0, C.POINTER(C.c_uint16)), shape=(N, K))
        return np.ctypeslib.as_array(C.cast(p0, C.POINTER(C.c_float)), shape=(K,))
