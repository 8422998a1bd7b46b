"""Tensor-level wrappers over the C ABI (torch tensors as device memory).

Each wrapper validates shapes and dtypes on the host, calls one C entry point
on torch's current stream and raises PQError with the library's message on a
negative return code.
"""
import torch

from . import check, lib

__all__ = ["stream_ptr", "Q8Weight", "q8_quant", "q8_gemv", "q8_gemm", "q8r_gemv", "q8r_gemv_fused", "QlowWeight", "qlow_gemv", "qlow_gemv_fused", "qlow_gemv_fused_swiglu", "qlow_gemm", "DT_F32", "DT_BF16", "rmsnorm", "qk_prep", "qk_prep_ref", "attn_ref", "attn_decode_ref", "attn_decode_ref_q8gate",
           "attn_decode", "conv", "silu_mul", "argmax", "embed", "q8k_quant", "tq2_gemv", "tq2_gemv_batch", "gemv_fused",
           "gemv_fused_swiglu",
           "argmax_parts", "attn_layer_decode", "q8r_gemv_fused_swiglu", "PRO_Q8", "PRO_RESNORM", "PRO_NORM", "PRO_EMBED", "PRO_SILU",
           "PRO_CONV", "PRO_F32"]

PRO_Q8, PRO_RESNORM, PRO_NORM, PRO_EMBED, PRO_SILU, PRO_CONV, PRO_F32 = 0, 1, 2, 3, 4, 5, 6

DT_F32 = 0
DT_BF16 = 1


def stream_ptr():
    return torch.cuda.current_stream().cuda_stream


def _ptr(t):
    return t.data_ptr() if t is not None else None


class Q8Weight:
    """A Q8_0 weight in the packed tile layout (from row-major codes/scales).
    gate_up=True packs a stacked [gate; up] [2F][K] weight with its rows
    interleaved in groups of 32 (pq_q8_pack_gate_up)."""

    def __init__(self, codes, scales, gate_up=False):
        if codes.dtype != torch.int8 or codes.dim() != 2:
            raise ValueError("codes must be int8 [N][K]")
        N, K = codes.shape
        if K % 32:
            raise ValueError("K must be a multiple of 32")
        if scales.dtype not in (torch.int16, torch.uint16, torch.float16) or tuple(scales.shape) != (N, K // 32):
            raise ValueError("scales must be fp16 bits [N][K/32]")
        dev = codes.device
        self.N, self.K = N, K
        L = lib()
        self.pcodes = torch.empty(L.pq_q8_packed_codes_bytes(N, K), dtype=torch.int8, device=dev)
        self.pscales = torch.empty(L.pq_q8_packed_scales_bytes(N, K) // 2, dtype=torch.int16, device=dev)
        codes = codes.contiguous()
        scales = scales.contiguous()
        self.gate_up = gate_up
        if gate_up:
            if N % 64:
                raise ValueError("gate_up weights need 2F rows with F a multiple of 32")
            check(L.pq_q8_pack_gate_up(codes.data_ptr(), scales.data_ptr(), N // 2, K, self.pcodes.data_ptr(),
                                       self.pscales.data_ptr(), stream_ptr()), "pq_q8_pack_gate_up")
        else:
            check(L.pq_q8_pack(codes.data_ptr(), scales.data_ptr(), N, K, self.pcodes.data_ptr(),
                               self.pscales.data_ptr(), stream_ptr()), "pq_q8_pack")

    @property
    def nbytes(self):
        return self.pcodes.numel() + 2 * self.pscales.numel()


def q8_quant(x):
    """x [T][K] fp32 or bf16 -> (qx int8 [T][K], dx fp32 [T][K/32])."""
    squeeze = x.dim() == 1
    x2 = x.reshape(1, -1) if squeeze else x
    T, K = x2.shape
    x2 = x2.contiguous()
    qx = torch.empty((T, K), dtype=torch.int8, device=x.device)
    dx = torch.empty((T, K // 32), dtype=torch.float32, device=x.device)
    L = lib()
    if x2.dtype == torch.float32:
        rc = L.pq_q8_quant_f32(x2.data_ptr(), qx.data_ptr(), dx.data_ptr(), K, T, stream_ptr())
    elif x2.dtype in (torch.bfloat16, torch.int16, torch.uint16):
        rc = L.pq_q8_quant_bf16(x2.data_ptr(), qx.data_ptr(), dx.data_ptr(), K, T, stream_ptr())
    else:
        raise ValueError("x must be fp32 or bf16")
    check(rc, "pq_q8_quant")
    return (qx[0], dx[0]) if squeeze else (qx, dx)


def q8_gemv(w, qx, dx, out_dtype=DT_F32, out=None):
    """y [N] = W . x for one position."""
    if qx.numel() != w.K or dx.numel() != w.K // 32:
        raise ValueError("x does not match K")
    if out is None:
        out = torch.empty(w.N, dtype=torch.float32 if out_dtype == DT_F32 else torch.bfloat16, device=qx.device)
    check(lib().pq_q8_gemv(w.pcodes.data_ptr(), w.pscales.data_ptr(), qx.data_ptr(), dx.data_ptr(), out.data_ptr(),
                           out_dtype, w.N, w.K, stream_ptr()), "pq_q8_gemv")
    return out


def q8_gemm(w, qx, dx, out_dtype=DT_F32, out=None, split=True, ws=None):
    """y [T][N] for T positions (position-first). split=True gives the kernel a
    workspace (pq_q8_gemm_ws) so small-N shapes split K over workgroups."""
    T = qx.shape[0]
    if qx.shape[1] != w.K or dx.shape != (T, w.K // 32):
        raise ValueError("x does not match K")
    if out is None:
        out = torch.empty((T, w.N), dtype=torch.float32 if out_dtype == DT_F32 else torch.bfloat16,
                          device=qx.device)
    nbytes = lib().pq_q8_gemm_workspace_bytes(w.N, w.K, T) if split else 0
    if nbytes and (ws is None or ws.numel() * ws.element_size() < nbytes):
        ws = torch.empty(nbytes, dtype=torch.uint8, device=qx.device)
    check(lib().pq_q8_gemm_ws(w.pcodes.data_ptr(), w.pscales.data_ptr(), qx.data_ptr(), dx.data_ptr(),
                              out.data_ptr(), out_dtype, w.N, w.K, T, _ptr(ws) if nbytes else None, nbytes,
                              stream_ptr()), "pq_q8_gemm")
    return out


def q8_gemm_noalloc(w, qx, dx, out_dtype=DT_F32, out=None):
    """q8_gemm through pq_q8_gemm_noalloc: the split-K partials go to the
    library's own 16 MiB device array (one per GPU), so the call allocates
    nothing when out is given. Every call on one GPU shares that array: calls
    that could overlap on one GPU (two streams, two threads) race and must be
    serialized by the caller -- use one stream per GPU. The first call on each
    GPU looks up the array's address and must be made outside graph capture;
    later calls may be captured."""
    T = qx.shape[0]
    if qx.shape[1] != w.K or dx.shape != (T, w.K // 32):
        raise ValueError("x does not match K")
    if out is None:
        out = torch.empty((T, w.N), dtype=torch.float32 if out_dtype == DT_F32 else torch.bfloat16,
                          device=qx.device)
    check(lib().pq_q8_gemm_noalloc(w.pcodes.data_ptr(), w.pscales.data_ptr(), qx.data_ptr(), dx.data_ptr(),
                                   out.data_ptr(), out_dtype, w.N, w.K, T, stream_ptr()), "pq_q8_gemm_noalloc")
    return out


def q8r_gemv(codes, scales, x, out_dtype=DT_BF16, out=None):
    """The reference's own GEMV numerics (pq_q8r_gemv): codes int8 [N][K],
    fp32 scales [N][K/32], x bf16 [K] or [T][K] -> y [N] or [T][N]."""
    N, K = codes.shape
    if scales.shape != (N, K // 32) or scales.dtype != torch.float32:
        raise ValueError("scales must be fp32 [N][K/32]")
    x2 = x.reshape(-1, K)
    T = x2.shape[0]
    if out is None:
        out = torch.empty((T, N), dtype=torch.float32 if out_dtype == DT_F32 else torch.bfloat16, device=codes.device)
    check(lib().pq_q8r_gemv(codes.data_ptr(), scales.data_ptr(), _bits16(x2), out.data_ptr(), out_dtype, N, K, T,
                            stream_ptr()), "pq_q8r_gemv")
    return out if x.dim() == 2 else out.reshape(N)


class QlowWeight:
    """A Q4 / Q5 tensor packed for pq_qlow_gemv: codes uint8 [N][K] (one code
    per byte, 0 .. 2^bits - 1) and scales fp16 bits [N][K/32][2] (d' = 128 d, mn)."""

    def __init__(self, codes, scales, bits):
        N, K = codes.shape
        if codes.dtype != torch.uint8 or scales.shape != (N, K // 32, 2) or scales.element_size() != 2:
            raise ValueError("codes uint8 [N][K], scales 16-bit [N][K/32][2]")
        self.N, self.K, self.bits = N, K, bits
        nc = lib().pq_qlow_packed_codes_bytes(N, K, bits)
        ns = lib().pq_qlow_packed_scales_bytes(N, K, bits)
        if nc == 0:
            raise ValueError("N a multiple of 32, K of 256, bits 4 or 5")
        self.pcodes = torch.empty(nc, dtype=torch.uint8, device=codes.device)
        self.pscales = torch.empty(ns // 2, dtype=torch.int16, device=codes.device)
        check(lib().pq_qlow_pack(codes.contiguous().data_ptr(), scales.contiguous().data_ptr(), N, K, bits,
                                 self.pcodes.data_ptr(), self.pscales.data_ptr(), stream_ptr()), "pq_qlow_pack")


def qlow_gemv(w, x, out_dtype=DT_BF16, out=None, split=True, ws=None):
    """y [N] = the reference's Q4/Q5 GEMV of x (bf16 [K]); split=True gives
    the kernel a workspace (pq_qlow_gemv_ws) so small N splits K."""
    if out is None:
        out = torch.empty(w.N, dtype=torch.float32 if out_dtype == DT_F32 else torch.bfloat16, device=x.device)
    nbytes = lib().pq_qlow_workspace_bytes(w.N, w.K, w.bits) if split else 0
    if nbytes and (ws is None or ws.numel() * ws.element_size() < nbytes):
        ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    check(lib().pq_qlow_gemv_ws(w.pcodes.data_ptr(), w.pscales.data_ptr(), _bits16(x), out.data_ptr(), out_dtype,
                                w.N, w.K, w.bits, _ptr(ws) if nbytes else None, nbytes, stream_ptr()), "pq_qlow_gemv")
    return out


def qlow_gemm(w, x, out_dtype=DT_BF16, out=None):
    """y [T][N] = the reference's Q4/Q5 GEMV of each row of x (bf16 [T][K]) in
    one launch (pq_qlow_gemm), each row bit for bit as qlow_gemv."""
    T = x.shape[0]
    if x.shape != (T, w.K) or not x.is_contiguous():
        raise ValueError("x must be a contiguous [T][K] tensor")
    if out is None:
        out = torch.empty((T, w.N), dtype=torch.float32 if out_dtype == DT_F32 else torch.bfloat16, device=x.device)
    if out.shape != (T, w.N) or out.stride(1) != 1:
        raise ValueError("out must be [T][N] with unit column stride")
    check(lib().pq_qlow_gemm(w.pcodes.data_ptr(), w.pscales.data_ptr(), _bits16(x), out.data_ptr(), out_dtype,
                             w.N, w.K, T, out.stride(0), w.bits, stream_ptr()), "pq_qlow_gemm")
    return out


def qlow_gemv_fused(w, kind, out_dtype=DT_BF16, out=None, eps=1e-5, **ptrs):
    """The Q4/Q5 GEMV at T = 1 with x from a prologue (pq_qlow_gemv_fused):
    kind RESNORM, NORM, SILU or CONV, ptrs as for gemv_fused."""
    import ctypes as C
    p = _prologue(kind, eps, ptrs)
    if out is None:
        out = torch.empty(w.N, dtype=torch.float32 if out_dtype == DT_F32 else torch.bfloat16, device=w.pcodes.device)
    check(lib().pq_qlow_gemv_fused(w.pcodes.data_ptr(), w.pscales.data_ptr(), C.byref(p), out.data_ptr(), out_dtype,
                                   w.N, w.K, w.bits, stream_ptr()), "pq_qlow_gemv_fused")
    return out


def qlow_gemv_fused_swiglu(w, kind, out=None, eps=1e-5, **ptrs):
    """The FFN's gate/up GEMV on a low-bit [gate | up] tensor (w.N = 2F rows)
    with a RESNORM or NORM prologue and the SwiGLU epilogue
    (pq_qlow_gemv_fused_swiglu): bf16 [F] = silu(gate) * up."""
    import ctypes as C
    p = _prologue(kind, eps, ptrs)
    F = w.N // 2
    if out is None:
        out = torch.empty(F, dtype=torch.bfloat16, device=w.pcodes.device)
    check(lib().pq_qlow_gemv_fused_swiglu(w.pcodes.data_ptr(), w.pscales.data_ptr(), C.byref(p), _bits16(out), F,
                                          w.K, w.bits, stream_ptr()), "pq_qlow_gemv_fused_swiglu")
    return out


# ---------------------------------------------------------------- layer ops
def _bits16(t):
    """bf16 / int16 / uint16 tensor -> its raw 16-bit storage pointer."""
    if t.element_size() != 2:
        raise ValueError("expected a 16-bit tensor")
    return t.data_ptr()


def rmsnorm(x, w0, eps=1e-5, h=None, w1=None, out=True, quant=False):
    """RMSNorm of the rows of x (bf16 [T][H]); residual form when h is given
    (x is updated in place). Returns (y or None, qx or None, dx or None)."""
    T, H = (1, x.numel()) if x.dim() == 1 else x.shape
    y = torch.empty_like(x) if out else None
    qx = torch.empty((T, H), dtype=torch.int8, device=x.device) if quant else None
    dx = torch.empty((T, H // 32), dtype=torch.float32, device=x.device) if quant else None
    check(lib().pq_rmsnorm(_bits16(x), _bits16(h) if h is not None else None, w0.data_ptr(),
                           w1.data_ptr() if w1 is not None else None, _bits16(y) if y is not None else None,
                           _ptr(qx), _ptr(dx), H, T, eps, stream_ptr()), "pq_rmsnorm")
    return y, qx, dx


def qk_prep(qkv, row_stride, q_norm, k_norm, rope_cs, kc, vc, pos0, nh, nkv, hd, rot, T, eps=1e-5):
    check(lib().pq_qk_prep(_bits16(qkv), row_stride, q_norm.data_ptr(), k_norm.data_ptr(), rope_cs.data_ptr(),
                           _bits16(kc), _bits16(vc), pos0, nh, nkv, hd, rot, T, eps, stream_ptr()), "pq_qk_prep")


def qk_prep_ref(qkv, row_stride, q_norm, k_norm, rope_cs, kc, vc, pos0, nh, nkv, hd, rot, T, eps=1e-5):
    """pq_qk_prep with the cache holding the bf16 k / v rows (pq_qk_prep_ref)."""
    check(lib().pq_qk_prep_ref(_bits16(qkv), row_stride, q_norm.data_ptr(), k_norm.data_ptr(), rope_cs.data_ptr(),
                               _bits16(kc), _bits16(vc), pos0, nh, nkv, hd, rot, T, eps, stream_ptr()),
          "pq_qk_prep_ref")


def attn_ref(q, q_stride, kc, vc, pos0, nh, nkv, hd, T, scale, out, out_stride, gate=None, gate_stride=0, win=0):
    """Attention in k_attn_head's order over the bf16 cache (pq_attn_ref)."""
    check(lib().pq_attn_ref(_bits16(q), q_stride, _bits16(kc), _bits16(vc),
                            _bits16(gate) if gate is not None else None, gate_stride, _bits16(out), out_stride, pos0,
                            nh, nkv, hd, T, scale, win, stream_ptr()), "pq_attn_ref")


def attn_decode_ref(qkv, q_norm, k_norm, rope_cs, kc, vc, pos, nh, nkv, hd, rot, scale, out, gate=None, eps=1e-5,
                    win=0):
    """One decode token's qk_prep_ref + attn_ref in one launch (pq_attn_decode_ref)."""
    check(lib().pq_attn_decode_ref(_bits16(qkv), q_norm.data_ptr(), k_norm.data_ptr(), rope_cs.data_ptr(),
                                   _bits16(kc), _bits16(vc), _bits16(gate) if gate is not None else None,
                                   _bits16(out), pos, nh, nkv, hd, rot, eps, scale, win, stream_ptr()),
          "pq_attn_decode_ref")


def attn_decode_ref_q8gate(qkv, q_norm, k_norm, rope_cs, kc, vc, gate_codes, gate_scales, x, x_norm, pos, nh, nkv, hd,
                           rot, scale, out, eps=1e-5, win=0):
    """attn_decode_ref with each head's gate formed in the launch from Q8 rows on rmsnorm(x, x_norm)
    (pq_attn_decode_ref_q8gate)."""
    check(lib().pq_attn_decode_ref_q8gate(_bits16(qkv), q_norm.data_ptr(), k_norm.data_ptr(), rope_cs.data_ptr(),
                                          _bits16(kc), _bits16(vc), gate_codes.data_ptr(), gate_scales.data_ptr(),
                                          _bits16(x), x_norm.data_ptr(), _bits16(out), pos, nh, nkv, hd, rot, eps,
                                          scale, win, stream_ptr()), "pq_attn_decode_ref_q8gate")


def attn_decode(q, q_stride, kc, vc, pos0, nh, nkv, hd, T, scale, gate=None, gate_stride=0, out=None,
                out_stride=0, qx=None, dx=None, ws=None, win=0):
    L = lib()
    need = L.pq_attn_workspace_bytes(nh, hd, pos0 + T, T)
    if ws is None:
        ws = torch.empty(max(need, 4), dtype=torch.uint8, device=q.device)
    check(L.pq_attn_decode(_bits16(q), q_stride, _bits16(kc), _bits16(vc),
                           _bits16(gate) if gate is not None else None, gate_stride,
                           _bits16(out) if out is not None else None, out_stride, _ptr(qx), _ptr(dx), pos0, nh, nkv,
                           hd, T, scale, win, ws.data_ptr(), ws.numel(), stream_ptr()), "pq_attn_decode")


def conv(ring, taps, bcx, out, H, T, ntaps):
    check(lib().pq_conv(_bits16(ring), taps.data_ptr(), _bits16(bcx), _bits16(out), H, T, ntaps, stream_ptr()),
          "pq_conv")


def silu_mul(gu, F, T, out=True, quant=False, interleaved=False):
    y = torch.empty((T, F), dtype=gu.dtype, device=gu.device) if out else None
    qx = torch.empty((T, F), dtype=torch.int8, device=gu.device) if quant else None
    dx = torch.empty((T, F // 32), dtype=torch.float32, device=gu.device) if quant else None
    fn = "pq_silu_mul_interleaved" if interleaved else "pq_silu_mul"
    check(getattr(lib(), fn)(_bits16(gu), _bits16(y) if y is not None else None, _ptr(qx), _ptr(dx), F, T,
                             stream_ptr()), fn)
    return y, qx, dx


def argmax(v):
    out = torch.empty(1, dtype=torch.int32, device=v.device)
    check(lib().pq_argmax(v.data_ptr(), v.numel(), out.data_ptr(), stream_ptr()), "pq_argmax")
    return out


def embed(w, tokens, H, vocab):
    T = tokens.numel()
    out = torch.empty((T, H), dtype=torch.int16, device=tokens.device)
    check(lib().pq_embed(w.pcodes.data_ptr(), w.pscales.data_ptr(), tokens.data_ptr(), out.data_ptr(), H, vocab, T,
                         stream_ptr()), "pq_embed")
    return out


# ------------------------------------------------------------- ternary path
def q8k_quant(x):
    """x fp32 [T][K] -> Q8_K blocks, uint8 [T][K/256*292]."""
    x2 = x.reshape(1, -1) if x.dim() == 1 else x
    T, K = x2.shape
    out = torch.empty((T, K // 256 * 292), dtype=torch.uint8, device=x.device)
    check(lib().pq_q8k_quant(x2.contiguous().data_ptr(), out.data_ptr(), K, T, stream_ptr()), "pq_q8k_quant")
    return out[0] if x.dim() == 1 else out


def tq2_gemv(codes, scales, xq, K, N, out=None):
    """PQ2_0 codes uint8 [N][K/4], fp16 scale bits [N][K/128], Q8_K xq -> y fp32 [N].
    K before N, as pq2_gemv_sm53_launch takes them (pq2_wrap.h:24-28)."""
    if out is None:
        out = torch.empty(N, dtype=torch.float32, device=codes.device)
    check(lib().pq_tq2_gemv(codes.data_ptr(), scales.data_ptr(), xq.data_ptr(), out.data_ptr(), K, N, stream_ptr()),
          "pq_tq2_gemv")
    return out


def tq2_gemv_batch(tensors, xq, K, outs=None):
    """1..3 ternary tensors [(codes, scales), ...] of one K over the same Q8_K
    xq in one launch (pq_tq2_gemv_batch) -> [y fp32 [N_i], ...]."""
    import ctypes as C
    n = len(tensors)
    rows = [int(c.shape[0]) for c, _ in tensors]
    if outs is None:
        outs = [torch.empty(r, dtype=torch.float32, device=xq.device) for r in rows]
    cp = (C.c_void_p * n)(*[c.data_ptr() for c, _ in tensors])
    sp = (C.c_void_p * n)(*[s.data_ptr() for _, s in tensors])
    yp = (C.c_void_p * n)(*[o.data_ptr() for o in outs])
    rp = (C.c_int * n)(*rows)
    check(lib().pq_tq2_gemv_batch(cp, sp, xq.data_ptr(), yp, K, rp, n, stream_ptr()), "pq_tq2_gemv_batch")
    return outs


# ------------------------------------------------------- fused decode path
def _prologue(kind, eps, ptrs):
    from ._abi import GemvPrologue
    p = GemvPrologue()
    p.kind = kind
    p.eps = eps
    for k, v in ptrs.items():
        if k == "emb":
            p.emb_pc, p.emb_ps = v.pcodes.data_ptr(), v.pscales.data_ptr()
        elif k == "emb_rows":   # (codes int8 [vocab][K], fp32 scales [vocab][K/32]): the row-major table
            p.emb_pc, p.emb_sf = v[0].data_ptr(), v[1].data_ptr()
        elif k in ("ntaps", "vocab"):
            setattr(p, k, int(v))
        else:
            setattr(p, k, v.data_ptr())
    return p


def gemv_fused(w, kind, out_dtype=DT_BF16, out=None, parts=None, eps=1e-5, **ptrs):
    """GEMV whose input x is produced by a prologue (pq_q8_gemv_fused). ptrs are
    tensors for the pq_gemv_prologue fields (qx, dx, h, x_in, x_out, w0, w1, gu,
    bcx, ring_in, ring_out, taps, emb (a Q8Weight), tok) plus ints ntaps, vocab."""
    import ctypes as C
    p = _prologue(kind, eps, ptrs)
    if out is None:
        out = torch.empty(w.N, dtype=torch.float32 if out_dtype == DT_F32 else torch.bfloat16, device=w.pcodes.device)
    check(lib().pq_q8_gemv_fused(w.pcodes.data_ptr(), w.pscales.data_ptr(), C.byref(p), out.data_ptr(), out_dtype,
                                 w.N, w.K, _ptr(parts), stream_ptr()), "pq_q8_gemv_fused")
    return out


def q8r_gemv_fused(codes, scales, kind, out_dtype=DT_BF16, out=None, parts=None, eps=1e-5, **ptrs):
    """The reference-numerics GEMV (codes int8 [N][K], fp32 scales [N][K/32])
    at T = 1 with x from a prologue (pq_q8r_gemv_fused): kind RESNORM, NORM,
    SILU or CONV, ptrs as for gemv_fused; parts (fp32, 2 * pq_q8r_gemv_parts(N))
    receives the per-workgroup argmax pairs."""
    import ctypes as C
    N, K = codes.shape
    if scales.shape != (N, K // 32) or scales.dtype != torch.float32:
        raise ValueError("scales must be fp32 [N][K/32]")
    p = _prologue(kind, eps, ptrs)
    if out is None:
        out = torch.empty(N, dtype=torch.float32 if out_dtype == DT_F32 else torch.bfloat16, device=codes.device)
    check(lib().pq_q8r_gemv_fused(codes.data_ptr(), scales.data_ptr(), C.byref(p), out.data_ptr(), out_dtype, N, K,
                                  _ptr(parts), stream_ptr()), "pq_q8r_gemv_fused")
    return out


def q8r_gemv_fused_swiglu(codes, scales, kind, out=None, eps=1e-5, **ptrs):
    """The reference-numerics gate/up GEMV (codes int8 [2F][K]: gate rows, then
    up rows) with a RESNORM or NORM prologue and the silu(gate) * up epilogue
    (pq_q8r_gemv_fused_swiglu): returns y bf16 [F]."""
    import ctypes as C
    N, K = codes.shape
    if scales.shape != (N, K // 32) or scales.dtype != torch.float32:
        raise ValueError("scales must be fp32 [N][K/32]")
    p = _prologue(kind, eps, ptrs)
    if out is None:
        out = torch.empty(N // 2, dtype=torch.bfloat16, device=codes.device)
    check(lib().pq_q8r_gemv_fused_swiglu(codes.data_ptr(), scales.data_ptr(), C.byref(p), out.data_ptr(), N // 2, K,
                                         stream_ptr()), "pq_q8r_gemv_fused_swiglu")
    return out


def gemv_fused_swiglu(w, kind, eps=1e-5, **ptrs):
    """gate/up GEMV (w packed with gate_up=True) with prologue `kind` and the
    silu(gate)*up epilogue: returns the Q8_0 row (qx int8 [F], dx fp32 [F/32])."""
    import ctypes as C
    if not getattr(w, "gate_up", False):
        raise ValueError("gemv_fused_swiglu needs a Q8Weight packed with gate_up=True")
    p = _prologue(kind, eps, ptrs)
    F = w.N // 2
    qx = torch.empty(F, dtype=torch.int8, device=w.pcodes.device)
    dx = torch.empty(F // 32, dtype=torch.float32, device=w.pcodes.device)
    check(lib().pq_q8_gemv_fused_swiglu(w.pcodes.data_ptr(), w.pscales.data_ptr(), C.byref(p), qx.data_ptr(),
                                        dx.data_ptr(), F, w.K, stream_ptr()), "pq_q8_gemv_fused_swiglu")
    return qx, dx


def argmax_parts(parts, nparts):
    out = torch.empty(1, dtype=torch.int32, device=parts.device)
    check(lib().pq_argmax_parts(parts.data_ptr(), nparts, out.data_ptr(), stream_ptr()), "pq_argmax_parts")
    return out


def attn_layer_decode(qkvg, q_norm, k_norm, rope_cs, kc, vc, pos, nh, nkv, hd, rot, scale, eps=1e-5, out=None,
                      win=0, quant=True):
    """The one-launch attention mixer; returns o_proj's Q8_0 input (qx, dx), or
    (None, None) with quant=False (then out, the bf16 output, is required)."""
    if not quant and out is None:
        raise ValueError("quant=False needs out")
    qx = torch.empty(nh * hd, dtype=torch.int8, device=qkvg.device) if quant else None
    dx = torch.empty(nh * hd // 32, dtype=torch.float32, device=qkvg.device) if quant else None
    check(lib().pq_attn_layer_decode(_bits16(qkvg), q_norm.data_ptr(), k_norm.data_ptr(), rope_cs.data_ptr(),
                                     _bits16(kc), _bits16(vc), pos, nh, nkv, hd, rot, win, eps, scale,
                                     _bits16(out) if out is not None else None, _ptr(qx), _ptr(dx),
                                     stream_ptr()), "pq_attn_layer_decode")
    return qx, dx
