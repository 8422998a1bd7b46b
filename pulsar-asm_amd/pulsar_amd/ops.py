"""Tensor-level wrappers over the C ABI (torch tensors as device memory).

Each wrapper validates shapes and dtypes on the host, calls one C entry point
on torch's current stream and raises PQError with the library's message on a
negative return code.
"""
import torch

from . import check, lib

__all__ = ["stream_ptr", "Q8Weight", "q8_quant", "q8_gemv", "q8_gemm", "DT_F32", "DT_BF16"]

DT_F32 = 0
DT_BF16 = 1


def stream_ptr():
    return torch.cuda.current_stream().cuda_stream


def _ptr(t):
    return t.data_ptr() if t is not None else None


class Q8Weight:
    """A Q8_0 weight in the packed tile layout (from row-major codes/scales)."""

    def __init__(self, codes, scales):
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


def q8_gemm(w, qx, dx, out_dtype=DT_F32, out=None):
    """y [T][N] for T positions (position-first)."""
    T = qx.shape[0]
    if qx.shape[1] != w.K or dx.shape != (T, w.K // 32):
        raise ValueError("x does not match K")
    if out is None:
        out = torch.empty((T, w.N), dtype=torch.float32 if out_dtype == DT_F32 else torch.bfloat16,
                          device=qx.device)
    check(lib().pq_q8_gemm(w.pcodes.data_ptr(), w.pscales.data_ptr(), qx.data_ptr(), dx.data_ptr(),
                           out.data_ptr(), out_dtype, w.N, w.K, T, stream_ptr()), "pq_q8_gemm")
    return out
