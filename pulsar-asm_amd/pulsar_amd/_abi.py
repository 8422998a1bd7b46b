"""ctypes signatures of every entry point of include/pulsar_amd.h."""
import ctypes as C

P = C.c_void_p
I = C.c_int
Z = C.c_size_t
F = C.c_float

SIGNATURES = {
    "pq_version": (C.c_char_p, []),
    "pq_last_error": (C.c_char_p, []),
    "pq_time_next_launch": (I, [P, P]),
    "pq_q8_quant_f32": (I, [P, P, P, I, I, P]),
    "pq_q8_quant_bf16": (I, [P, P, P, I, I, P]),
    "pq_q8_packed_codes_bytes": (Z, [I, I]),
    "pq_q8_packed_scales_bytes": (Z, [I, I]),
    "pq_q8_pack": (I, [P, P, I, I, P, P, P]),
    "pq_q8_gemv": (I, [P, P, P, P, P, I, I, I, P]),
    "pq_q8_gemm": (I, [P, P, P, P, P, I, I, I, I, P]),
}


def bind(lib):
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib
