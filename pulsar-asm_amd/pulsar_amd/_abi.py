"""ctypes signatures of every entry point of include/pulsar_amd.h."""
import ctypes as C

P = C.c_void_p
I = C.c_int
Z = C.c_size_t
F = C.c_float
U64 = C.c_uint64


class ModelCfg(C.Structure):
    """pq_model_cfg."""
    _fields_ = [("hidden", C.c_int), ("ffn", C.c_int), ("vocab", C.c_int), ("nlayers", C.c_int),
                ("nh", C.c_int), ("nkv", C.c_int), ("hd", C.c_int), ("rot", C.c_int),
                ("ntaps", C.c_int), ("ctx", C.c_int), ("eps", C.c_float), ("theta", C.c_float),
                ("seed", C.c_uint64), ("attn_mask", C.c_uint32), ("prefill_chunk", C.c_int),
                ("numerics", C.c_int), ("slide_mask", C.c_uint32), ("slide_win", C.c_int),
                ("slide_rot", C.c_int), ("slide_theta", C.c_float)]


class BlobTensor(C.Structure):
    """pq_blob_tensor."""
    _fields_ = [("name", C.c_char * 128), ("dtype", C.c_int), ("ndim", C.c_int), ("ne", C.c_longlong * 4),
                ("ncodes", C.c_longlong), ("nscales", C.c_longlong), ("crc", C.c_uint)]


class GemvPrologue(C.Structure):
    """pq_gemv_prologue."""
    _fields_ = [("kind", C.c_int), ("qx", C.c_void_p), ("dx", C.c_void_p), ("h", C.c_void_p), ("x_in", C.c_void_p),
                ("x_out", C.c_void_p), ("w0", C.c_void_p), ("w1", C.c_void_p), ("eps", C.c_float),
                ("gu", C.c_void_p), ("bcx", C.c_void_p), ("ring_in", C.c_void_p), ("ring_out", C.c_void_p),
                ("taps", C.c_void_p), ("ntaps", C.c_int), ("emb_pc", C.c_void_p), ("emb_ps", C.c_void_p),
                ("tok", C.c_void_p), ("vocab", C.c_int), ("xf", C.c_void_p), ("emb_sf", C.c_void_p)]


SIGNATURES = {
    "pq_version": (C.c_char_p, []),
    "pq_last_error": (C.c_char_p, []),
    "pq_time_next_launch": (I, [P, P]),
    "pq_check_bf16_cvt": (I, [P, P, P]),
    "pq_check_quant_div": (I, [P, P, C.c_uint32, P]),
    "pq_clock_mhz": (I, [P, P]),
    "pq_stream_read": (I, [P, Z, P, P]),
    "pq_q8_quant_f32": (I, [P, P, P, I, I, P]),
    "pq_q8_quant_bf16": (I, [P, P, P, I, I, P]),
    "pq_q8_packed_codes_bytes": (Z, [I, I]),
    "pq_q8_packed_scales_bytes": (Z, [I, I]),
    "pq_q8_pack": (I, [P, P, I, I, P, P, P]),
    "pq_q8_pack_gate_up": (I, [P, P, I, I, P, P, P]),
    "pq_q8_gemv": (I, [P, P, P, P, P, I, I, I, P]),
    "pq_q8_gemm": (I, [P, P, P, P, P, I, I, I, I, P]),
    "pq_q8_gemm_workspace_bytes": (Z, [I, I, I]),
    "pq_q8_gemm_ws": (I, [P, P, P, P, P, I, I, I, I, P, Z, P]),
    "pq_q8r_gemv": (I, [P, P, P, P, I, I, I, I, P]),
    "pq_qlow_packed_codes_bytes": (Z, [I, I, I]),
    "pq_qlow_packed_scales_bytes": (Z, [I, I, I]),
    "pq_qlow_pack": (I, [P, P, I, I, I, P, P, P]),
    "pq_qlow_gemv": (I, [P, P, P, P, I, I, I, I, P]),
    "pq_qlow_workspace_bytes": (Z, [I, I, I]),
    "pq_qlow_gemv_ws": (I, [P, P, P, P, I, I, I, I, P, Z, P]),
    "pq_qlow_gemm": (I, [P, P, P, P, I, I, I, I, I, I, P]),
    "pq_rmsnorm": (I, [P, P, P, P, P, P, P, I, I, F, P]),
    "pq_qk_prep": (I, [P, I, P, P, P, P, P, I, I, I, I, I, I, F, P]),
    "pq_attn_workspace_bytes": (Z, [I, I, I, I]),
    "pq_attn_decode": (I, [P, I, P, P, P, I, P, I, P, P, I, I, I, I, I, F, I, P, Z, P]),
    "pq_qk_prep_ref": (I, [P, I, P, P, P, P, P, I, I, I, I, I, I, F, P]),
    "pq_attn_ref": (I, [P, I, P, P, P, I, P, I, I, I, I, I, I, F, I, P]),
    "pq_attn_decode_ref": (I, [P, P, P, P, P, P, P, P, I, I, I, I, I, F, F, I, P]),
    "pq_attn_decode_ref_q8gate": (I, [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, F, F, I, P]),
    "pq_conv": (I, [P, P, P, P, I, I, I, P]),
    "pq_silu_mul": (I, [P, P, P, P, I, I, P]),
    "pq_silu_mul_interleaved": (I, [P, P, P, P, I, I, P]),
    "pq_argmax": (I, [P, I, P, P]),
    "pq_embed": (I, [P, P, P, P, I, I, I, P]),
    "pq_embed_rows": (I, [P, P, P, P, I, I, I, P]),
    "pq_embed_bf16": (I, [P, P, P, I, I, I, P]),
    "pq_bf16_gemv_parts": (I, [I]),
    "pq_bf16_gemv": (I, [P, P, P, I, I, P, P]),
    "pq_engine_set_q8_f32": (I, [P, I, I, P, P]),
    "pq_q8_gemv_parts": (I, [I, I]),
    "pq_q8_gemv_fused": (I, [P, P, C.POINTER(GemvPrologue), P, I, I, I, P, P]),
    "pq_argmax_parts": (I, [P, I, P, P]),
    "pq_q8r_gemv_fused": (I, [P, P, C.POINTER(GemvPrologue), P, I, I, I, P, P]),
    "pq_qlow_gemv_fused": (I, [P, P, C.POINTER(GemvPrologue), P, I, I, I, I, P]),
    "pq_qlow_gemv_fused_swiglu": (I, [P, P, C.POINTER(GemvPrologue), P, I, I, I, P]),
    "pq_q8r_gemv_parts": (I, [I]),
    "pq_q8r_gemv_fused_swiglu": (I, [P, P, C.POINTER(GemvPrologue), P, I, I, P]),
    "pq_q8_gemv_fused_swiglu": (I, [P, P, C.POINTER(GemvPrologue), P, P, I, I, P]),
    "pq_attn_layer_decode": (I, [P, P, P, P, P, P, I, I, I, I, I, I, F, F, P, P, P, P]),
    "pq_tq2_gemv": (I, [P, P, P, P, I, I, P]),
    "pq_tq2_gemv_batch": (I, [P, P, P, P, I, P, I, P]),
    "pq_q8_gemm_scratch_bytes": (Z, []),
    "pq_q8_gemm_noalloc": (I, [P, P, P, P, P, I, I, I, I, P]),
    "pq_q8k_quant": (I, [P, P, I, I, P]),
    "pq_synth_fill": (I, [I, U64, P, Z, F, F]),
    "pq_engine_create": (P, [C.POINTER(ModelCfg)]),
    "pq_engine_destroy": (I, [P]),
    "pq_engine_load_synthetic": (I, [P]),
    "pq_engine_set_q8": (I, [P, I, I, P, P]),
    "pq_engine_set_f32": (I, [P, I, I, P, Z]),
    "pq_engine_mark_loaded": (I, [P]),
    "pq_engine_load_blob": (I, [P, C.c_char_p]),
    "pq_blob_open": (P, [C.c_char_p]),
    "pq_blob_close": (I, [P]),
    "pq_blob_count": (I, [P]),
    "pq_blob_find": (I, [P, C.c_char_p]),
    "pq_blob_tensor_info": (I, [P, I, C.POINTER(BlobTensor)]),
    "pq_blob_read": (I, [P, I, P, P]),
    "pq_blob_config": (C.c_char_p, [P]),
    "pq_crc32": (C.c_uint, [C.c_uint, P, Z]),
    "pq_engine_reset": (I, [P]),
    "pq_engine_feed": (I, [P, P, I, P, P]),
    "pq_engine_greedy": (I, [P, P, I, I, P]),
    "pq_engine_decode": (I, [P, I, P]),
    "pq_engine_set_fused": (I, [P, I]),
    "pq_engine_set_graph": (I, [P, I]),
    "pq_engine_set_chunk": (I, [P, I]),
    "pq_engine_sync": (I, [P]),
    "pq_engine_stream": (P, [P]),
    "pq_engine_position": (I, [P]),
    "pq_engine_hidden": (I, [P, P]),
    "pq_engine_weight_bytes": (Z, [P]),
}


def bind(lib):
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib
