"""The C ABI library: it loads without a GPU, exports every declared entry point,
and its host-side checks reject bad arguments before touching the device."""
import os
import re
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pulsar_amd.h")
LIB = os.path.join(ROOT, "pulsar-asm_amd", "pulsar_amd", "libpulsar_amd.so")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pq_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported():
    names = declared()
    assert len(names) >= 8
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (pq_[a-z0-9_]+)$", out, flags=re.M))
    missing = [n for n in names if n not in exported]
    assert not missing, missing


def test_bindings_cover_header():
    from pulsar_amd import _abi
    assert sorted(_abi.SIGNATURES) == declared()


def test_loads_and_rejects_bad_args():
    import pulsar_amd as pq
    L = pq.lib()
    assert L.pq_version().startswith(b"pulsar-amd")
    assert L.pq_q8_packed_codes_bytes(130, 288) == 3 * 9 * 2048
    assert L.pq_q8_packed_scales_bytes(130, 288) == 3 * 2 * 64 * 8 * 2
    assert L.pq_q8_packed_codes_bytes(10, 33) == 0
    assert L.pq_q8_gemv(None, None, None, None, None, 0, 64, 2048, None) == -1
    assert b"null pointer" in L.pq_last_error()
    assert L.pq_q8_quant_f32(8, 8, 8, 33, 1, None) == -1          # K not a multiple of 32
    assert b"multiple of 32" in L.pq_last_error()
    assert L.pq_time_next_launch(None, 8) == -1
    assert L.pq_stream_read(16, 24, 16, None) == -1               # not a multiple of 16 bytes
    assert b"multiple of 16" in L.pq_last_error()


def test_python_wrappers_exported():
    import pulsar_amd as pq
    for name in ("q8_quant", "q8_gemv", "q8_gemm", "rmsnorm", "qk_prep", "attn_decode", "conv", "silu_mul",
                 "argmax", "embed", "Q8Weight"):
        assert callable(getattr(pq, name)), name
    from pulsar_amd.engine import Engine, synth_fill  # noqa: F401
