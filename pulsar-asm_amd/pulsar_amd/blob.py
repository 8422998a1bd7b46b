"""The .lfm3q8 weight blob from Python: the reader over the C ABI (pq_blob_*)
and a writer of the same format (the reference's export_lfm3_q8.py layout:
magic, uint32 header length, JSON header with the tensor table, payloads with
their zlib crc32) for tensors already quantized -- used to hand the engine the
synthetic model as a file."""
import ctypes as C
import json
import struct
import zlib

import numpy as np

from . import PQError, check, lib
from ._abi import BlobTensor

MAGIC = b"LFM3Q8\x01\x00"
T_Q8, T_F32, T_BF16, T_Q4, T_Q5 = 1, 2, 3, 6, 7


class Blob:
    """An open .lfm3q8 file (host memory only; no GPU needed)."""

    def __init__(self, path):
        self.h = lib().pq_blob_open(str(path).encode())
        if not self.h:
            raise PQError("pq_blob_open failed: " + lib().pq_last_error().decode())

    def close(self):
        if self.h:
            lib().pq_blob_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:   # interpreter shutdown
            pass

    def __len__(self):
        return lib().pq_blob_count(self.h)

    def config(self):
        return json.loads(lib().pq_blob_config(self.h).decode())

    def find(self, name):
        return lib().pq_blob_find(self.h, name.encode())

    def info(self, i):
        t = BlobTensor()
        check(lib().pq_blob_tensor_info(self.h, i, C.byref(t)), "pq_blob_tensor_info")
        return {"name": t.name.decode(), "dtype": t.dtype, "ne": list(t.ne[:t.ndim]), "ncodes": t.ncodes,
                "nscales": t.nscales, "crc": t.crc}

    def read(self, name_or_index):
        """Q8: (codes int8 [N][K], scales fp32 [N][K/32]); fp32 / bf16: the array."""
        i = self.find(name_or_index) if isinstance(name_or_index, str) else name_or_index
        if i < 0:
            raise KeyError(name_or_index)
        t = self.info(i)
        codes = np.empty(t["ncodes"], np.uint8)
        scales = np.empty(max(1, t["nscales"]), np.uint8)
        check(lib().pq_blob_read(self.h, i, codes.ctypes.data_as(C.c_void_p), scales.ctypes.data_as(C.c_void_p)),
              "pq_blob_read")
        if t["dtype"] == T_Q8:
            N, K = t["ne"]
            return codes.view(np.int8).reshape(N, K), scales[:t["nscales"]].view(np.float32).reshape(N, K // 32)
        if t["dtype"] in (T_Q4, T_Q5):   # the pre-tiled payload as stored: code bytes, (d', mn) fp16 bits
            return codes, scales[:t["nscales"]].view(np.uint16)
        dt = np.float32 if t["dtype"] == T_F32 else np.uint16
        return codes.view(dt).reshape(t["ne"])


def write_blob(path, cfg, tensors):
    """tensors: list of (name, value) with value (codes int8 [N][K], scales
    fp32 [N][K/32]) for Q8, an fp32 array, ("bf16", uint16 array), or
    ("qlow", bits, N, K, code bytes, scale bits) for a Q4 / Q5 tensor already
    in the exporter's tiled payload (dtype 6 / 7, .auto/lfm3/export_qlow.py)."""
    entries, blobs, off = [], [], 0
    for name, v in tensors:
        if isinstance(v, tuple) and isinstance(v[0], str) and v[0] == "qlow":
            _, bits, N, K, pc, ps = v
            pc = np.ascontiguousarray(pc, np.uint8)
            ps = np.ascontiguousarray(ps, np.uint16)
            assert bits in (4, 5) and N % 32 == 0 and K % 256 == 0
            assert pc.nbytes == N * K // 32 * (16 if bits == 4 else 20) and ps.nbytes == N * K // 32 * 4
            payload = [pc.tobytes(), ps.tobytes()]
            e = dict(name=name, dtype=T_Q4 if bits == 4 else T_Q5, ne=[N, K], off=off, ncodes=pc.nbytes,
                     nscales=ps.nbytes)
        elif isinstance(v, tuple) and len(v) == 2 and not isinstance(v[0], str):
            codes = np.ascontiguousarray(v[0], np.int8)
            scales = np.ascontiguousarray(v[1], np.float32)
            assert codes.ndim == 2 and scales.shape == (codes.shape[0], codes.shape[1] // 32)
            payload = [codes.tobytes(), scales.tobytes()]
            e = dict(name=name, dtype=T_Q8, ne=list(codes.shape), off=off, ncodes=codes.nbytes, nscales=scales.nbytes)
        elif isinstance(v, tuple):
            a = np.ascontiguousarray(v[1], np.uint16)
            payload = [a.tobytes()]
            e = dict(name=name, dtype=T_BF16, ne=list(a.shape), off=off, ncodes=a.nbytes, nscales=0)
        else:
            a = np.ascontiguousarray(v, np.float32)
            payload = [a.tobytes()]
            e = dict(name=name, dtype=T_F32, ne=list(a.shape), off=off, ncodes=a.nbytes, nscales=0)
        crc = 0
        for p in payload:
            crc = zlib.crc32(p, crc)
        e["crc"] = crc & 0xFFFFFFFF
        entries.append(e)
        blobs.extend(payload)
        off += sum(len(p) for p in payload)
    hdr = dict(magic=MAGIC.decode(), cfg=cfg, n_tensors=len(entries), vocab_size=cfg.get("vocab_size", 0),
               hidden_size=cfg.get("hidden_size", 0), data_bytes=off, table=entries)
    hj = json.dumps(hdr, separators=(",", ":")).encode()
    with open(path, "wb") as fh:
        fh.write(MAGIC)
        fh.write(struct.pack("<I", len(hj)))
        fh.write(hj)
        for b in blobs:
            fh.write(b)
