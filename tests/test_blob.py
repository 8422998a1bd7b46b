"""The .lfm3q8 blob reader (pq_blob_*, host-side: no GPU) against files in the
reference exporter's layout (export_lfm3_q8.py:172-180)."""
import os
import struct
import zlib

import numpy as np
import pytest

from pulsar_amd import PQError, lib
from pulsar_amd.blob import MAGIC, Blob, write_blob


def _tensors(seed=7):
    rng = np.random.default_rng(seed)
    W = rng.integers(-128, 128, (96, 160)).astype(np.int8)   # the exporter clamps to -128..127
    S = (np.abs(rng.standard_normal((96, 5))) * 0.01).astype(np.float32)
    taps = rng.standard_normal((32, 1, 7)).astype(np.float32)
    emb = rng.integers(0, 65535, (10, 32)).astype(np.uint16)
    return [("lfm.model.layers.0.conv.in_proj.weight", (W, S)),
            ("lfm.model.layers.0.conv.conv.weight", taps),
            ("lfm.model.embed_tokens.weight", ("bf16", emb))]


def test_round_trip(tmp_path):
    p = tmp_path / "m.lfm3q8"
    cfg = {"hidden_size": 32, "vocab_size": 10, "layer_types": ["conv", "full_attention"], "rope_theta": 1e6}
    ts = _tensors()
    write_blob(p, cfg, ts)
    b = Blob(p)
    assert len(b) == 3 and b.config() == cfg
    assert b.find("nope") == -1
    i = b.find("lfm.model.layers.0.conv.in_proj.weight")
    info = b.info(i)
    assert info["dtype"] == 1 and info["ne"] == [96, 160] and info["ncodes"] == 96 * 160 and info["nscales"] == 96 * 5 * 4
    c, s = b.read(i)
    assert np.array_equal(c, ts[0][1][0]) and np.array_equal(s.view(np.uint32), ts[0][1][1].view(np.uint32))
    assert np.array_equal(b.read("lfm.model.layers.0.conv.conv.weight"), ts[1][1])
    assert np.array_equal(b.read("lfm.model.embed_tokens.weight"), ts[2][1][1])
    b.close()


def test_crc32_is_zlib():
    L = lib()
    assert L.pq_crc32(0, b"123456789", 9) == 0xCBF43926   # the CRC-32 check value
    rng = np.random.default_rng(3)
    for n in (0, 1, 7, 8, 9, 63, 1000, 4099):
        a = rng.integers(0, 256, n).astype(np.uint8)
        want = zlib.crc32(a.tobytes()) & 0xFFFFFFFF
        assert L.pq_crc32(0, a.ctypes.data, n) == want, n
        if n > 5:   # chained like the reader's 16 MB pieces
            h = L.pq_crc32(0, a.ctypes.data, 5)
            assert L.pq_crc32(h, a[5:].ctypes.data, n - 5) == want


def test_corrupt_payload_is_a_data_error(tmp_path):
    p = tmp_path / "m.lfm3q8"
    write_blob(p, {}, _tensors())
    raw = bytearray(p.read_bytes())
    raw[-100] ^= 0x01                      # a byte of the last tensor's payload
    p.write_bytes(bytes(raw))
    b = Blob(p)
    b.read(0)                              # the others still read
    with pytest.raises(PQError, match="crc mismatch"):
        b.read(b.find("lfm.model.embed_tokens.weight"))


def test_bad_files_are_refused(tmp_path):
    p = tmp_path / "m.lfm3q8"
    write_blob(p, {}, _tensors())
    raw = p.read_bytes()
    cases = {
        "magic": b"LFM3Q9\x01\x00" + raw[8:],
        "truncated": raw[:-10],
        "header length": raw[:8] + struct.pack("<I", len(raw)) + raw[12:],
        "not json": raw[:12] + b"{" * (len(raw) - 12),
    }
    for why, data in cases.items():
        q = tmp_path / ("bad_" + why.replace(" ", "_"))
        q.write_bytes(data)
        with pytest.raises(PQError):
            Blob(q)
    # a payload size that does not match the shape and dtype
    n = struct.unpack("<I", raw[8:12])[0]
    hj = raw[12:12 + n].replace(b'"ne":[96,160]', b'"ne":[96,128]')
    q = tmp_path / "bad_shape"
    q.write_bytes(raw[:8] + struct.pack("<I", len(hj)) + hj + raw[12 + n:])
    with pytest.raises(PQError, match="does not match"):
        Blob(q)
    with pytest.raises(PQError):
        Blob(tmp_path / "missing.lfm3q8")


def test_header_matches_exporter_layout(tmp_path):
    """Magic, little-endian uint32 length, compact JSON with the exporter's
    keys (export_lfm3_q8.py:172-180), payloads back to back from 12 + n."""
    p = tmp_path / "m.lfm3q8"
    ts = _tensors()
    write_blob(p, {"hidden_size": 32}, ts)
    raw = p.read_bytes()
    assert raw[:8] == MAGIC
    n = struct.unpack("<I", raw[8:12])[0]
    import json
    h = json.loads(raw[12:12 + n])
    assert list(h) == ["magic", "cfg", "n_tensors", "vocab_size", "hidden_size", "data_bytes", "table"]
    assert list(h["table"][0]) == ["name", "dtype", "ne", "off", "ncodes", "nscales", "crc"]
    assert h["data_bytes"] == len(raw) - 12 - n
    e = h["table"][0]
    body = raw[12 + n + e["off"]:12 + n + e["off"] + e["ncodes"] + e["nscales"]]
    assert zlib.crc32(body) & 0xFFFFFFFF == e["crc"]


def _rewrite_entry(raw, idx, **fields):
    """The blob with table entry idx's fields replaced (header re-serialized
    compactly; payload offsets are relative to the data start, so they hold)."""
    import json
    n = struct.unpack("<I", raw[8:12])[0]
    h = json.loads(raw[12:12 + n])
    h["table"][idx].update(fields)
    hj = json.dumps(h, separators=(",", ":")).encode()
    return raw[:8] + struct.pack("<I", len(hj)) + hj + raw[12 + n:]


def test_oversized_sizes_are_refused(tmp_path):
    """Shape products and offsets that would overflow 64 bits (or wrap the
    end-of-payload sum) are refused, not taken as small tensors."""
    p = tmp_path / "m.lfm3q8"
    write_blob(p, {}, _tensors())
    raw = p.read_bytes()
    cases = {
        # 2^96 elements: wraps to 0 in 64 bits, so ncodes 0 would have matched
        "wrap_ne": dict(dtype=2, ne=[2 ** 32, 2 ** 32, 2 ** 32], ncodes=0, nscales=0),
        "big_ne": dict(dtype=3, ne=[10 ** 12, 10 ** 12], ncodes=2 * 10 ** 24 % 2 ** 64, nscales=0),
        "big_off": dict(off=2 ** 64 - 2048),
        "big_ncodes": dict(dtype=2, ne=[2 ** 61], ncodes=2 ** 63, nscales=0),
    }
    for why, f in cases.items():
        q = tmp_path / why
        q.write_bytes(_rewrite_entry(raw, 1, **f))
        with pytest.raises(PQError):
            Blob(q)


def _raw_blob(path, entries, payloads):
    """A file with a hand-written table (for sizes write_blob would refuse)."""
    import json
    hj = json.dumps(dict(magic=MAGIC.decode(), cfg={}, n_tensors=len(entries), table=entries)).encode()
    with open(path, "wb") as fh:
        fh.write(MAGIC)
        fh.write(struct.pack("<I", len(hj)))
        fh.write(hj)
        for b in payloads:
            fh.write(b)


@pytest.mark.parametrize("bits", [4, 5])
def test_lowbit_tensors(tmp_path, bits):
    """Q4 / Q5 tensors (dtype 6 / 7, the pre-tiled payload of
    .auto/lfm3/export_qlow.py): N a multiple of 32, K of 256, N*K/32 groups of
    16 (Q4) or 20 (Q5) code bytes, then 4 bytes of (d', mn) per group, as the
    reference's loader checks them (lfm3_nanode.cu:1494-1500). The payload reads
    back as stored; a size or shape off that rule is refused."""
    rng = np.random.default_rng(bits)
    N, K = 64, 512
    G = N * K // 32
    pc = rng.integers(0, 256, G * (16 if bits == 4 else 20)).astype(np.uint8)
    ps = rng.integers(0, 65536, G * 2).astype(np.uint16)
    p = tmp_path / "q.lfm3q8"
    write_blob(p, {}, [("lfm.model.layers.0.feed_forward.w2.weight", ("qlow", bits, N, K, pc, ps))])
    b = Blob(p)
    t = b.info(0)
    assert t["dtype"] == (6 if bits == 4 else 7) and t["ne"] == [N, K]
    c, s = b.read(0)
    assert np.array_equal(c, pc) and np.array_equal(s, ps)
    b.close()
    dt = 6 if bits == 4 else 7
    for (n, k, nc, ns) in ((N, K, pc.nbytes - 16, ps.nbytes), (N, K, pc.nbytes, ps.nbytes + 4),
                           (40, K, 40 * K // 32 * (pc.nbytes // G), 40 * K // 32 * 4),
                           (N, 480, N * 15 * (pc.nbytes // G), N * 15 * 4)):
        q = tmp_path / "bad.lfm3q8"
        payload = bytes(nc + ns)
        _raw_blob(q, [dict(name="w", dtype=dt, ne=[n, k], off=0, ncodes=nc, nscales=ns,
                           crc=zlib.crc32(payload) & 0xFFFFFFFF)], [payload])
        with pytest.raises(PQError, match="does not match its shape"):
            Blob(q)
