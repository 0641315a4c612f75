"""The library's reader of compiled model stores (tlm_hip_manifest_*,
tlm_hip_packet_read, tlm_hip_dir_find) on the store that the reference's own
compiler writes for the 4-layer synthetic model (oracle/make_c1.sh), checked
against what the reference recorded for that store and against the
reference's own reader (tlm_manifest_load, tlm_packet_verify in oracle/_ref),
plus corruption cases its loader rejects (src/lib/tlm_packet.c:673-815).
CPU only: the reader is host code."""
import ctypes as C
import hashlib
import os
import shutil
import struct

import numpy as np
import pytest

from tierlm_amd._lib import HipError, lib
from tierlm_amd.packet import LAYER_NONE, PK_DENSE, PK_EMBED, PK_EXPERT, PK_META, Manifest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
C1 = os.path.join(ROOT, "oracle", "_ref", "c1", "c1.tlmm")
needs_c1 = pytest.mark.skipif(not os.path.exists(C1), reason="oracle/_ref/c1 not built (oracle/make_c1.sh)")


def crc32c_bytes(b):
    return lib.tlm_hip_crc32c(0, C.c_char_p(bytes(b)), len(b))


def test_crc32c_and_sha256_known_answers():
    assert crc32c_bytes(b"123456789") == 0xE3069283            # the CRC-32C check value
    assert crc32c_bytes(b"") == 0
    assert crc32c_bytes(bytes(32)) == 0x8A9136AA                # RFC 3720 B.4: 32 zero bytes
    assert crc32c_bytes(bytes([0xFF] * 32)) == 0x62A8AB43       # RFC 3720 B.4: 32 x 0xFF
    rng = np.random.default_rng(0)
    for n in (1, 7, 8, 63, 64, 65, 1000, 4096 + 3):
        b = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        out = (C.c_uint8 * 32)()
        lib.tlm_hip_sha256(C.c_char_p(b), n, out)
        assert bytes(out) == hashlib.sha256(b).digest(), n
        # chained CRC over a split equals the CRC of the whole
        assert lib.tlm_hip_crc32c(crc32c_bytes(b[:n // 2]), C.c_char_p(b[n // 2:]), n - n // 2) == crc32c_bytes(b)


@needs_c1
def test_c1_store_matches_recorded_values():
    """The synthetic model's store: geometry, sample packet CRCs and the
    SHA-256 over every (type, layer, id, crc32c, total_len) record, as
    recorded when the reference was surveyed."""
    m = Manifest(C1)
    g = m.geom
    assert (g.n_layers, g.d_model, g.n_heads, g.n_kv_heads, g.head_dim) == (4, 512, 8, 2, 64)
    assert (g.vocab, g.n_experts, g.top_k, g.d_expert, g.n_shared) == (4096, 32, 4, 256, 1)
    crc = {(p.type, p.layer, p.id): p.crc32c for p in m.packets()}
    assert crc[(PK_DENSE, 0, 0)] == 0xf76c97e8
    assert crc[(PK_EXPERT, 0, 0)] == 0x74f32156
    assert crc[(PK_EXPERT, 3, 31)] == 0xba0c5570
    assert crc[(PK_EMBED, LAYER_NONE, 0)] == 0xb182b0d6
    assert crc[(PK_META, LAYER_NONE, 0)] == 0x29e008b8
    recs = b"".join(struct.pack("<HHIIQ", p.type, p.layer, p.id, p.crc32c, p.total_len) for p in m.packets())
    assert hashlib.sha256(recs).hexdigest() == "678dc02ba5d5b4cc3d8306eba7fe2bc96d9d58885ad4bff6c90276183051e643"
    m.close()


@needs_c1
def test_every_packet_reads_and_verifies():
    m = Manifest(C1)
    n_exp = 0
    for p in m.packets():
        buf, pl = m.read(p)
        assert crc32c_bytes(pl.tobytes()) == p.crc32c
        if p.type == PK_EXPERT:
            dt, off = m.header(buf)
            assert dt == 14 and off[0] == 0 and off[1] % 64 == 0 and off[2] % 64 == 0     # Q6_K, 64-B items
            n_exp += 1
    assert n_exp == 4 * 32
    _, pl = m.read(m.find(PK_DENSE, 0))
    t, data = m.tensor(pl, "attn_q")
    assert (t.dtype, t.ndim, t.shape[0], t.shape[1], t.nbytes) == (8, 2, 512, 512, 512 * 544)
    t, _ = m.tensor(pl, "router")
    assert (t.dtype, t.shape[0], t.shape[1]) == (0, 32, 512)             # the router stays f32
    assert m.tensor(pl, "no_such_tensor") is None
    _, pl = m.read(m.find(PK_META, LAYER_NONE))
    t, _ = m.tensor(pl, "lm_head")
    assert (t.dtype, t.shape[0], t.shape[1]) == (8, 4096, 512)
    m.close()


@needs_c1
def test_reader_agrees_with_the_reference_reader():
    """tlm_manifest_load + tlm_packet_verify of the reference (oracle/_ref)
    see the same records and the same payload bytes."""
    import oracle
    if oracle.ref is None:
        pytest.skip("oracle/_ref not built")
    ref = oracle.ref
    ref.tlm_manifest_find.restype = C.c_void_p
    ref.tlm_manifest_find.argtypes = [C.c_void_p, C.c_int, C.c_uint16, C.c_uint32]
    ref.tlm_manifest_load.argtypes = [C.c_void_p, C.c_char_p]
    ref.tlm_packet_verify.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.POINTER(C.c_void_p),
                                      C.POINTER(C.c_uint64)]
    mbuf = C.create_string_buffer(1 << 16)          # tlm_manifest is far smaller
    assert ref.tlm_manifest_load(mbuf, C1.encode()) == 0
    m = Manifest(C1)
    for p in m.packets()[::7]:
        loc = ref.tlm_manifest_find(mbuf, p.type, p.layer, p.id)
        assert loc
        raw = C.cast(loc, C.POINTER(C.c_uint8 * 48))
        fields = struct.unpack_from("<HHIBBH", bytes(raw.contents))
        assert fields[:3] == (p.type, p.layer, p.id)
        buf, pl = m.read(p)
        payload, plen = C.c_void_p(), C.c_uint64()
        assert ref.tlm_packet_verify(loc, buf.ctypes.data, p.total_len, C.byref(payload), C.byref(plen)) == 0
        assert plen.value == pl.nbytes and payload.value == buf.ctypes.data + 64
    m.close()


@needs_c1
def test_corruption_is_rejected(tmp_path):
    """Header CRC, table SHA-256 and payload CRC each catch one flipped byte."""
    raw = bytearray(open(C1, "rb").read())
    for at, what in ((200, "header checksum"), (len(raw) - 10, "")):
        bad = bytearray(raw)
        if what:
            bad[at] ^= 0x40
        else:                                      # inside the packet table
            n_drives = struct.unpack_from("<I", raw, 16)[0]
            bad[512 + 256 * n_drives + 5] ^= 0x40
        p = tmp_path / "bad.tlmm"
        p.write_bytes(bytes(bad))
        with pytest.raises(HipError) as e:
            Manifest(str(p))
        assert e.value.code == -4
    # a payload byte flipped in a copy of the drive file
    m = Manifest(C1)
    drive = lib.tlm_hip_manifest_drive_path(m.h, 0).decode()
    at = m.find(PK_EXPERT, 1, 3).offset + 64 + 100     # (the record lives in m: read it before close)
    m.close()
    ddir = tmp_path / "d0"
    ddir.mkdir()
    shutil.copy(drive, ddir / os.path.basename(drive))
    data = bytearray(raw)
    n_drives = struct.unpack_from("<I", raw, 16)[0]
    assert n_drives == 1
    path = str(ddir).encode()
    data[512:512 + 256] = path + bytes(256 - len(path))
    hcrc = lib.tlm_hip_crc32c(lib.tlm_hip_crc32c(0, C.c_char_p(bytes(data[:508])), 508),
                              C.c_char_p(bytes(data[512:768])), 256)
    data[508:512] = struct.pack("<I", hcrc)
    (tmp_path / "c1.tlmm").write_bytes(bytes(data))
    with open(ddir / os.path.basename(drive), "r+b") as f:
        f.seek(at)
        b = f.read(1)
        f.seek(at)
        f.write(bytes([b[0] ^ 1]))
    m2 = Manifest(str(tmp_path / "c1.tlmm"))
    with pytest.raises(HipError) as e:
        m2.read(m2.find(PK_EXPERT, 1, 3))
    assert e.value.code == -4
    m2.read(m2.find(PK_EXPERT, 1, 4))               # the others still read
    m2.close()
