"""strixw files without a GPU: the library's reader (sx_strixw_open and friends, host code) against the oracle's
restatement of the format (oracle/strixw.py), the committed fixtures written by the reference's own StrixwWriter, and -
where oracle/_ref is built - the reference's StrixwFile itself.

Pins:
  - strix_hash64: the oracle's word-by-word restatement and the library's hash against strixw_hash.npz (the
    reference's values for every length 0..300 and a few long buffers: every block / leftover-word / tail split);
  - the writer restatement: byte-identical to strixw_small.strixw, which the reference wrote from the same plan, and
    to a live reference write of a second plan;
  - the reader: the same listing (header fields, metadata, every record) as the oracle's plain parse and the
    reference's StrixwFile, and the same accept / reject decision on crafted corruptions and valid variants (each
    rejection's message is this reader's own and is checked for naming the fault).
"""
import ctypes
import os
import struct

import numpy as np
import pytest

from oracle import oracle as orc
from oracle import strixw as ow

HERE = os.path.dirname(os.path.abspath(__file__))
SMALL = os.path.join(HERE, "golden", "strixw_small.strixw")
ref_only = pytest.mark.skipif(not orc.ref_available(), reason="oracle/_ref not built (no reference tree)")


def sw():
    from strixite_amd import strixw
    return strixw


def product_listing(f):
    """The listing ref_strixw_read prints, built from the library's reader."""
    info = dict(version=f.version, file_bytes=f.file_bytes, data_offset=f.data_offset, meta=f.meta,
                tensors=[dict(name=t.name, enc=t.encoding, shape=t.shape, G=t.group_size, experts=t.experts,
                              parts=t.parts, comps=[[c.role, c.offset, c.bytes, c.hash] for c in t.components])
                         for t in f.tensors])
    return ow.listing(info)


def open_error(path):
    """The library's rejection message with its 'sx_strixw_open: ' prefix dropped, or None if it opened."""
    import strixite_amd as sx
    try:
        sw().StrixwFile(path).close()
        return None
    except sx.SxError as e:
        assert e.code == sx.SX_EINVAL
        msg = str(e)
        assert msg.startswith("sx_strixw_open: "), msg
        return msg[len("sx_strixw_open: "):]


# ---------------- the checksum ----------------

def test_hash_matches_reference_vectors():
    g = np.load(os.path.join(HERE, "golden", "strixw_hash.npz"))
    at = 0
    for n, h in zip(g["lens"], g["hash"]):
        buf = g["data"][at:at + n].tobytes()
        at += n
        assert ow.hash64(buf) == int(h), f"oracle hash, {n} bytes"
        assert sw().hash64(buf) == int(h), f"library hash, {n} bytes"


def test_hash_distinguishes_what_a_slip_would_merge():
    """Length is mixed in (zero buffers of different lengths differ), lanes are not interchangeable (swapping two
    8-byte words changes the hash), and the tail's count tag matters (a trailing zero byte changes it)."""
    hs = {ow.hash64(bytes(n)) for n in range(80)}
    assert len(hs) == 80
    b = np.random.default_rng(3).integers(0, 256, 64, dtype=np.uint8).tobytes()
    swapped = b[8:16] + b[0:8] + b[16:]
    assert ow.hash64(b) != ow.hash64(swapped)
    assert ow.hash64(b[:61]) != ow.hash64(b[:61] + b"\0")


@ref_only
def test_hash_matches_live_reference():
    rng = np.random.default_rng(11)
    for n in list(range(0, 130)) + [1 << 20, (1 << 20) + 5]:
        b = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert ow.hash64(b) == ow.ref_hash64(b) == sw().hash64(b), n


# ---------------- the writer restatement ----------------

def test_oracle_writer_matches_reference_fixture(tmp_path):
    meta, specs, payloads = ow.sample_plan(seed=7)
    p = tmp_path / "o.strixw"
    ow.write(p, meta, specs, payloads)
    assert p.read_bytes() == open(SMALL, "rb").read()


@ref_only
def test_oracle_writer_matches_live_reference(tmp_path):
    meta, specs, payloads = ow.sample_plan(seed=21, E=2, d=128, I=128, V=70)
    meta = dict(meta, zeta="last", Alpha="upper first", empty="")
    ow.write(tmp_path / "o.strixw", meta, specs, payloads)
    ow.ref_write(tmp_path / "r.strixw", meta, specs, payloads)
    assert (tmp_path / "o.strixw").read_bytes() == (tmp_path / "r.strixw").read_bytes()


# ---------------- the reader ----------------

def test_reader_lists_the_fixture():
    f = sw().StrixwFile(SMALL)
    blob = open(SMALL, "rb").read()
    assert product_listing(f) == ow.listing(ow.parse(blob))
    assert f.version == 4 and f.file_bytes == len(blob) and f.data_offset % 4096 == 0
    assert f.meta_value("arch") == "qwen4exp"
    router = f.get("model.language_model.layers.0.mlp.router")
    assert router.parts == [("model.language_model.layers.0.mlp.gate.weight", 0, 4),
                            ("model.language_model.layers.0.mlp.shared_expert_gate.weight", 4, 1)]
    for t in f.tensors:
        for c in t.components:
            assert c.offset % 256 == 0 and sw().hash64(blob[c.offset:c.offset + c.bytes]) == c.hash
        assert t.components[0].offset % 4096 == 0
    f.verify_hashes(4)
    import strixite_amd as sx
    with pytest.raises(sx.SxError, match="has no metadata 'nope'"):
        f.meta_value("nope")
    assert f.find("nope") is None


@ref_only
def test_reader_listing_matches_reference():
    listing, err = ow.ref_read(SMALL, threads=2)
    assert err is None
    assert product_listing(sw().StrixwFile(SMALL)) == listing


def test_views_on_the_mapping_point_at_the_components():
    """sx_strixw_qview / sx_strixw_data with no device base: pointers into the file's mapping, checked."""
    import strixite_amd as sx
    L = sx.lib()
    f = sw().StrixwFile(SMALL)
    blob = open(SMALL, "rb").read()
    name = "lm_head.weight"
    t = f.get(name)
    v = sx.QView()
    assert L.sx_strixw_qview(f._h, None, name.encode(), 8, 300, 256, ctypes.byref(v)) == 0
    assert v.G == 64 and (v.N, v.K) == (300, 256)
    for ptr, c in zip((v.q, v.scale, v.minv), t.components):
        assert ctypes.string_at(ptr, c.bytes) == blob[c.offset:c.offset + c.bytes]
    assert L.sx_strixw_qview(f._h, None, name.encode(), 4, 300, 256, ctypes.byref(v)) == sx.SX_EINVAL
    assert b"'lm_head.weight' in" in L.sx_last_error() and b"is q8 [300, 256], expected q4 [300, 256]" in L.sx_last_error()
    assert L.sx_strixw_qview(f._h, None, name.encode(), 0, 300, 128, ctypes.byref(v)) == sx.SX_EINVAL
    assert L.sx_strixw_qview(f._h, None, b"q6.weight", 0, 4, 128, ctypes.byref(v)) == sx.SX_EINVAL  # q6: no kernel here
    norm = "model.language_model.norm.weight"
    shape = (ctypes.c_int64 * 1)(256)
    p = ctypes.c_void_p()
    assert L.sx_strixw_data(f._h, None, norm.encode(), 4, shape, 1, ctypes.byref(p)) == 0
    c = f.get(norm).components[0]
    assert ctypes.string_at(p.value, 1024) == blob[c.offset:c.offset + 1024]
    assert L.sx_strixw_data(f._h, None, norm.encode(), 3, shape, 1, ctypes.byref(p)) == sx.SX_EINVAL
    assert L.sx_strixw_data(f._h, None, b"absent", 4, shape, 1, ctypes.byref(p)) == sx.SX_EINVAL
    assert b"has no tensor 'absent'" in L.sx_last_error()


# ---------------- rejections ----------------

def _rehash(blob, index_bytes=None):
    """Recomputes the index hash (over index_bytes, default the header's) and then the header hash."""
    b = bytearray(blob)
    ib = struct.unpack_from("<Q", b, 24)[0] if index_bytes is None else index_bytes
    struct.pack_into("<Q", b, 24, ib)
    struct.pack_into("<Q", b, 48, ow.hash64(bytes(b[128:128 + ib])))
    struct.pack_into("<Q", b, 120, ow.hash64(bytes(b[:120])))
    return bytes(b)


def _with_index(blob, mutate):
    """Re-encodes the index after mutate(info) (same data region and offsets), fixing both hashes."""
    info = ow.parse(blob)
    mutate(info)
    idx = ow.encode_index(info["meta"], info["tensors"])
    doff = info["data_offset"]
    assert 128 + len(idx) <= doff
    b = bytearray(blob)
    b[128:doff] = idx + bytes(doff - 128 - len(idx))
    return _rehash(bytes(b), len(idx))


def _corruptions(blob):
    """name -> (file bytes, the message fragment the reference's StrixwFile raises)."""
    first = ow.parse(blob)["tensors"][0]["comps"][0][1]
    cases = {}
    b = bytearray(blob)
    b[0] = ord("X")
    cases["magic"] = (bytes(b), "no STRIXWT signature at byte 0")
    b = bytearray(blob)
    struct.pack_into("<I", b, 8, 5)
    cases["version"] = (_rehash(bytes(b)), "written as version 5")
    b = bytearray(blob)
    struct.pack_into("<I", b, 12, 256)
    cases["header size"] = (_rehash(bytes(b)), "declares a 256-byte header, not 128")
    b = bytearray(blob)
    b[100] ^= 1
    cases["header hash"] = (bytes(b), "checksum of header bytes 0..119 does not match")
    cases["truncated"] = (blob[:-1], "differs from the recorded")
    cases["appended"] = (blob + b"\0", "differs from the recorded")
    cases["short"] = (blob[:100], "too short for the 128-byte header")
    b = bytearray(blob)
    b[140] ^= 0x40
    cases["index hash"] = (bytes(b), "checksum of the index does not match")
    b = bytearray(blob)
    struct.pack_into("<Q", b, 32, 4096 + 8)
    cases["data offset"] = (_rehash(bytes(b)), "data region start 4104")
    b = bytearray(blob)
    struct.pack_into("<Q", b, 16, 64)
    cases["index offset"] = (_rehash(bytes(b)), "index [64, +")

    def dup_name(i):
        i["tensors"][1]["name"] = i["tensors"][0]["name"]
    cases["tensor twice"] = (_with_index(blob, dup_name), "is listed more than once")

    def overlap(i):
        i["tensors"][1]["comps"][0][1] = i["tensors"][0]["comps"][0][1]
    cases["overlap"] = (_with_index(blob, overlap), "two components share bytes from")

    def unaligned(i):
        i["tensors"][0]["comps"][0][1] += 16
    cases["unaligned"] = (_with_index(blob, unaligned), "-byte boundary")

    def outside(i):
        i["tensors"][-1]["comps"][0][1] = len(blob) // 256 * 256
    cases["outside"] = (_with_index(blob, outside), "fall outside the data region")

    def before(i):
        i["tensors"][0]["comps"][0][1] = 256
    cases["before data"] = (_with_index(blob, before), "fall outside the data region")

    def wrong_bytes(i):
        i["tensors"][3]["comps"][1][2] += 2
    cases["component size"] = (_with_index(blob, wrong_bytes), "listed component 1 (scale, ")

    def wrong_role(i):
        i["tensors"][3]["comps"][1][0] = 3
    cases["component role"] = (_with_index(blob, wrong_role), "listed component 1 (min, ")

    def drop_comp(i):
        i["tensors"][3]["comps"].pop()
    cases["component count"] = (_with_index(blob, drop_comp), "stores 3 components, the index lists 2")

    def bad_group(i):
        i["tensors"][3]["G"] = 48
    cases["group"] = (_with_index(blob, bad_group), "group size 48")

    def bad_enc(i):
        i["tensors"][4]["enc"] = 12
    cases["encoding"] = (_with_index(blob, bad_enc), "encoding code 12 is not one")

    def bad_experts(i):
        i["tensors"][1]["experts"] = 7
    cases["experts"] = (_with_index(blob, bad_experts), "7 experts cannot share")

    def gap_parts(i):
        i["tensors"][0]["parts"][1] = (i["tensors"][0]["parts"][1][0], 5, 1)
    cases["parts gap"] = (_with_index(blob, gap_parts), "where row 4 comes next")

    def short_parts(i):
        i["tensors"][0]["parts"].pop()
    cases["parts cover"] = (_with_index(blob, short_parts), "its parts end at row 4 of 5")

    def zero_dim(i):
        i["tensors"][5]["shape"] = [3, 0]
    cases["zero dim"] = (_with_index(blob, zero_dim), "shape is [3, 0]")

    def empty_name(i):
        i["tensors"][2]["name"] = ""
    cases["empty name"] = (_with_index(blob, empty_name), "an unnamed tensor")

    def f32_group(i):
        i["tensors"][4]["G"] = 64
    cases["dense group"] = (_with_index(blob, f32_group), "take no group size (found 64)")

    def no_tensors(i):
        i["tensors"] = []
    cases["no tensors"] = (_with_index(blob, no_tensors), "lists no tensors")

    # an index one byte longer than its records (the hash covers the extra byte)
    ib = struct.unpack_from("<Q", blob, 24)[0]
    cases["unread bytes"] = (_rehash(blob, ib + 1), "1 bytes past its last tensor record")
    # an index cut inside its last record
    cases["index ends"] = (_rehash(blob, ib - 5), "stops short of the component checksum")
    del first
    return cases


def test_reader_rejects_corruptions(tmp_path):
    blob = open(SMALL, "rb").read()
    for name, (data, fragment) in _corruptions(blob).items():
        p = tmp_path / (name.replace(" ", "_") + ".strixw")
        p.write_bytes(data)
        msg = open_error(p)
        assert msg is not None, f"{name}: accepted"
        assert msg.startswith(f"strixw '{p}': "), (name, msg)
        assert fragment in msg, (name, msg)
    assert open_error(tmp_path / "missing.strixw").endswith("open failed: No such file or directory")


def _valid_variants(blob):
    """name -> file bytes: rewrites of the fixture that the format allows, which a reader must accept."""
    def no_meta(i):
        i["meta"] = {}

    def one_part(i):
        t = i["tensors"][0]
        t["parts"] = [("whole", 0, t["shape"][0])]

    def no_parts(i):
        i["tensors"][0]["parts"] = []

    def no_experts(i):
        i["tensors"][1]["experts"] = 0

    def one_expert(i):
        i["tensors"][2]["experts"] = 1

    def odd_meta(i):
        i["meta"] = dict(i["meta"], **{"": "empty key", "z" * 300: "v" * 500})

    cases = {name: _with_index(blob, fn) for name, fn in
             [("no metadata", no_meta), ("one part", one_part), ("no parts", no_parts), ("no experts", no_experts),
              ("one expert", one_expert), ("odd metadata", odd_meta)]}
    b = bytearray(blob)
    struct.pack_into("<I", b, 8, 1)
    cases["version 1"] = _rehash(bytes(b))
    return cases


def test_reader_accepts_valid_variants(tmp_path):
    blob = open(SMALL, "rb").read()
    for name, data in _valid_variants(blob).items():
        p = tmp_path / (name.replace(" ", "_") + ".strixw")
        p.write_bytes(data)
        assert open_error(p) is None, name
        assert product_listing(sw().StrixwFile(p)) == ow.listing(ow.parse(data)), name


@ref_only
def test_reader_decisions_match_reference(tmp_path):
    """The reference's StrixwFile and this reader take the same accept / reject decision on every corrupted and every
    valid variant (the messages are this reader's own), and list accepted files the same way."""
    blob = open(SMALL, "rb").read()
    for name, (data, _) in _corruptions(blob).items():
        p = tmp_path / (name.replace(" ", "_") + ".strixw")
        p.write_bytes(data)
        _, ref_msg = ow.ref_read(p)
        assert ref_msg is not None, f"{name}: the reference accepted it"
        assert open_error(p) is not None, f"{name}: accepted here"
    for name, data in _valid_variants(blob).items():
        p = tmp_path / ("ok_" + name.replace(" ", "_") + ".strixw")
        p.write_bytes(data)
        listing, ref_msg = ow.ref_read(p)
        assert ref_msg is None, f"{name}: the reference rejected it: {ref_msg}"
        assert open_error(p) is None, name
        assert product_listing(sw().StrixwFile(p)) == listing, name


def _past_the_end(blob):
    """The last component moved to the first 256-byte boundary after the end of the file."""
    def past(i):
        i["tensors"][-1]["comps"][-1][1] = (len(blob) + 255) // 256 * 256
    return _with_index(blob, past)


def test_reader_rejects_a_component_past_the_end(tmp_path):
    """A component that starts beyond the end of the file is refused. The reference's StrixwFile accepts this file:
    its bound check computes file size - offset in unsigned arithmetic (formats/strixw.cpp, the component check of
    the StrixwFile constructor), which wraps for such an offset; a later read of the component would leave the
    mapping. This reader checks the offset first."""
    blob = open(SMALL, "rb").read()
    p = tmp_path / "past.strixw"
    p.write_bytes(_past_the_end(blob))
    msg = open_error(p)
    assert msg is not None and "fall outside the data region" in msg, msg
    if orc.ref_available():
        _, ref_msg = ow.ref_read(p)
        assert ref_msg is None  # the divergence stated above


def test_verify_hashes_names_the_first_corrupt_component(tmp_path):
    import strixite_amd as sx
    blob = bytearray(open(SMALL, "rb").read())
    info = ow.parse(bytes(blob))
    t2, t5 = info["tensors"][2], info["tensors"][5]
    blob[t5["comps"][0][1] + 3] ^= 1
    blob[t2["comps"][2][1]] ^= 0x80  # the min component of tensor 2: first in file order
    p = tmp_path / "c.strixw"
    p.write_bytes(bytes(blob))
    f = sw().StrixwFile(p)  # opens: component hashes are not checked at open
    with pytest.raises(sx.SxError, match=f"hash mismatch in tensor '{t2['name']}' min"):
        f.verify_hashes(3)
    if orc.ref_available():
        _, msg = ow.ref_read(p, threads=1)
        assert msg is not None and "hash mismatch in tensor" in msg
