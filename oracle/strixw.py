"""The strixw weight-file format, restated for the tests (test infrastructure only, never the product): a writer that
lays out a planned set of tensors as formats/strixw.cpp's StrixwWriter does, a plain parser of what a file holds, and
the file's checksum (oracle.cpp's or_strix_hash64).

Layout (formats/strixw.hpp, formats/strixw.cpp:276-330):
  header, 128 bytes: "STRIXWT\\0" | u32 version | u32 header bytes (128) | u64 index offset (128) | u64 index bytes |
    u64 data offset | u64 file bytes | u64 hash of the index | zeros | u64 hash of header bytes 0..119 at 120;
  index: u32 metadata count, (u16 key length, key, u32 value length, value) in key order; u32 tensor count; per tensor:
    u16 name length, name, u8 encoding, u8 ndim, i64 dims, i64 group size, i64 experts, u16 part count, (u16 source
    length, source, i64 row offset, i64 rows), u8 component count, (u8 role, u64 offset, u64 bytes, u64 hash);
  data: from align_up(128 + index bytes, 4096); each tensor from the next 4096 boundary, each of its components from
    the next 256 boundary, in the order of components().
"""
import ctypes
import struct

import numpy as np

from . import oracle as _orc

MAGIC = b"STRIXWT\0"
HEADER, TENSOR_ALIGN, COMPONENT_ALIGN, VERSION = 128, 4096, 256, 4
Q4, Q4CM, BF16, F32, I64, Q8, Q8CM, Q6, Q5 = 1, 2, 3, 4, 5, 6, 7, 8, 9
DATA, Q, SCALE, MIN = 0, 1, 2, 3


def hash64(buf):
    """strix_hash64 of a bytes-like object (or_strix_hash64)."""
    a = np.frombuffer(bytes(buf), dtype=np.uint8) if not isinstance(buf, np.ndarray) else np.ascontiguousarray(buf)
    L = _orc.lib()
    if not hasattr(L, "_strixw_bound"):
        L.or_strix_hash64.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
        L.or_strix_hash64.restype = ctypes.c_uint64
        L._strixw_bound = True
    return int(L.or_strix_hash64(a.ctypes.data_as(ctypes.c_void_p) if a.size else None, a.nbytes))


def components(enc, shape, G):
    """(role, bytes) of each component, in file order (formats/strixw.cpp:177-251); ValueError if the shape does not
    suit the encoding."""
    n = int(np.prod(shape))
    if enc in (Q4, Q4CM, Q8, Q8CM, Q6, Q5):
        if len(shape) != 2:
            raise ValueError(f"encoding {enc} needs shape [N, K], got {shape}")
        N, K = shape
        need = {Q6: 64, Q5: 128}.get(enc, 1)
        if G not in (32, 64, 128) or K % G or K % need:
            raise ValueError(f"encoding {enc} with K = {K}, group size {G}")
        codes = {Q4: N * K // 2, Q4CM: N * K // 2, Q8: N * K, Q8CM: N * K, Q6: N * (K // 2 + K // 4),
                 Q5: N * (K // 2 + K // 8)}[enc]
        return [(Q, codes), (SCALE, N * (K // G) * 2), (MIN, N * (K // G) * 2)]
    if enc in (BF16, F32, I64):
        if G != 0:
            raise ValueError(f"encoding {enc} has group size {G}, expected 0")
        return [(DATA, n * {BF16: 2, F32: 4, I64: 8}[enc])]
    raise ValueError(f"unknown encoding {enc}")


def _up(v, a):
    return (v + a - 1) // a * a


def _s16(s):
    b = s.encode()
    return struct.pack("<H", len(b)) + b


def encode_index(meta, tensors):
    """The index bytes for `meta` (dict) and `tensors` (dicts with name, enc, shape, G, experts, parts, comps)."""
    out = [struct.pack("<I", len(meta))]
    for k in sorted(meta, key=lambda s: s.encode()):
        v = meta[k].encode()
        out += [_s16(k), struct.pack("<I", len(v)), v]
    out.append(struct.pack("<I", len(tensors)))
    for t in tensors:
        out += [_s16(t["name"]), struct.pack("<BB", t["enc"], len(t["shape"]))]
        out += [struct.pack("<q", d) for d in t["shape"]]
        out += [struct.pack("<qqH", t["G"], t["experts"], len(t["parts"]))]
        for src, r0, rows in t["parts"]:
            out += [_s16(src), struct.pack("<qq", r0, rows)]
        out.append(struct.pack("<B", len(t["comps"])))
        out += [struct.pack("<BQQQ", *c) for c in t["comps"]]
    return b"".join(out)


def header(index, data_offset, file_bytes, version=VERSION):
    h = bytearray(HEADER)
    h[0:8] = MAGIC
    struct.pack_into("<IIQQQQQ", h, 8, version, HEADER, HEADER, len(index), data_offset, file_bytes, hash64(index))
    struct.pack_into("<Q", h, 120, hash64(bytes(h[:120])))
    return bytes(h)


def plan(meta, specs):
    """Lays out the tensors (specs: dicts name, enc, shape, G=0, experts=0, parts=[]): returns (tensors with comps
    [role, offset, bytes, 0], data offset, file bytes), as StrixwWriter's constructor does."""
    tensors = []
    for s in specs:
        t = dict(name=s["name"], enc=s["enc"], shape=list(s["shape"]), G=s.get("G", 0), experts=s.get("experts", 0),
                 parts=list(s.get("parts", [])))
        t["comps"] = [[r, 0, b, 0] for r, b in components(t["enc"], t["shape"], t["G"])]
        tensors.append(t)
    data_offset = _up(HEADER + len(encode_index(meta, tensors)), TENSOR_ALIGN)
    cur = data_offset
    for t in tensors:
        cur = _up(cur, TENSOR_ALIGN)
        for c in t["comps"]:
            cur = _up(cur, COMPONENT_ALIGN)
            c[1] = cur
            cur += c[2]
    return tensors, data_offset, cur


def write(path, meta, specs, payloads):
    """Writes a file: payloads[i] is the list of component byte strings of specs[i], in components() order. Returns
    the planned tensors (offsets and hashes filled in)."""
    tensors, data_offset, size = plan(meta, specs)
    buf = bytearray(size)
    for t, parts in zip(tensors, payloads):
        assert len(parts) == len(t["comps"]), t["name"]
        for c, p in zip(t["comps"], parts):
            p = bytes(p)
            assert len(p) == c[2], (t["name"], c[0], len(p), c[2])
            buf[c[1]:c[1] + c[2]] = p
            c[3] = hash64(p)
    index = encode_index(meta, tensors)
    buf[HEADER:HEADER + len(index)] = index
    buf[0:HEADER] = header(index, data_offset, size)
    with open(path, "wb") as f:
        f.write(buf)
    return tensors


def parse(blob):
    """What a file holds, read without validation: dict(version, file_bytes, data_offset, index_bytes, meta,
    tensors) with tensors as in plan()."""
    version, hsize, ioff, ibytes, doff, fbytes = struct.unpack_from("<IIQQQQ", blob, 8)
    at = ioff

    def take(fmt):
        nonlocal at
        v = struct.unpack_from("<" + fmt, blob, at)
        at += struct.calcsize("<" + fmt)
        return v if len(v) > 1 else v[0]

    def text(n):
        nonlocal at
        s = bytes(blob[at:at + n]).decode()
        at += n
        return s

    meta = {}
    for _ in range(take("I")):
        k = text(take("H"))
        meta[k] = text(take("I"))
    tensors = []
    for _ in range(take("I")):
        name = text(take("H"))
        enc, nd = take("BB")
        shape = [take("q") for _ in range(nd)]
        G, experts, nparts = take("qqH")
        parts = []
        for _ in range(nparts):
            src = text(take("H"))
            parts.append((src, *take("qq")))
        comps = [list(take("BQQQ")) for _ in range(take("B"))]
        tensors.append(dict(name=name, enc=enc, shape=shape, G=G, experts=experts, parts=parts, comps=comps))
    return dict(version=version, file_bytes=fbytes, data_offset=doff, index_bytes=ibytes, meta=meta, tensors=tensors)


def listing(info):
    """The tab-separated listing ref_strixw_read produces, from parse() or an equivalent dict."""
    lines = [f"H\t{info['version']}\t{info['file_bytes']}\t{info['data_offset']}"]
    lines += [f"M\t{k}\t{v}" for k, v in sorted(info["meta"].items(), key=lambda kv: kv[0].encode())]
    for t in info["tensors"]:
        f = ["T", t["name"], t["enc"], t["G"], t["experts"], len(t["shape"]), *t["shape"], len(t["parts"])]
        for p in t["parts"]:
            f += list(p)
        f.append(len(t["comps"]))
        for c in t["comps"]:
            f += list(c)
        lines.append("\t".join(str(x) for x in f))
    return "\n".join(lines) + "\n"


# ---- the compiled reference (oracle/_ref), when built ----

def _ref():
    L = _orc.ref()
    if not hasattr(L, "_strixw_bound"):
        L.ref_strix_hash64.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
        L.ref_strix_hash64.restype = ctypes.c_uint64
        L.ref_strixw_write.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_uint64,
                                       ctypes.c_char_p, ctypes.c_int64]
        L.ref_strixw_write.restype = ctypes.c_int
        L.ref_strixw_read.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_char_p, ctypes.c_int64, ctypes.c_char_p,
                                      ctypes.c_int64]
        L.ref_strixw_read.restype = ctypes.c_int
        L._strixw_bound = True
    return L


def ref_hash64(buf):
    a = np.frombuffer(bytes(buf), dtype=np.uint8)
    return int(_ref().ref_strix_hash64(a.ctypes.data_as(ctypes.c_void_p) if a.size else None, a.nbytes))


def ref_write(path, meta, specs, payloads):
    """The reference's StrixwWriter on the same plan and payloads; raises RuntimeError with its message if it threw."""
    lines = [f"M\t{k}\t{v}" for k, v in meta.items()]
    for s in specs:
        f = ["T", s["name"], s["enc"], s.get("G", 0), s.get("experts", 0), len(s["shape"]), *s["shape"],
             len(s.get("parts", []))]
        for p in s.get("parts", []):
            f += list(p)
        lines.append("\t".join(str(x) for x in f))
    data = b"".join(bytes(p) for parts in payloads for p in parts)
    msg = ctypes.create_string_buffer(4096)
    rc = _ref().ref_strixw_write(str(path).encode(), "\n".join(lines).encode(), data, len(data), msg, 4096)
    if rc:
        raise RuntimeError(msg.value.decode())


def ref_read(path, threads=0):
    """The reference's StrixwFile (and verify_hashes when threads > 0): (listing, None) or (None, its message)."""
    dump, msg = ctypes.create_string_buffer(1 << 20), ctypes.create_string_buffer(4096)
    rc = _ref().ref_strixw_read(str(path).encode(), threads, dump, 1 << 20, msg, 4096)
    return (None, msg.value.decode()) if rc else (dump.value.decode(), None)


def sample_plan(seed=0, E=4, d=256, I=64, V=300):
    """A small file of every encoding, laid out like a one-layer qwen4exp conversion (router BF16 [E + 1, d], stacked
    q4 experts gate_up [(E + 1) * 2I, d] and down [(E + 1) * d, I], a q8 LM head [V, d]) plus q6 / q5 / chunk-major /
    f32 / i64 records: (meta, specs, payloads), payloads seeded random bytes (BF16 scales and mins of small finite
    values)."""
    rng = np.random.default_rng(seed)
    L = "model.language_model."
    Ew = E + 1
    specs = [
        dict(name=L + "layers.0.mlp.router", enc=BF16, shape=[Ew, d], parts=[(L + "layers.0.mlp.gate.weight", 0, E),
                                                                              (L + "layers.0.mlp.shared_expert_gate.weight", E, 1)]),
        dict(name=L + "layers.0.mlp.experts_gate_up", enc=Q4, shape=[Ew * 2 * I, d], G=128, experts=Ew),
        dict(name=L + "layers.0.mlp.experts_down", enc=Q4, shape=[Ew * d, I], G=64, experts=Ew),
        dict(name="lm_head.weight", enc=Q8, shape=[V, d], G=64, parts=[("lm_head.weight", 0, V)]),
        dict(name=L + "norm.weight", enc=F32, shape=[d]),
        dict(name="positions", enc=I64, shape=[3, 5]),
        dict(name="q6.weight", enc=Q6, shape=[4, 128], G=64),
        dict(name="q5.weight", enc=Q5, shape=[2, 256], G=128),
        dict(name="mix_up", enc=Q4CM, shape=[8, 128], G=32),
        dict(name="mix_up8", enc=Q8CM, shape=[4, 64], G=64),
    ]
    meta = {"arch": "qwen4exp", "globals": "yes", "layers": "0", "shared_expert": "stacked", "source_fingerprint": "x1"}
    payloads = []
    for s in specs:
        parts = []
        for role, nbytes in components(s["enc"], s["shape"], s.get("G", 0)):
            if role in (SCALE, MIN) or s["enc"] == BF16:
                v = (rng.standard_normal(nbytes // 2) * (0.01 if role == SCALE else 0.1)).astype(np.float32)
                if role == SCALE:
                    v = np.abs(v) + 1e-3
                parts.append(((v.view(np.uint32) + 0x8000) >> 16).astype(np.uint16).tobytes())
            elif s["enc"] == F32:
                parts.append(rng.standard_normal(nbytes // 4).astype(np.float32).tobytes())
            else:
                parts.append(rng.integers(0, 256, nbytes, dtype=np.uint8).tobytes())
        payloads.append(parts)
    return meta, specs, payloads
