"""strixw weight files: the reader (StrixwFile, formats/strixw.hpp:86-112) and the device copy (StrixwDevice,
runtime/strixw_loader.hpp:22-52), over the library's sx_strixw_* entry points.

    dev = StrixwDevice("weights.strixw")                 # validates, then streams the data region into HBM
    gate_up = dev.qw("model.language_model.layers.0.mlp.experts_gate_up", [513 * 2 * 1024, 4096])
    router = dev.bf16("model.language_model.layers.0.mlp.router", [513, 4096])

The file's data region lands in one uint8 device tensor; every tensor keeps its file offset inside it, so the views
are slices of that tensor (4096-byte alignment per tensor, 256 per component, as in the file).
"""
import ctypes
from dataclasses import dataclass, field

import torch

from . import QView, StrixwTensorC, check, lib
from .kernels import QWeight

Q4, Q4_CHUNK_MAJOR, BF16, F32, I64, Q8, Q8_CHUNK_MAJOR, Q6, Q5 = 1, 2, 3, 4, 5, 6, 7, 8, 9
DATA, Q, SCALE, MIN = 0, 1, 2, 3
ENCODING_NAMES = {1: "q4", 2: "q4-chunk-major", 3: "bf16", 4: "f32", 5: "i64", 6: "q8", 7: "q8-chunk-major", 8: "q6",
                  9: "q5"}
_DTYPES = {BF16: torch.bfloat16, F32: torch.float32, I64: torch.int64}


def hash64(buf):
    """strix_hash64 (formats/strixw.hpp:50) of a bytes-like object."""
    b = bytes(buf)
    return int(lib().sx_strix_hash64(ctypes.c_char_p(b) if b else None, len(b)))


@dataclass
class StrixwComponent:
    role: int
    offset: int
    bytes: int
    hash: int


@dataclass
class StrixwTensor:
    name: str
    encoding: int
    shape: list
    group_size: int
    experts: int
    parts: list = field(default_factory=list)  # (source, row_offset, rows)
    components: list = field(default_factory=list)

    def bytes(self):
        return sum(c.bytes for c in self.components)


class StrixwFile:
    """An open, validated file (the library maps it read-only). Raises SxError naming the file and the problem."""

    def __init__(self, path):
        self.path = str(path)
        h = ctypes.c_void_p()
        check(lib().sx_strixw_open(self.path.encode(), ctypes.byref(h)))
        self._h = h
        v, fb, do = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64()
        nt, nm = ctypes.c_int64(), ctypes.c_int64()
        check(lib().sx_strixw_summary(h, ctypes.byref(v), ctypes.byref(fb), ctypes.byref(do), ctypes.byref(nt),
                                       ctypes.byref(nm)))
        self.version, self.file_bytes, self.data_offset = v.value, fb.value, do.value
        self.meta = {}
        for i in range(nm.value):
            k, val = ctypes.c_char_p(), ctypes.c_char_p()
            check(lib().sx_strixw_meta_at(h, i, ctypes.byref(k), ctypes.byref(val)))
            self.meta[k.value.decode()] = val.value.decode()
        self.tensors = [self._tensor(i) for i in range(nt.value)]
        self._by_name = {t.name: t for t in self.tensors}

    def _tensor(self, i):
        t = StrixwTensorC()
        check(lib().sx_strixw_tensor_at(self._h, i, ctypes.byref(t)))
        parts = []
        for p in range(t.nparts):
            src, r0, rows = ctypes.c_char_p(), ctypes.c_int64(), ctypes.c_int64()
            check(lib().sx_strixw_part_at(self._h, i, p, ctypes.byref(src), ctypes.byref(r0), ctypes.byref(rows)))
            parts.append((src.value.decode(), r0.value, rows.value))
        comps = [StrixwComponent(t.comp[c].role, t.comp[c].offset, t.comp[c].bytes, t.comp[c].hash)
                 for c in range(t.ncomp)]
        return StrixwTensor(t.name.decode(), t.encoding, list(t.shape[:t.ndim]), t.group_size, t.experts, parts, comps)

    def close(self):
        if getattr(self, "_h", None):
            lib().sx_strixw_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def meta_value(self, key):
        """StrixwFile::meta(key): raises (naming the file) when absent."""
        v = ctypes.c_char_p()
        check(lib().sx_strixw_meta(self._h, key.encode(), ctypes.byref(v)))
        return v.value.decode()

    def find(self, name):
        return self._by_name.get(name)

    def get(self, name):
        t = self._by_name.get(name)
        if t is None:
            raise KeyError(f"strixw '{self.path}' has no tensor '{name}'")
        return t

    def verify_hashes(self, threads=8):
        check(lib().sx_strixw_verify_hashes(self._h, threads))

    def data_bytes(self):
        return self.file_bytes - self.data_offset


class StrixwDevice:
    """The file's data region resident on `device` (StrixwDevice): one uint8 tensor, filled by read_threads concurrent
    preads through pinned staging and async copies. Accessors check encoding and shape, as the reference's do."""

    def __init__(self, path, read_threads=8, device="cuda", stream=None):
        self.file = StrixwFile(path)
        n = self.file.data_bytes()
        self.data = torch.empty(n, dtype=torch.uint8, device=device)
        secs = ctypes.c_double()
        s = stream.cuda_stream if stream is not None else torch.cuda.current_stream(self.data.device).cuda_stream
        check(lib().sx_strixw_load(self.file._h, self.data.data_ptr(), n, read_threads, ctypes.byref(secs), s))
        self.load_seconds = secs.value

    def data_bytes(self):
        return self.data.numel()

    def _slice(self, offset, nbytes):
        a = offset - self.file.data_offset
        return self.data[a:a + nbytes]

    def tensor(self, name, encoding, shape):
        t = self.file.get(name)
        if t.encoding != encoding or list(t.shape) != list(shape):
            raise ValueError(f"StrixwDevice: '{name}' in '{self.file.path}' is {ENCODING_NAMES.get(t.encoding)} "
                             f"{t.shape}, expected {ENCODING_NAMES.get(encoding)} {list(shape)}")
        return t

    def _qweight(self, name, bits, shape):
        N, K = shape
        v = QView()
        check(lib().sx_strixw_qview(self.file._h, self.data.data_ptr(), name.encode(), bits, N, K, ctypes.byref(v)))
        t = self.file.get(name)
        q, s, m = (self._slice(c.offset, c.bytes) for c in t.components)
        assert (q.data_ptr(), s.data_ptr(), m.data_ptr()) == (v.q, v.scale, v.minv)
        return QWeight(4 if t.encoding == Q4 else 8, q, s.view(torch.int16), m.view(torch.int16), N, K, v.G)

    def q4(self, name, shape):
        return self._qweight(name, 4, shape)

    def q8(self, name, shape):
        return self._qweight(name, 8, shape)

    def qw(self, name, shape):
        """A dense projection stored as q4 or q8 row-major, whichever the file has (the encodings this library's
        kernels take; q5 / q6 / chunk-major raise)."""
        return self._qweight(name, 0, shape)

    def _dense(self, name, encoding, shape):
        arr = (ctypes.c_int64 * max(1, len(shape)))(*shape)
        p = ctypes.c_void_p()
        check(lib().sx_strixw_data(self.file._h, self.data.data_ptr(), name.encode(), encoding, arr, len(shape),
                                    ctypes.byref(p)))
        t = self.file.get(name)
        c = t.components[0]
        out = self._slice(c.offset, c.bytes).view(_DTYPES[encoding]).view(list(shape))
        assert out.data_ptr() == p.value
        return out

    def bf16(self, name, shape):
        return self._dense(name, BF16, shape)

    def f32(self, name, shape):
        return self._dense(name, F32, shape)

    def i64(self, name, shape):
        return self._dense(name, I64, shape)
