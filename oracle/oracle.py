"""ctypes bindings of the CPU oracle (oracle.cpp) and, when built, of the compiled reference (_ref/libstrix_ref.so).

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker.
The product library (strixite_amd) never imports this module.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(_HERE, "liboracle.so")
REF_SO = os.path.join(_HERE, "_ref", "libstrix_ref.so")

F32, BF16 = 0, 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_INT = ctypes.c_int
_D = ctypes.c_double


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_P)


def build():
    """Compiles liboracle.so (and _ref/ when the reference tree is present) with oracle/Makefile."""
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"oracle library {ORACLE_SO} is not built (run `make -C oracle`)")
        L = ctypes.CDLL(ORACLE_SO)
        L.or_dequant.argtypes = [_INT, _P, _P, _P, _I64, _I64, _I64, _P]
        L.or_linear_q.argtypes = [_INT, _P, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _INT, _INT, _INT]
        L.or_linear_f32w.argtypes = [_P, _P, _I64, _I64, _P, _I64, _INT, _INT]
        L.or_quantize_q4.argtypes = [_P, _I64, _I64, _I64, _P, _P, _P]
        L.or_quantize_q4.restype = _INT
        L.or_q4_from_q8.argtypes = [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _INT]
        L.or_q4_from_q8.restype = _INT
        L.or_linear_bf16w.argtypes = [_P, _P, _I64, _I64, _P, _I64, _INT, _INT, _INT]
        L.or_moe_shared_add.argtypes = [_P, _P, _P, _I64, _I64, _I64, ctypes.c_uint32, _P, _P, _I64, _INT, _P]
        L.or_moe_router.argtypes = [_P, _I64, _I64, _I64, _I64, _P, _I64, _I32, _P, _P, _P]
        L.or_moe_router.restype = _INT
        for f in (L.or_experts_gather, L.or_experts_gather_swiglu):
            f.argtypes = [_INT, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P, _INT, _P, _INT]
        L.or_experts_combine.argtypes = [_INT, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _P, _INT,
                                         _P, _INT]
        L.or_swiglu.argtypes = [_P, _P, _I64, _I64, _INT]
        L.or_logits_topk.argtypes = [_P, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _P]
        L.or_top2.argtypes = [_P, _I64, _P, _P, _P, _P]
        L.or_rng_new.argtypes = [ctypes.c_uint64]
        L.or_rng_new.restype = _P
        L.or_rng_free.argtypes = [_P]
        L.or_rng_canonical.argtypes = [_P]
        L.or_rng_canonical.restype = _D
        L.or_sample_row.argtypes = [_P, _P, _I64, _D, _I64, _D]
        L.or_sample_row.restype = _I32
        L.or_accept.argtypes = [_P, _P, _I64, _I64, _I64, _P, _D, _I64, _D, _P, _P]
        L.or_accept.restype = _I64
        _lib = L
    return _lib


def _act_of(a):
    return F32 if a.dtype == np.float32 else BF16


def _new_like(act, shape):
    return np.empty(shape, np.float32 if act == F32 else np.uint16)


class QWeight:
    """Host copy of a q4 / q8 weight in the reference layout (formats/q4.hpp:3-6, q8.hpp:3-11)."""

    def __init__(self, bits, q, scale, minv, N, K, G):
        self.bits, self.q, self.scale, self.minv = bits, np.ascontiguousarray(q), np.ascontiguousarray(scale), \
            np.ascontiguousarray(minv)
        self.N, self.K, self.G = int(N), int(K), int(G)
        groups = self.N * (self.K // self.G)
        need = self.N * self.K // (2 if bits == 4 else 1)
        if self.q.size != need or self.scale.size != groups or self.minv.size != groups:
            raise ValueError(f"q{bits} weight [{N}, {K}] G{G}: {self.q.size} code bytes (need {need}), "
                             f"{self.scale.size}/{self.minv.size} scales/mins (need {groups})")

    def args(self):
        return (_ptr(self.q), _ptr(self.scale), _ptr(self.minv))


def dequant(w):
    out = np.empty((w.N, w.K), np.float32)
    lib().or_dequant(w.bits, *w.args(), w.N, w.K, w.G, _ptr(out))
    return out


def linear_q(x, w, out_act=None, threads=0):
    """x [M, K] float32 (act F32) or uint16 bf16 bits (act BF16) -> y [M, N] in out_act."""
    act = _act_of(x)
    out_act = act if out_act is None else out_act
    M = x.shape[0]
    y = _new_like(out_act, (M, w.N))
    lib().or_linear_q(w.bits, _ptr(np.ascontiguousarray(x)), *w.args(), w.N, w.K, w.G, _ptr(y), M, act, out_act,
                      threads)
    return y


def linear_f32w(x, W, threads=0):
    act = _act_of(x)
    M, (N, K) = x.shape[0], W.shape
    y = np.empty((M, N), np.float32)
    lib().or_linear_f32w(_ptr(np.ascontiguousarray(x)), _ptr(np.ascontiguousarray(W, np.float32)), N, K, _ptr(y), M,
                         act, threads)
    return y


def quantize_q4(w, G):
    """formats/q4.cpp quantize_q4 restated: FP32 [N, K] -> QWeight (q4)."""
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    q = np.empty(N * K // 2, np.uint8)
    s = np.empty(N * (K // G), np.uint16)
    m = np.empty(N * (K // G), np.uint16)
    if lib().or_quantize_q4(_ptr(w), N, K, G, _ptr(q), _ptr(s), _ptr(m)):
        raise ValueError("quantize_q4: non-finite weight")
    return QWeight(4, q, s, m, N, K, G)


def q4_from_q8(w8, G4, threads=0):
    """formats/q4_from_q8.cpp restated: a q8 QWeight -> the q4 QWeight of its exactly dequantized rows."""
    N, K = w8.N, w8.K
    q = np.empty(N * K // 2, np.uint8)
    s = np.empty(N * (K // G4), np.uint16)
    m = np.empty(N * (K // G4), np.uint16)
    if lib().or_q4_from_q8(*w8.args(), N, K, w8.G, G4, _ptr(q), _ptr(s), _ptr(m), threads):
        raise ValueError("q4_from_q8: non-finite dequantized weight")
    return QWeight(4, q, s, m, N, K, G4)


def linear_bf16w(x, W, out_act=None, threads=0):
    """x [M, K] float32 or BF16 bits, W [N, K] BF16 bits (uint16) -> y [M, N] in out_act (default: x's dtype)."""
    act = _act_of(x)
    out_act = act if out_act is None else out_act
    M, (N, K) = x.shape[0], W.shape
    y = _new_like(out_act, (M, N))
    lib().or_linear_bf16w(_ptr(np.ascontiguousarray(x)), _ptr(np.ascontiguousarray(W, np.uint16)), N, K, _ptr(y), M,
                          act, out_act, threads)
    return y


def moe_shared_add(y, s, gate_logit, gate_ld, gate_index, x=None, w_in=None):
    """moe_shared_add (x None) or moe_shared_add_inject on host arrays: returns (y', x' or None, err). y, s [M, N] and
    x [M, H * N] float32 or BF16 bits; gate_logit float32 with row stride gate_ld; w_in float32 [M, H]."""
    act = _act_of(y)
    M, N = y.shape
    y = np.array(y, copy=True)
    x = None if x is None else np.array(x, copy=True)
    H = 0 if x is None else x.shape[1] // N
    err = np.zeros(3, np.uint32)
    lib().or_moe_shared_add(_ptr(y), _ptr(np.ascontiguousarray(s)), _ptr(np.ascontiguousarray(gate_logit, np.float32)),
                            gate_ld, M, N, gate_index, _ptr(x),
                            None if w_in is None else _ptr(np.ascontiguousarray(w_in, np.float32)), H, act, _ptr(err))
    return y, x, err


def moe_router(logits, E, k, shared=None, shared_ld=1, shared_id=0):
    logits = np.ascontiguousarray(logits, np.float32)
    M, ld = logits.shape
    A = k + (1 if shared is not None else 0)
    ids = np.empty((M, A), np.int32)
    coef = np.empty((M, A), np.float32)
    err = np.zeros(3, np.uint32)
    lib().or_moe_router(_ptr(logits), ld, M, E, k, _ptr(shared), shared_ld, shared_id, _ptr(ids), _ptr(coef),
                        _ptr(err))
    return ids, coef, err


def experts_gather(x, w, E, ids, swiglu=False, threads=0):
    act = _act_of(x)
    M, A = ids.shape
    N = w.N // E
    y = _new_like(act, (M, A, N // 2 if swiglu else N))
    err = np.zeros(3, np.uint32)
    f = lib().or_experts_gather_swiglu if swiglu else lib().or_experts_gather
    f(w.bits, _ptr(np.ascontiguousarray(x)), *w.args(), w.N, w.K, w.G, E, _ptr(np.ascontiguousarray(ids, np.int32)),
      M, A, _ptr(y), act, _ptr(err), threads)
    return y, err


def experts_combine(h, w, E, ids, coef, threads=0):
    act = _act_of(h)
    M, A = ids.shape
    N = w.N // E
    y = _new_like(act, (M, N))
    err = np.zeros(3, np.uint32)
    lib().or_experts_combine(w.bits, _ptr(np.ascontiguousarray(h)), *w.args(), w.N, w.K, w.G, E,
                             _ptr(np.ascontiguousarray(ids, np.int32)), _ptr(np.ascontiguousarray(coef, np.float32)),
                             M, A, _ptr(y), act, _ptr(err), threads)
    return y, err


def swiglu(gu):
    act = _act_of(gu)
    rows, I2 = gu.shape
    h = _new_like(act, (rows, I2 // 2))
    lib().or_swiglu(_ptr(np.ascontiguousarray(gu)), _ptr(h), rows, I2 // 2, act)
    return h


def logits_topk(logits, n_valid, k, mask=None):
    logits = np.ascontiguousarray(logits, np.float32)
    rows, ld = logits.shape
    v = np.empty((rows, k), np.float32)
    i = np.empty((rows, k), np.int32)
    nan = np.empty(rows, np.uint32)
    mw = 0 if mask is None else mask.shape[1]
    lib().or_logits_topk(_ptr(logits), rows, ld, n_valid, k, _ptr(mask), mw, _ptr(v), _ptr(i), _ptr(nan))
    return v, i, nan


def top2(x):
    x = np.ascontiguousarray(x, np.float32)
    b, bv, sv, nan = ctypes.c_int32(), ctypes.c_float(), ctypes.c_float(), ctypes.c_uint32()
    lib().or_top2(_ptr(x), x.size, ctypes.byref(b), ctypes.byref(bv), ctypes.byref(sv), ctypes.byref(nan))
    return b.value, bv.value, sv.value, nan.value


class Rng:
    """std::mt19937_64(seed), the generator serve/sampler.hpp:80 keeps."""

    def __init__(self, seed):
        self.h = lib().or_rng_new(seed)

    def canonical(self):
        return lib().or_rng_canonical(self.h)

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_rng_free(self.h)
            self.h = None


def sample_row(rng, row, n_valid, temperature, top_k, top_p):
    row = np.ascontiguousarray(row, np.float32)
    return lib().or_sample_row(rng.h, _ptr(row), n_valid, temperature, top_k, top_p)


def accept(rng, logits, drafts, n_valid, temperature, top_k, top_p):
    """serve/engine.cpp:592-610 on full rows: returns (j, tokens[: j + 1] or fewer on error, status)."""
    logits = np.ascontiguousarray(logits, np.float32)
    k = len(drafts)
    out = np.full(k + 1, -1, np.int32)
    st = ctypes.c_int32()
    j = lib().or_accept(rng.h, _ptr(logits), k, logits.shape[1], n_valid, _ptr(np.ascontiguousarray(drafts, np.int32)),
                        temperature, top_k, top_p, _ptr(out), ctypes.byref(st))
    return int(j), out, st.value


# ----- the compiled reference (formats + sampler), when oracle/_ref was built -----

_ref = None


def ref_available():
    return os.path.exists(REF_SO)


def ref():
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"{REF_SO} not built (needs /root/reference; `make -C oracle`)")
        L = ctypes.CDLL(REF_SO)
        L.ref_quantize.argtypes = [_INT, _P, _I64, _I64, _I64, _P, _P, _P, _P]
        L.ref_quantize.restype = _INT
        L.ref_dequantize.argtypes = [_INT, _P, _P, _P, _I64, _I64, _I64, _P]
        L.ref_dequantize.restype = _INT
        L.ref_q4_from_q8.argtypes = [_P, _P, _P, _I64, _I64, _I64, _I64, _INT, _P, _P, _P]
        L.ref_q4_from_q8.restype = _INT
        L.ref_top2.argtypes = [_P, _I64, _P, _P, _P, _P]
        L.ref_sampler_new.argtypes = [_D, _I64, _D, ctypes.c_uint64, _I64]
        L.ref_sampler_new.restype = _P
        L.ref_sampler_free.argtypes = [_P]
        L.ref_sampler_sample.argtypes = [_P, _P, _I64]
        L.ref_sampler_sample.restype = _I32
        L.ref_sampler_sample_candidates.argtypes = [_P, _P, _P, _I64, _INT]
        L.ref_sampler_sample_candidates.restype = _I32
        _ref = L
    return _ref


def ref_quantize(bits, w, G):
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    q = np.empty(N * K // (2 if bits == 4 else 1), np.uint8)
    s = np.empty(N * (K // G), np.uint16)
    m = np.empty(N * (K // G), np.uint16)
    d = np.empty((N, K), np.float32)
    rc = ref().ref_quantize(bits, _ptr(w), N, K, G, _ptr(q), _ptr(s), _ptr(m), _ptr(d))
    if rc != 0:
        raise ValueError("reference quantize refused the input")
    return QWeight(bits, q, s, m, N, K, G), d


def ref_q4_from_q8(w8, G4, threads=4):
    N, K = w8.N, w8.K
    q = np.empty(N * K // 2, np.uint8)
    s = np.empty(N * (K // G4), np.uint16)
    m = np.empty(N * (K // G4), np.uint16)
    if ref().ref_q4_from_q8(*w8.args(), N, K, w8.G, G4, threads, _ptr(q), _ptr(s), _ptr(m)) != 0:
        raise ValueError("reference quantize_q4_from_q8 refused the input")
    return QWeight(4, q, s, m, N, K, G4)


def ref_dequantize(w):
    d = np.empty((w.N, w.K), np.float32)
    if ref().ref_dequantize(w.bits, *w.args(), w.N, w.K, w.G, _ptr(d)) != 0:
        raise ValueError("reference dequantize refused the input")
    return d


def ref_top2(x):
    x = np.ascontiguousarray(x, np.float32)
    b, bv, sv, nan = ctypes.c_int32(), ctypes.c_float(), ctypes.c_float(), ctypes.c_uint32()
    ref().ref_top2(_ptr(x), x.size, ctypes.byref(b), ctypes.byref(bv), ctypes.byref(sv), ctypes.byref(nan))
    return b.value, bv.value, sv.value, nan.value


class RefSampler:
    def __init__(self, temperature, top_k, top_p, seed, n_valid):
        self.h = ref().ref_sampler_new(temperature, top_k, top_p, seed, n_valid)
        if not self.h:
            raise ValueError("reference Sampler refused the parameters")

    def sample(self, row):
        row = np.ascontiguousarray(row, np.float32)
        return ref().ref_sampler_sample(self.h, _ptr(row), row.size)

    def sample_candidates(self, v, ids, nan=False):
        v = np.ascontiguousarray(v, np.float32)
        ids = np.ascontiguousarray(ids, np.int32)
        return ref().ref_sampler_sample_candidates(self.h, _ptr(v), _ptr(ids), v.size, int(nan))

    def __del__(self):
        if getattr(self, "h", None):
            ref().ref_sampler_free(self.h)
            self.h = None
