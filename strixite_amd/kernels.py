"""Python face of the C ABI over torch device tensors: the reference's strix::kernels operators by name
(kernels/linear_q4.hpp, linear_q8.hpp, moe_router.hpp, moe_grouped.hpp, swiglu.hpp, logits_topk.hpp, mtp_pick.hpp).

torch supplies device memory and the stream (torch.cuda.current_stream() unless one is passed); every computation is
a libstrixite_amd.so kernel. Activations are torch.float32 (Act::F32) or torch.bfloat16 (Act::BF16, raw bits).
"""
import ctypes

import torch

from . import (ACT_BF16, ACT_F32, MOE_F32, LogitCand, MtpPick, QView, check, lib)

_c = ctypes.c_void_p


def _p(t):
    return None if t is None else _c(t.data_ptr())


def _s(stream=None):
    return _c((stream if stream is not None else torch.cuda.current_stream()).cuda_stream)


def act_of(t):
    if t.dtype == torch.float32:
        return ACT_F32
    if t.dtype == torch.bfloat16:
        return ACT_BF16
    raise TypeError(f"activations are float32 or bfloat16, got {t.dtype}")


def dtype_of(act):
    return torch.float32 if act == ACT_F32 else torch.bfloat16


class QWeight:
    """A q4 / q8 weight resident on the device (Q4Device / Q8Device, runtime/q4_device.hpp:23-36): codes uint8,
    scale / min as BF16 bits (int16 tensors), in the formats/q4.hpp / q8.hpp layout."""

    def __init__(self, bits, q, scale, minv, N, K, G):
        self.bits, self.q, self.scale, self.minv = bits, q, scale, minv
        self.N, self.K, self.G = int(N), int(K), int(G)
        self._view = QView(q.data_ptr(), scale.data_ptr(), minv.data_ptr(), self.N, self.K, self.G)

    @classmethod
    def upload(cls, host, device="cuda"):
        """From a host weight with numpy arrays q, scale, minv (e.g. oracle.QWeight)."""
        t = lambda a: torch.from_numpy(a.view(a.dtype)).to(device)
        return cls(host.bits, t(host.q), t(host.scale.view("int16")), t(host.minv.view("int16")), host.N, host.K, host.G)

    def view(self):
        return ctypes.byref(self._view)

    def nbytes(self):
        return self.q.numel() + 2 * self.scale.numel() + 2 * self.minv.numel()


def linear(x, w, out_act=None, y=None, stream=None):
    """y[M, N] = x[M, K] * deq(W)^T (linear_q4 / linear_q8)."""
    act = act_of(x)
    out_act = act if out_act is None else out_act
    M = x.shape[0]
    if y is None:
        y = torch.empty((M, w.N), dtype=dtype_of(out_act), device=x.device)
    f = lib().sx_linear_q4 if w.bits == 4 else lib().sx_linear_q8
    check(f(_p(x), w.view(), _p(y), M, act, out_act, _s(stream)))
    return y


def _err(device):
    return torch.zeros(4, dtype=torch.int32, device=device)


def experts_gather(x, w, E, ids, swiglu=False, y=None, err=None, stream=None):
    """Per-slot gather (linear_q4_experts_gather) or its SwiGLU form (linear_q4_experts_gather_swiglu)."""
    act = act_of(x)
    M, A = ids.shape
    N = w.N // E
    out_n = N // 2 if swiglu else N
    y = torch.empty((M, A, out_n), dtype=x.dtype, device=x.device) if y is None else y
    err = _err(x.device) if err is None else err
    f = lib().sx_linear_q4_experts_gather_swiglu if swiglu else lib().sx_linear_q4_experts_gather
    check(f(_p(x), w.view(), E, _p(ids), M, A, _p(y), act, _p(err), _s(stream)))
    return y, err


def experts_combine(h, w, E, ids, coef, y=None, err=None, stream=None):
    act = act_of(h)
    M, A = ids.shape
    N = w.N // E
    y = torch.empty((M, N), dtype=h.dtype, device=h.device) if y is None else y
    err = _err(h.device) if err is None else err
    check(lib().sx_linear_q4_experts_combine(_p(h), w.view(), E, _p(ids), _p(coef), M, A, _p(y), act, _p(err),
                                             _s(stream)))
    return y, err


def moe_router(logits, E, k, shared=None, shared_ld=1, shared_id=0, ids=None, coef=None, err=None, stream=None):
    M, ld = logits.shape
    A = k + (1 if shared is not None else 0)
    ids = torch.empty((M, A), dtype=torch.int32, device=logits.device) if ids is None else ids
    coef = torch.empty((M, A), dtype=torch.float32, device=logits.device) if coef is None else coef
    err = _err(logits.device) if err is None else err
    check(lib().sx_moe_router(_p(logits), ld, M, E, k, _p(shared), shared_ld, shared_id, _p(ids), _p(coef),
                              act_of(logits), _p(err), _s(stream)))
    return ids, coef, err


def route_workspace_bytes(M, A, E):
    n = ctypes.c_size_t()
    check(lib().sx_moe_route_workspace_bytes(M, A, E, ctypes.byref(n)))
    return n.value


def router_group(logits, E, k, ws=None, ids=None, coef=None, router_err=None, expert_err=None, stream=None):
    """moe_router + moe_group_routes in one launch (M * k <= 2048)."""
    M, ld = logits.shape
    dev = logits.device
    ws = torch.empty(route_workspace_bytes(M, k, E) // 4, dtype=torch.int32, device=dev) if ws is None else ws
    ids = torch.empty((M, k), dtype=torch.int32, device=dev) if ids is None else ids
    coef = torch.empty((M, k), dtype=torch.float32, device=dev) if coef is None else coef
    router_err = _err(dev) if router_err is None else router_err
    expert_err = _err(dev) if expert_err is None else expert_err
    check(lib().sx_moe_router_group(_p(logits), ld, M, E, k, act_of(logits), _p(ids), _p(coef), _p(router_err),
                                    _p(ws), ws.numel() * 4, _p(expert_err), _s(stream)))
    return ids, coef, ws, router_err, expert_err


def verify_supported(M, A, E, k, Ew, gate_up, down, act=ACT_BF16):
    """Whether the two-launch verify FFN (verify_gate_up + verify_down) takes this shape."""
    return lib().sx_moe_verify_supported(M, A, E, k, Ew, gate_up.view(), down.view(), act) == 0


def verify_gate_up(x, logits, w, E, k, Ew=None, shared_logit=None, shared_id=0, ids=None, coef=None, h=None,
                   router_err=None, expert_err=None, h_sums=None, sync=None, plan=None, stream=None):
    """moe_router + gather_swiglu in one launch at verify width: ids, coef [M, A], h [M, A, I]. h_sums (optional,
    FP32 [M * A, ceil(I / 16)]) receives the 16-feature sums of h that verify_down can take. sync (optional,
    verify_layer_sync(), one per stream): after a fixed run each compute unit takes weight tiles from a shared pool
    (K = 4096), so the faster ones take more; same outputs. plan (optional, verify_plan()) receives the routing in
    the form verify_down takes it."""
    M, ld = x.shape[0], logits.stride(0)
    Ew = E if Ew is None else Ew
    A = k + (shared_logit is not None)
    I = w.N // Ew // 2
    dev = x.device
    ids = torch.empty((M, A), dtype=torch.int32, device=dev) if ids is None else ids
    coef = torch.empty((M, A), dtype=torch.float32, device=dev) if coef is None else coef
    h = torch.empty((M, A, I), dtype=x.dtype, device=dev) if h is None else h
    router_err = _err(dev) if router_err is None else router_err
    expert_err = _err(dev) if expert_err is None else expert_err
    sld = 0 if shared_logit is None else shared_logit.stride(0)
    check(lib().sx_moe_verify_gate_up(_p(x), M, _p(logits), ld, E, k, _p(shared_logit), sld, shared_id, w.view(), Ew,
                                      _p(ids), _p(coef), _p(h), _p(h_sums), act_of(x), _p(router_err),
                                      _p(expert_err), _p(sync), _p(plan), _s(stream)))
    return ids, coef, h, router_err, expert_err


def verify_down(h, w, ids, coef, Ew, y=None, expert_err=None, h_sums=None, plan=None, stream=None):
    """y[M, N] = sum_a coef[m, a] * (h[m, a] . W[ids[m, a]]) in one launch at verify width (h_sums: verify_gate_up's
    sums of this h, optional; plan: the routing plan verify_gate_up stored with these ids, optional)."""
    M, A = ids.shape
    N = w.N // Ew
    y = torch.empty((M, N), dtype=h.dtype, device=h.device) if y is None else y
    expert_err = _err(h.device) if expert_err is None else expert_err
    check(lib().sx_moe_verify_down(_p(h), _p(h_sums), M, A, _p(ids), _p(coef), w.view(), Ew, _p(y), act_of(h),
                                   _p(expert_err), _p(plan), _s(stream)))
    return y, expert_err


VERIFY_PLAN_BYTES = 4096  # SX_VERIFY_PLAN_BYTES


def verify_plan(device="cuda"):
    """A buffer for the routing plan verify_gate_up stores and verify_down takes."""
    return torch.empty(VERIFY_PLAN_BYTES // 4, dtype=torch.int32, device=device)


def verify_layer_sync(device="cuda"):
    """A zeroed sync buffer for verify_layer and verify_gate_up (one per stream; each launch readies it for the next)."""
    n = ctypes.c_size_t()
    check(lib().sx_moe_verify_layer_sync_bytes(ctypes.byref(n)))
    return torch.zeros((n.value + 3) // 4, dtype=torch.int32, device=device)


def verify_layer(x, Wr, gate_up, down, E, k, sync, shared=False, shared_id=0, Ew=None, logits=None, ids=None,
                 coef=None, h=None, h_sums=None, y=None, router_err=None, expert_err=None, stream=None):
    """The verify-width MoE sublayer in one launch: x [M, d] BF16, Wr [rows, d] FP32 or BF16 (raw bits as int16 or
    torch.bfloat16) -> logits [M, rows], ids / coef [M, A], h [M, A, I], h_sums, y [M, d]."""
    M, d = x.shape
    rows = Wr.shape[0]
    Ew = E if Ew is None else Ew
    A = k + (1 if shared else 0)
    I = gate_up.N // Ew // 2
    dev = x.device
    wr_act = ACT_F32 if Wr.dtype == torch.float32 else ACT_BF16
    logits = torch.empty((M, rows), dtype=torch.float32, device=dev) if logits is None else logits
    ids = torch.empty((M, A), dtype=torch.int32, device=dev) if ids is None else ids
    coef = torch.empty((M, A), dtype=torch.float32, device=dev) if coef is None else coef
    h = torch.empty((M, A, I), dtype=x.dtype, device=dev) if h is None else h
    h_sums = torch.empty((M * A, (I + 15) // 16), dtype=torch.float32, device=dev) if h_sums is None else h_sums
    y = torch.empty((M, down.N // Ew), dtype=x.dtype, device=dev) if y is None else y
    router_err = _err(dev) if router_err is None else router_err
    expert_err = _err(dev) if expert_err is None else expert_err
    check(lib().sx_moe_verify_layer(_p(x), M, _p(Wr), wr_act, rows, E, k, int(shared), shared_id, gate_up.view(),
                                    down.view(), Ew, _p(logits), _p(ids), _p(coef), _p(h), _p(h_sums), _p(y),
                                    act_of(x), _p(router_err), _p(expert_err), _p(sync), _s(stream)))
    return logits, ids, coef, h, y, router_err, expert_err


def group_routes(ids, E, ws=None, err=None, stream=None):
    M, A = ids.shape
    nb = route_workspace_bytes(M, A, E)
    ws = torch.empty(nb // 4, dtype=torch.int32, device=ids.device) if ws is None else ws
    err = _err(ids.device) if err is None else err
    check(lib().sx_moe_group_routes(_p(ids), M, A, E, _p(ws), ws.numel() * 4, _p(err), _s(stream)))
    return ws, err


def gather_grouped(x, w, E, ws, M, A, swiglu=False, y=None, math=MOE_F32, stream=None):
    act = act_of(x)
    N = w.N // E
    out_n = N // 2 if swiglu else N
    y = torch.empty((M, A, out_n), dtype=x.dtype, device=x.device) if y is None else y
    if swiglu:
        check(lib().sx_linear_q4_experts_gather_swiglu_grouped(_p(x), w.view(), E, _p(ws), ws.numel() * 4, M, A, _p(y),
                                                               act, _s(stream)))
    else:
        check(lib().sx_linear_q4_experts_gather_grouped(_p(x), w.view(), E, _p(ws), ws.numel() * 4, M, A, _p(y), act,
                                                        math, _s(stream)))
    return y


def combine_grouped(h, w, E, ids, coef, ws, partial=None, y=None, math=MOE_F32, stream=None):
    act = act_of(h)
    M, A = ids.shape
    N = w.N // E
    y = torch.empty((M, N), dtype=h.dtype, device=h.device) if y is None else y
    partial = torch.empty((M * A, N), dtype=torch.float32, device=h.device) if partial is None else partial
    check(lib().sx_linear_q4_experts_combine_grouped(_p(h), w.view(), E, _p(ids), _p(coef), _p(ws), ws.numel() * 4,
                                                     _p(partial), M, A, _p(y), act, math, _s(stream)))
    return y


def swiglu(gu, h=None, stream=None):
    rows, I2 = gu.shape
    h = torch.empty((rows, I2 // 2), dtype=gu.dtype, device=gu.device) if h is None else h
    check(lib().sx_swiglu(_p(gu), _p(h), rows, I2 // 2, act_of(gu), _s(stream)))
    return h


def linear_f32w(x, W, y=None, stream=None):
    M, K = x.shape
    N = W.shape[0]
    y = torch.empty((M, N), dtype=torch.float32, device=x.device) if y is None else y
    check(lib().sx_linear_f32w(_p(x), _p(W), N, K, _p(y), M, act_of(x), _s(stream)))
    return y


def linear_bf16w(x, W, out_act=None, y=None, wmma=False, stream=None):
    """y[M, N] = x[M, K] * W^T with W BF16 [N, K] (linear_bf16w; wmma: linear_bf16w_wmma, x rounded to BF16)."""
    act = act_of(x)
    out_act = act if out_act is None else out_act
    M, K = x.shape
    N = W.shape[0]
    y = torch.empty((M, N), dtype=dtype_of(out_act), device=x.device) if y is None else y
    f = lib().sx_linear_bf16w_wmma if wmma else lib().sx_linear_bf16w
    check(f(_p(x), _p(W), _p(y), M, N, K, act, out_act, _s(stream)))
    return y


def moe_shared_add(y, s, gate_logit, gate_index, err, x=None, w_in=None, stream=None):
    """moe_shared_add (x None) or moe_shared_add_inject, in place on y (and x [M, H * N]). gate_logit: FP32 column
    view (row stride = its stride(0))."""
    M, N = y.shape
    gl = gate_logit.stride(0)
    if x is None:
        check(lib().sx_moe_shared_add(_p(y), _p(s), _p(gate_logit), gl, M, N, gate_index, act_of(y), _p(err),
                                      _s(stream)))
    else:
        check(lib().sx_moe_shared_add_inject(_p(y), _p(s), _p(gate_logit), gl, M, N, gate_index, _p(x), _p(w_in),
                                             x.shape[1] // N, act_of(y), _p(err), _s(stream)))
    return y


def topk_workspace_bytes(rows, n_valid, k):
    n = ctypes.c_size_t()
    check(lib().sx_logits_topk_workspace_bytes(rows, n_valid, k, ctypes.byref(n)))
    return n.value


def logits_topk(logits, n_valid, k=20, mask=None, ws=None, out=None, nan=None, stream=None):
    """Per row the best k (value desc, lower id on a tie) of logits [rows, >= n_valid] (any row stride). Returns
    (values f32 [rows, k], ids i32 [rows, k], nan, the raw [rows, k, 2] candidates)."""
    rows, ld = logits.shape[0], logits.stride(0)
    out = torch.empty((rows, k, 2), dtype=torch.int32, device=logits.device) if out is None else out
    nan = torch.empty(rows, dtype=torch.int32, device=logits.device) if nan is None else nan
    if ws is None:
        ws = torch.empty(topk_workspace_bytes(rows, n_valid, k) // 8 + 1, dtype=torch.int64, device=logits.device)
    mw = 0 if mask is None else mask.shape[1]
    check(lib().sx_logits_topk(_p(logits), rows, ld, n_valid, k, _p(out), _p(nan), _p(ws), ws.numel() * 8, _p(mask), mw,
                               _s(stream)))
    return out[..., 0].view(torch.float32), out[..., 1], nan, out


def logits_topk_noalloc(logits, n_valid, k=20, mask=None, out=None, nan=None, stream=None):
    """logits_topk on the library's fixed scratch (sx_logits_topk_noalloc: no workspace, nothing allocated by the
    call). Same returns as logits_topk."""
    rows, ld = logits.shape[0], logits.stride(0)
    out = torch.empty((rows, k, 2), dtype=torch.int32, device=logits.device) if out is None else out
    nan = torch.empty(rows, dtype=torch.int32, device=logits.device) if nan is None else nan
    mw = 0 if mask is None else mask.shape[1]
    check(lib().sx_logits_topk_noalloc(_p(logits), rows, ld, n_valid, k, _p(out), _p(nan), _p(mask), mw, _s(stream)))
    return out[..., 0].view(torch.float32), out[..., 1], nan, out


def quantize_q4_from_q8(w8, G=64, rows=None, err=None, stream=None):
    """The Q4 copy of the first `rows` rows of a Q8 weight (formats/q4_from_q8.hpp), made on the device: a QWeight."""
    rows = w8.N if rows is None else rows
    dev = w8.q.device
    q = torch.empty(rows * w8.K // 2, dtype=torch.uint8, device=dev)
    s = torch.empty(rows * (w8.K // G), dtype=torch.int16, device=dev)
    m = torch.empty(rows * (w8.K // G), dtype=torch.int16, device=dev)
    err = _err(dev) if err is None else err
    src = QView(w8.q.data_ptr(), w8.scale.data_ptr(), w8.minv.data_ptr(), rows, w8.K, w8.G)
    check(lib().sx_quantize_q4_from_q8(ctypes.byref(src), G, _p(q), _p(s), _p(m), _p(err), _s(stream)))
    return QWeight(4, q, s, m, rows, w8.K, G), err


def mtp_pick_ws_bytes(n):
    b = ctypes.c_size_t()
    check(lib().sx_mtp_pick_ws_bytes(n, ctypes.byref(b)))
    return b.value


def mtp_pick(logits, router_err, expert_err, attn_err, emb_err, out=None, ws=None, stream=None):
    """The 64-byte pick of `logits`. With `ws` (a zeroed device uint8 buffer of mtp_pick_ws_bytes, reused across
    calls on one stream) the one-launch many-block pick runs; its output is bit-identical to the single-block one's."""
    out = torch.empty(64, dtype=torch.uint8, device=logits.device) if out is None else out
    if ws is None:
        check(lib().sx_mtp_pick(_p(logits), logits.numel(), _p(router_err), _p(expert_err), _p(attn_err),
                                _p(emb_err), _p(out), _s(stream)))
    else:
        check(lib().sx_mtp_pick_ws(_p(logits), logits.numel(), _p(router_err), _p(expert_err), _p(attn_err),
                                   _p(emb_err), _p(out), _p(ws), ws.numel() * ws.element_size(), _s(stream)))
    return out


def mtp_head_pick(x, w, logits, router_err, expert_err, attn_err, emb_err, ws, out=None, stream=None):
    """The draft head's logits (x BF16 [1, K] against the q4 / q8 head, FP32 [N] into `logits`) and their pick, one
    launch; `ws` a zeroed device uint8 buffer of mtp_pick_ws_bytes. Returns the 64-byte pick."""
    out = torch.empty(64, dtype=torch.uint8, device=x.device) if out is None else out
    assert x.dtype == torch.bfloat16 and x.numel() == w.K and logits.numel() >= w.N
    check(lib().sx_mtp_head_pick(_p(x), w.view(), w.bits, _p(logits), _p(router_err), _p(expert_err), _p(attn_err),
                                 _p(emb_err), _p(out), _p(ws), ws.numel() * ws.element_size(), _s(stream)))
    return out


def pick_from_bytes(b):
    """The 64 bytes of an sx_mtp_pick_t (host) as the ctypes struct."""
    return MtpPick.from_buffer_copy(bytes(b.cpu().numpy().tobytes()))


def verify_tail_workspace_bytes(rows, n_valid, kc):
    n = ctypes.c_size_t()
    check(lib().sx_verify_tail_workspace_bytes(rows, n_valid, kc, ctypes.byref(n)))
    return n.value


def verify_tail_workspace(rows, n_valid, kc, device="cuda"):
    """A zeroed workspace for verify_tail (one per stream; each launch leaves its counters at zero)."""
    return torch.zeros(verify_tail_workspace_bytes(rows, n_valid, kc) // 8 + 1, dtype=torch.int64, device=device)


def verify_tail(logits, n_valid, kc, ws, drafts=None, u=None, temperature=0.0, top_k=1, top_p=1.0, mask=None,
                cands=None, nan=None, out=None, stream=None):
    """logits_topk (kc candidates a row) and, with drafts, mtp_accept in one launch. Returns (cands [rows, kc, 2],
    nan, out or None)."""
    rows, ld = logits.shape[0], logits.stride(0)
    dev = logits.device
    cands = torch.empty((rows, kc, 2), dtype=torch.int32, device=dev) if cands is None else cands
    nan = torch.empty(rows, dtype=torch.int32, device=dev) if nan is None else nan
    k = 0 if drafts is None else drafts.numel()
    if drafts is not None and out is None:
        out = torch.full((2 + k + 1,), -1, dtype=torch.int32, device=dev)
    mw = 0 if mask is None else mask.shape[1]
    check(lib().sx_verify_tail(_p(logits), rows, ld, n_valid, kc, _p(cands), _p(nan), _p(mask), mw, _p(drafts), k,
                               _p(u), float(temperature), int(top_k), float(top_p),
                               _p(out) if drafts is not None else None, _p(ws), ws.numel() * 8, _s(stream)))
    return cands, nan, out


def mtp_accept(cands, nan, drafts, u, temperature, top_k, top_p, n_valid, out=None, stream=None):
    """cands: the raw [k+1, kc, 2] int32 output of logits_topk. Returns the device int32 vector
    [j, status, tokens...]."""
    rows, kc = cands.shape[0], cands.shape[1]
    k = drafts.numel()
    assert rows >= k + 1, "one candidate row per draft plus the last"
    out = torch.full((2 + k + 1,), -1, dtype=torch.int32, device=cands.device) if out is None else out
    check(lib().sx_mtp_accept(_p(cands), _p(nan), kc, _p(drafts), k, _p(u), float(temperature), int(top_k),
                              float(top_p), int(n_valid), _p(out), _s(stream)))
    return out
