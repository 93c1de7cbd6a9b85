"""The verify path as the reference's runtime strings the operators together (runtime/qwen4exp.cpp:1130-1160 for the
MoE sublayer at T >= kGroupedMinTokens, 1191-1210 for the head, serve/engine.cpp:592-610 for the accept loop), on
preallocated device buffers so a forward allocates nothing.
"""
import torch

from . import MOE_F32, SxError
from . import kernels as kx


class MoeVerifyLayer:
    """One MoE FFN sublayer. Weights: Wr FP32 [E, d], gate_up q4 [E * 2I, d], down q4 [E * d, I] (experts stacked,
    runtime/qwen4exp.cpp:126-129). At verify width (the shapes kernels.verify_supported takes) three launches:
    router projection -> routing + gate_up + SwiGLU (the tails of its compute units' shares balanced through a sync
    buffer the layer owns) -> down + combine (the sequence qwen4exp.cpp:1139-1163 runs below kGroupedMinTokens). Otherwise (or fused=False): router projection -> moe_router + moe_group_routes -> grouped
    gate_up with the SwiGLU epilogue -> grouped down + combine."""

    def __init__(self, Wr, gate_up, down, E, k, max_tokens, act_dtype=torch.bfloat16, fused=True):
        self.Wr, self.gate_up, self.down, self.E, self.k = Wr, gate_up, down, E, k
        self.d = gate_up.K
        self.I = down.K
        assert gate_up.N == E * 2 * self.I and down.N == E * self.d
        dev = Wr.device
        M, A = max_tokens, k
        self.M = M
        self.logits = torch.empty((M, E), dtype=torch.float32, device=dev)
        self.ids = torch.empty((M, A), dtype=torch.int32, device=dev)
        self.coef = torch.empty((M, A), dtype=torch.float32, device=dev)
        self.router_err = torch.zeros(4, dtype=torch.int32, device=dev)
        self.expert_err = torch.zeros(4, dtype=torch.int32, device=dev)
        self.ws = torch.empty(kx.route_workspace_bytes(M, A, E) // 4, dtype=torch.int32, device=dev)
        self.h = torch.empty((M, A, self.I), dtype=act_dtype, device=dev)
        self.h_sums = torch.empty((M * A, (self.I + 15) // 16), dtype=torch.float32, device=dev)
        self.partial = torch.empty((M * A, self.d), dtype=torch.float32, device=dev)
        self.y = torch.empty((M, self.d), dtype=act_dtype, device=dev)
        self.fused = fused and act_dtype == torch.bfloat16
        # the gate_up pool's sync buffers, one per stream: launches on one buffer must run in order, which only one
        # stream guarantees
        self._syncs = {}
        self.plan = kx.verify_plan(dev)  # the routing gate_up hands to down (written and read in stream order)
        self._dev = dev

    def _sync_for(self, stream):
        key = (stream or torch.cuda.current_stream(self._dev)).cuda_stream
        if key not in self._syncs:
            self._syncs[key] = kx.verify_layer_sync(self._dev)
        return self._syncs[key]

    def _fused(self, M):
        return self.fused and kx.verify_supported(M, self.k, self.E, self.k, self.E, self.gate_up, self.down)

    def forward(self, x, stream=None):
        M = x.shape[0]
        assert M <= self.M
        ws = self.ws if M == self.M else self.ws[:kx.route_workspace_bytes(M, self.k, self.E) // 4]
        kx.linear_f32w(x, self.Wr, y=self.logits[:M], stream=stream)
        if self._fused(M):
            kx.verify_gate_up(x, self.logits[:M], self.gate_up, self.E, self.k, ids=self.ids[:M], coef=self.coef[:M],
                              h=self.h[:M], router_err=self.router_err, expert_err=self.expert_err,
                              h_sums=self.h_sums, sync=self._sync_for(stream), plan=self.plan, stream=stream)
            kx.verify_down(self.h[:M], self.down, self.ids[:M], self.coef[:M], self.E, y=self.y[:M],
                           expert_err=self.expert_err, h_sums=self.h_sums, plan=self.plan, stream=stream)
            return self.y[:M]
        if M * self.k <= 2048:  # top-k + grouping in one launch
            kx.router_group(self.logits[:M], self.E, self.k, ws=ws, ids=self.ids[:M], coef=self.coef[:M],
                            router_err=self.router_err, expert_err=self.expert_err, stream=stream)
        else:
            kx.moe_router(self.logits[:M], self.E, self.k, ids=self.ids[:M], coef=self.coef[:M],
                          err=self.router_err, stream=stream)
            kx.group_routes(self.ids[:M], self.E, ws=ws, err=self.expert_err, stream=stream)
        kx.gather_grouped(x, self.gate_up, self.E, ws, M, self.k, swiglu=True, y=self.h[:M], stream=stream)
        kx.combine_grouped(self.h[:M], self.down, self.E, self.ids[:M], self.coef[:M], ws,
                           partial=self.partial[:M * self.k], y=self.y[:M], math=MOE_F32, stream=stream)
        return self.y[:M]

    def weight_bytes_touched(self, M=None):
        """Algorithmic bytes of the last forward: the distinct experts' gate_up + down rows, the router weight and
        the activations in and out (synchronizes to read the ids)."""
        M = self.M if M is None else M
        U = int(torch.unique(self.ids[:M]).numel())
        per_expert = (self.gate_up.nbytes() + self.down.nbytes()) // self.E
        act = M * self.d * self.y.element_size()
        return U, U * per_expert + self.Wr.numel() * 4 + 2 * act


class VerifyTail:
    """The verify head: q8 LM head [V, d] -> FP32 logits [M, V] -> logits_topk (k candidates) -> device acceptance."""

    def __init__(self, lm_head, n_valid, k_cands, max_rows):
        self.w, self.n_valid, self.kc = lm_head, n_valid, k_cands
        dev = lm_head.q.device
        self.logits = torch.empty((max_rows, lm_head.N), dtype=torch.float32, device=dev)
        self.cands = torch.empty((max_rows, k_cands, 2), dtype=torch.int32, device=dev)
        self.nan = torch.empty(max_rows, dtype=torch.int32, device=dev)
        self.ws = torch.empty(kx.topk_workspace_bytes(max_rows, n_valid, k_cands) // 8 + 1, dtype=torch.int64,
                              device=dev)
        self.out = torch.empty(2 + max_rows, dtype=torch.int32, device=dev)
        # top-k and acceptance as one launch where the first level's candidates fit one block a row
        try:
            self.tail_ws = kx.verify_tail_workspace(max_rows, n_valid, k_cands, dev)
        except SxError:  # more first-level candidates a row than one block reduces: two launches
            self.tail_ws = None

    def forward(self, h, drafts, u, temperature, top_k, top_p, stream=None):
        M = h.shape[0]
        kx.linear(h, self.w, out_act=0, y=self.logits[:M], stream=stream)
        out = self.out[:2 + drafts.numel() + 1]
        if self.tail_ws is not None and M >= drafts.numel() + 1:
            kx.verify_tail(self.logits[:M], self.n_valid, self.kc, self.tail_ws, drafts=drafts, u=u,
                           temperature=temperature, top_k=top_k, top_p=top_p, cands=self.cands[:M],
                           nan=self.nan[:M], out=out, stream=stream)
            return out
        kx.logits_topk(self.logits[:M], self.n_valid, self.kc, ws=self.ws, out=self.cands[:M], nan=self.nan[:M],
                       stream=stream)
        return kx.mtp_accept(self.cands[:M], self.nan[:M], drafts, u, temperature, top_k, top_p, self.n_valid,
                             out=out, stream=stream)
