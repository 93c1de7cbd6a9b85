"""The draft side of the MTP step: the draft head's Q4 copy and its top-2 pick, and the engine's decisions around a
verify (serve/engine.cpp:560-653).

DraftHead is the tail of Qwen4ExpSession::run_mtp / forward_mtp_top2 (runtime/qwen4exp.cpp:1540-1560, 1418-1443):
the MTP layer's collapsed hidden state through the first mtp_vocab rows of the LM head - the Q4 copy
Qwen4ExpModel::make_draft_head_q4 makes of the Q8 head (runtime/qwen4exp.cpp:192-238, formats/q4_from_q8.hpp), made
here on the device from the resident Q8 rows - to FP32 logits, then mtp_pick's top-2 with the forward's error words
in one 64-byte record. The pick runs inside the GEMV's launch (sx_mtp_head_pick: each block keeps the top-2 of the
logits it writes, the last block to finish merges them), bit-identical to the separate pick. The MTP layer itself
(attention, hyper-connections) is outside this library.

draft_continues and commit_after_accept are the engine's host-side rules (serve/engine.cpp:574-581, 612-645): whether a
draft is kept and chained, and which part of the verify the session keeps once the accepted length is known.
"""
import torch

from . import kernels as kx


class DraftHead:
    def __init__(self, lm_head_q8, mtp_vocab, G=64):
        """lm_head_q8: the served Q8 LM head (kernels.QWeight, bits 8); its first mtp_vocab rows get a Q4 copy with
        group G (the served draft head uses 64)."""
        assert lm_head_q8.bits == 8 and 1 <= mtp_vocab <= lm_head_q8.N
        self.mtp_vocab = mtp_vocab
        self.w, self.copy_err = kx.quantize_q4_from_q8(lm_head_q8, G, rows=mtp_vocab)
        dev = lm_head_q8.q.device
        self.logits = torch.empty((1, mtp_vocab), dtype=torch.float32, device=dev)
        self.pick = torch.empty(64, dtype=torch.uint8, device=dev)
        self.pick_ws = torch.zeros(kx.mtp_pick_ws_bytes(mtp_vocab), dtype=torch.uint8, device=dev)
        self.zero_err = torch.zeros(4, dtype=torch.int32, device=dev)
        self.zero_emb = torch.zeros(1, dtype=torch.int64, device=dev)

    def forward(self, h, router_err=None, expert_err=None, attn_err=None, emb_err=None, stream=None):
        """h: BF16 [1, d], the head's hidden state. Queues the logits and the pick (no synchronisation)."""
        z = self.zero_err
        return kx.mtp_head_pick(h, self.w, self.logits, router_err if router_err is not None else z,
                                expert_err if expert_err is not None else z, attn_err if attn_err is not None else z,
                                emb_err if emb_err is not None else self.zero_emb, self.pick_ws, out=self.pick,
                                stream=stream)

    def top2(self):
        """The pick read back (one synchronisation, as forward_mtp_top2 does): an MtpPick."""
        return kx.pick_from_bytes(self.pick)


def draft_continues(pick, margin, stop_ids):
    """serve/engine.cpp:574-581: a draft is kept (and the chain goes on) when its top-1 margin reaches `margin` and it
    is no end-of-turn token; a NaN in the draft logits is an error."""
    if pick.nan:
        raise RuntimeError("NaN in the MTP draft logits")
    return pick.best_v - pick.second_v >= margin and pick.best not in stop_ids


def commit_after_accept(j, k):
    """serve/engine.cpp:612-645: after j of k drafts were accepted, the verify rows the session keeps (whether or not
    the response ends there). Returns ("keep_verify", k + 1) when every draft was accepted, else
    ("keep_verify_prefix", j + 1): the verified token and the j accepted drafts (Qwen4ExpSession::keep_verify_prefix,
    runtime/qwen4exp.cpp:1298-1362)."""
    if not 0 <= j <= k:
        raise ValueError(f"accepted length {j} outside 0..{k}")
    if j == k:
        return ("keep_verify", k + 1)
    return ("keep_verify_prefix", j + 1)
