"""The verify-width MoE sublayer in one launch (sx_moe_verify_layer) on cuda:0 through the C ABI.

Checked two ways on the same seeded inputs:
  - against the CPU oracle: the router logits (FP32 or BF16 weight, 1e-3), the routing bit-exact on those logits, h
    and y of the experts (runtime/qwen4exp.cpp:1132-1163's sequence);
  - against this library's two-launch path (sx_moe_verify_gate_up + sx_moe_verify_down) fed the one-launch kernel's
    own logits: ids, coefficients, h and y must be bit-identical, since the arithmetic is the same and only the hand-off
    of h between blocks differs. Repeated launches (16 batches back to back) check that each launch's hand-off flags
    never satisfy the next launch's waits.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests import util

pytestmark = pytest.mark.gpu


def kx():
    from strixite_amd import kernels
    return kernels


def sync():
    import torch
    torch.cuda.synchronize()


def two_launch(x, logits, gu, dn, E, k, shared, shared_id):
    """The two-launch FFN on given logits: ids, coef, h, y."""
    import torch
    M = x.shape[0]
    sl = logits[:, E:E + 1] if shared else None
    Ew = gu.N // (2 * dn.K)
    A = k + (1 if shared else 0)
    h_sums = torch.empty((M * A, dn.K // 16), dtype=torch.float32, device=x.device)
    ids, coef, h, rerr, eerr = kx().verify_gate_up(x, logits, gu, E, k, Ew=Ew, shared_logit=sl, shared_id=shared_id,
                                                   h_sums=h_sums)
    y, eerr2 = kx().verify_down(h, dn, ids, coef, Ew, h_sums=h_sums)
    return ids, coef, h, y, rerr, eerr


def check_against_oracle(x, Wr_host, wr_bf16, logits, ids, coef, h, y, gu, dn, E, k, I, d):
    from strixite_amd import synthetic as syn
    xh = util.host_bits(x)
    L = logits.cpu().numpy()
    ref_L = orc.linear_bf16w(xh, Wr_host, out_act=orc.F32) if wr_bf16 else orc.linear_f32w(xh, Wr_host)
    util.assert_close(L, ref_L, what="layer logits")
    ref_ids, ref_coef, _ = orc.moe_router(L[:, :E], E, k)
    g_ids = ids.cpu().numpy()[:, :k]
    assert np.array_equal(g_ids, ref_ids), "expert ids differ from the oracle on the layer's logits"
    util.assert_close(coef.cpu().numpy()[:, :k], ref_coef, tol=1e-6, what="coef")
    touched = np.unique(ref_ids)
    U = len(touched)
    rid = np.searchsorted(touched, ref_ids).astype(np.int32)
    cat = lambda w, rows: [np.concatenate(p) for p in zip(*[syn.host_rows(w, e * rows, (e + 1) * rows) for e in touched])]
    hgu = orc.QWeight(4, *cat(gu, 2 * I), U * 2 * I, d, 128)
    hdn = orc.QWeight(4, *cat(dn, d), U * d, I, 128)
    ref_h, _ = orc.experts_gather(xh, hgu, U, rid, swiglu=True)
    gh = util.host_bits(h)[:, :k]
    util.assert_close(gh, ref_h, roundings=4, what="layer h")
    ref_y, _ = orc.experts_combine(np.ascontiguousarray(gh), hdn, U, rid, coef.cpu().numpy()[:, :k])
    if ids.shape[1] == k:  # without a shared slot y is the routed experts' combine
        util.assert_close(util.host_bits(y), ref_y, what="layer y")


@pytest.mark.parametrize("wr_bf16", [False, True])
def test_layer_config3_matches_oracle_and_two_launch(wr_bf16):
    """BASELINE config 3 (M = 6, d = 4096, E = 512, top-10, I = 1024, q4 G = 128): FP32 router weight as the config
    states it, and the served model's BF16 weight."""
    import torch
    from strixite_amd import synthetic as syn
    E, d, I, k, M = 512, 4096, 1024, 10, 6
    gu = syn.qweight(4, E * 2 * I, d, 128, seed=71)
    dn = syn.qweight(4, E * d, I, 128, seed=72)
    Wr = syn.router_weight(E, d, seed=73)
    if wr_bf16:
        Wr = Wr.to(torch.bfloat16)
    Wr_host = util.host_bits(Wr)
    sy = kx().verify_layer_sync()
    for r in range(3):
        x = syn.activations(M, d, seed=74 + r)
        print(f"layer: config 3, wr_bf16={wr_bf16}, batch {r}", flush=True)
        logits, ids, coef, h, y, rerr, eerr = kx().verify_layer(x, Wr, gu, dn, E, k, sy)
        ids2, coef2, h2, y2, rerr2, eerr2 = two_launch(x, logits, gu, dn, E, k, False, 0)
        sync()
        assert list(rerr.cpu().numpy()[:3]) == [0, 0, 0] and list(eerr.cpu().numpy()[:3]) == [0, 0, 0]
        assert torch.equal(ids, ids2) and torch.equal(coef, coef2)
        assert torch.equal(h.view(torch.int16), h2.view(torch.int16)), "h differs from the two-launch path"
        assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), "y differs from the two-launch path"
        if r == 0:
            check_against_oracle(x, Wr_host, wr_bf16, logits, ids, coef, h, y, gu, dn, E, k, I, d)


def test_layer_shared_slot_and_back_to_back_batches():
    """The served layout: BF16 router weight [513, d] whose row 512 is the shared expert's gate, the shared expert
    stacked as expert 512 (A = 11, so M = 5 for M * A <= 64); 16 batches launched back to back, then each compared
    with the two-launch path on the same logits, bit for bit."""
    import torch
    from strixite_amd import synthetic as syn
    E, d, I, k, M, R = 512, 4096, 1024, 10, 5, 16
    Ew = E + 1
    gu = syn.qweight(4, Ew * 2 * I, d, 128, seed=81)
    dn = syn.qweight(4, Ew * d, I, 128, seed=82)
    Wr = syn.router_weight(E + 1, d, seed=83).to(torch.bfloat16)
    sy = kx().verify_layer_sync()
    xs = [syn.activations(M, d, seed=90 + r) for r in range(R)]
    outs = []
    for r in range(R):  # back to back: no host synchronisation between launches
        outs.append(kx().verify_layer(xs[r], Wr, gu, dn, E, k, sy, shared=True, shared_id=E, Ew=Ew))
    sync()
    print("layer: 16 back-to-back launches done", flush=True)
    for r in range(R):
        logits, ids, coef, h, y, rerr, eerr = outs[r]
        ids2, coef2, h2, y2, _, _ = two_launch(xs[r], logits, gu, dn, E, k, True, E)
        sync()
        assert list(eerr.cpu().numpy()[:3]) == [0, 0, 0], f"batch {r}: expert error {eerr.cpu().numpy()[:3]}"
        assert torch.equal(ids, ids2) and torch.equal(coef, coef2), f"batch {r}: routing"
        assert (ids[:, k] == E).all()
        assert torch.equal(h.view(torch.int16), h2.view(torch.int16)), f"batch {r}: h"
        assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), f"batch {r}: y"


def test_layer_nonfinite_token():
    """A token whose activations hold a NaN: its logits are NaN, the router fails it (ids -1, coef NaN, router error
    {1, token, 0}), its y row is NaN and the other tokens are unaffected - as in the two-launch path."""
    import torch
    from strixite_amd import synthetic as syn
    E, d, I, k, M = 512, 4096, 1024, 10, 6
    gu = syn.qweight(4, E * 2 * I, d, 128, seed=71)
    dn = syn.qweight(4, E * d, I, 128, seed=72)
    Wr = syn.router_weight(E, d, seed=73)
    x = syn.activations(M, d, seed=77)
    x[3, 100] = float("nan")
    sy = kx().verify_layer_sync()
    logits, ids, coef, h, y, rerr, eerr = kx().verify_layer(x, Wr, gu, dn, E, k, sy)
    ids2, coef2, h2, y2, rerr2, eerr2 = two_launch(x, logits, gu, dn, E, k, False, 0)
    sync()
    assert list(rerr.cpu().numpy()[:3]) == [1, 3, 0]
    assert (ids[3] == -1).all() and torch.isnan(coef[3]).all()
    assert torch.isnan(y[3].float()).all() and not torch.isnan(y[[0, 1, 2, 4, 5]].float()).any()
    assert torch.equal(ids, ids2)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))


def test_layer_rejects_unsupported_shapes():
    import strixite_amd as sx
    import torch
    from strixite_amd import synthetic as syn
    gu = syn.qweight(4, 8 * 2 * 1024, 2048, 128, seed=1)  # d = 2048: the two-launch FFN's, not the one-launch's
    dn = syn.qweight(4, 8 * 2048, 1024, 128, seed=2)
    x = torch.zeros((2, 2048), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(sx.SxError, match="d = 4096"):
        kx().verify_layer(x, torch.zeros((8, 2048), device="cuda"), gu, dn, 8, 2, kx().verify_layer_sync())
