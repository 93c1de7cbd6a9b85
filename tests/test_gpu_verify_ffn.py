"""The two-launch verify FFN (sx_moe_verify_gate_up + sx_moe_verify_down) on cuda:0 against the CPU oracle's
moe_router -> experts_gather_swiglu -> experts_combine (the sequence runtime/qwen4exp.cpp:1139-1163 runs below
kGroupedMinTokens), and against this library's own per-slot kernels for the error paths."""
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


def make(seed, Ew, I, d):
    rng = np.random.default_rng(seed)
    wgu = util.rand_qweight(rng, 4, Ew * 2 * I, d, 128)
    wdn = util.rand_qweight(rng, 4, Ew * d, I, 128)
    return wgu, wdn, rng


def run_fused(x, L, wgu, wdn, E, k, shared, sums=True):
    """gate_up then down; with `sums` gate_up also writes h_sums and down takes them (the layer's path), which is
    checked here against h itself (each 16-feature run of a valid slot's row, summed in float64)."""
    import torch
    Ew = E + (1 if shared else 0)
    Wgu, Wdn = kx().QWeight.upload(wgu), kx().QWeight.upload(wdn)
    Ld = util.f32_dev(L)
    sl = Ld[:, E:] if shared else None
    M, I = x.shape[0], wdn.K
    A = k + (1 if shared else 0)
    hs = torch.full((M * A, I // 16), float("nan"), dtype=torch.float32, device="cuda") if sums else None
    plan = kx().verify_plan()
    ids, coef, h, rerr, eerr = kx().verify_gate_up(util.bf16_dev(x), Ld, Wgu, E, k, Ew=Ew, shared_logit=sl,
                                                   shared_id=E, h_sums=hs, plan=plan)
    y, _ = kx().verify_down(h, Wdn, ids, coef, Ew, expert_err=eerr, h_sums=hs)
    # the same down taking gate_up's plan instead of rebuilding the routing from ids / coef: the same bits
    eerr_p = torch.zeros(4, dtype=torch.int32, device="cuda")
    y_p, _ = kx().verify_down(h, Wdn, ids, coef, Ew, expert_err=eerr_p, h_sums=hs, plan=plan)
    sync()
    assert torch.equal(y.view(torch.int16), y_p.view(torch.int16)), "down with the plan differs"
    assert torch.equal(eerr[:3], eerr_p[:3]), "down with the plan reports other errors"
    hb = util.host_bits(h)
    if sums:
        hf = util.as_f32(hb).reshape(M * A, I // 16, 16).astype(np.float64)
        ref = hf.sum(-1)
        got = hs.cpu().numpy().astype(np.float64)
        ok = ~np.isnan(ref).any(-1)  # the valid slots (NaN h rows: invalid, their sums unwritten)
        bound = 1e-6 * np.abs(hf).sum(-1)
        assert (np.abs(got[ok] - ref[ok]) <= bound[ok]).all(), "h_sums differ from the sums of h"
    return (ids.cpu().numpy(), coef.cpu().numpy(), hb, util.host_bits(y),
            rerr.cpu().numpy()[:3].view(np.uint32), eerr.cpu().numpy()[:3].view(np.uint32))


@pytest.mark.parametrize("sums", [True, False])
@pytest.mark.parametrize("M,E,k,d,shared", [(6, 64, 10, 512, False), (1, 16, 4, 1024, False), (16, 40, 3, 512, True),
                                            (5, 300, 8, 2048, True), (4, 1000, 16, 512, False)])
def test_verify_ffn_matches_oracle(M, E, k, d, shared, sums):
    I = 1024
    Ew = E + (1 if shared else 0)
    wgu, wdn, rng = make(M * 7 + E, Ew, I, d)
    x = util.f32_to_bf16(rng.standard_normal((M, d)).astype(np.float32))
    L = (rng.standard_normal((M, Ew)) * 1.3).astype(np.float32)
    if E >= 8:
        L[0, [2, 5]] = 4.0  # a tie: lower index first
    ids, coef, h, y, rerr, eerr = run_fused(x, L, wgu, wdn, E, k, shared, sums)
    if shared:
        r_ids, r_coef, r_err = orc.moe_router(L, E, k, shared=L[:, E].copy(), shared_ld=1, shared_id=E)
    else:
        r_ids, r_coef, r_err = orc.moe_router(L, E, k)
    assert np.array_equal(ids, r_ids)
    util.assert_close(coef, r_coef, tol=1e-6, what="coef")
    ref_h, _ = orc.experts_gather(x, wgu, Ew, r_ids, swiglu=True)
    util.assert_close(h, ref_h, what="h", roundings=4)
    ref_y, _ = orc.experts_combine(h, wdn, Ew, r_ids, r_coef)
    util.assert_close(y, ref_y, what="y")
    assert rerr[0] == 0 and eerr[0] == 0


def test_verify_ffn_nonfinite_logit_matches_per_slot_path():
    """A NaN logit fails its token in the router (ids -1, coef NaN, router error); the experts then see bad ids:
    NaN h rows for those slots, a NaN y row for the token and the expert error of its first slot - the same words and
    values as moe_router followed by this library's per-slot gather_swiglu / combine."""
    import torch
    M, E, k, d, I = 6, 64, 8, 512, 1024
    wgu, wdn, rng = make(3, E, I, d)
    x = util.f32_to_bf16(rng.standard_normal((M, d)).astype(np.float32))
    L = rng.standard_normal((M, E)).astype(np.float32)
    L[3, 17] = np.nan
    ids, coef, h, y, rerr, eerr = run_fused(x, L, wgu, wdn, E, k, False)
    r_ids, r_coef, r_err = orc.moe_router(L, E, k)
    assert np.array_equal(ids, r_ids) and (ids[3] == -1).all()
    assert list(rerr) == list(r_err) == [1, 3, 17]
    Wgu, Wdn = kx().QWeight.upload(wgu), kx().QWeight.upload(wdn)
    ids_d = torch.from_numpy(r_ids).cuda()
    hs, e1 = kx().experts_gather(util.bf16_dev(x), Wgu, E, ids_d, swiglu=True)
    ys, e2 = kx().experts_combine(hs, Wdn, E, ids_d, util.f32_dev(r_coef))
    sync()
    # the fused path reports the first bad slot; the per-slot kernel one of them (its blocks race for the flag)
    assert list(eerr) == [1, 0xFFFFFFFF, 3 * k]
    e1 = e1.cpu().numpy()[:3].view(np.uint32)
    assert e1[0] == 1 and e1[1] == 0xFFFFFFFF and 3 * k <= e1[2] < 4 * k
    hf, hsf = util.as_f32(h), util.as_f32(util.host_bits(hs))
    assert np.isnan(hf[3]).all() and np.isnan(hsf[3]).all()
    ok = [m for m in range(M) if m != 3]
    util.assert_close(h[ok], util.host_bits(hs)[ok], what="h of the healthy tokens")
    yf, ysf = util.as_f32(y), util.as_f32(util.host_bits(ys))
    assert np.isnan(yf[3]).all() and np.isnan(ysf[3]).all()
    util.assert_close(y[ok], util.host_bits(ys)[ok], what="y of the healthy tokens")


def test_verify_down_bad_and_repeated_ids():
    """verify_down alone: an id outside [0, Ew) and an id repeated within a token make their tokens' rows NaN and
    report the first such slot; the other tokens match the oracle's combine."""
    import torch
    M, A, Ew, d, I = 5, 6, 24, 512, 1024
    _, wdn, rng = make(5, Ew, I, d)
    h = util.f32_to_bf16(rng.standard_normal((M, A, I)).astype(np.float32))
    ids = np.stack([rng.choice(Ew, A, replace=False) for _ in range(M)]).astype(np.int32)
    coef = rng.random((M, A)).astype(np.float32)
    ids[1, 4] = Ew + 3  # out of range: slot 10
    ids[3, 2] = ids[3, 0]  # repeated within token 3: slot 20
    Wdn = kx().QWeight.upload(wdn)
    y, err = kx().verify_down(util.bf16_dev(h), Wdn, torch.from_numpy(ids).cuda(), util.f32_dev(coef), Ew)
    sync()
    yh = util.host_bits(y)
    assert list(err.cpu().numpy()[:3].view(np.uint32)) == [1, Ew + 3, 1 * A + 4]
    assert np.isnan(util.as_f32(yh[1])).all() and np.isnan(util.as_f32(yh[3])).all()
    ok = [0, 2, 4]
    ref_y, _ = orc.experts_combine(h[ok], wdn, Ew, ids[ok], coef[ok])
    util.assert_close(yh[ok], ref_y, what="y")


def test_verify_supported_limits():
    from strixite_amd import synthetic as syn
    gu = syn.qweight(4, 8 * 2 * 1024, 4096, 128, seed=1)
    dn = syn.qweight(4, 8 * 4096, 1024, 128, seed=2)
    assert kx().verify_supported(6, 10, 8, 10, 8, gu, dn) is False  # k > E
    assert kx().verify_supported(6, 8, 8, 8, 8, gu, dn) is True
    assert kx().verify_supported(16, 4, 8, 4, 8, gu, dn) is True
    assert kx().verify_supported(17, 1, 8, 1, 8, gu, dn) is False  # M > 16
    assert kx().verify_supported(9, 8, 8, 8, 8, gu, dn) is False   # M * A > 64
    assert kx().verify_supported(1, 4, 1100, 4, 8, gu, dn) is False  # E > 1024 logits: those past 1024 go unread
    assert kx().verify_supported(1, 32, 40, 32, 8, gu, dn) is True
    assert kx().verify_supported(1, 33, 40, 33, 8, gu, dn) is False  # k > 32
    import strixite_amd as sx
    import torch
    x = torch.zeros((2, 4096), dtype=torch.bfloat16, device="cuda")
    logits = torch.zeros((2, 9), dtype=torch.float32, device="cuda")
    with pytest.raises(sx.SxError, match="shared_id"):  # a shared slot needs a valid expert row block
        kx().verify_gate_up(x, logits, gu, 8, 4, shared_logit=logits[:, 8:], shared_id=-1)


@pytest.mark.parametrize("M,E,k,shared", [(6, 512, 10, False), (5, 64, 8, True), (1, 8, 1, False)])
def test_verify_gate_up_pool_matches_static_split(M, E, k, shared):
    """gate_up with a sync buffer (fixed runs, then the shared pool; K = 4096) gives the same ids, coef, h and
    h_sums, bit for bit, as the fixed split, over launches back to back on one buffer (both counter sets in turn);
    (1, 8, 1): fewer tiles than compute units, so no fixed run and most blocks get no round."""
    import torch
    from strixite_amd import synthetic as syn
    d, I = 4096, 1024
    Ew = E + (1 if shared else 0)
    gu = syn.qweight(4, Ew * 2 * I, d, 128, seed=81)
    sy = kx().verify_layer_sync()
    A = k + (1 if shared else 0)
    for r in range(5):
        print(f"pool: M={M} E={E} k={k} shared={shared} launch {r}", flush=True)
        x = syn.activations(M, d, seed=90 + r)
        L = torch.randn((M, Ew), device="cuda") * 1.5
        sl = L[:, E:] if shared else None
        outs = []
        for s in (None, sy):
            hs = torch.full((M * A, I // 16), float("nan"), dtype=torch.float32, device="cuda")
            ids, coef, h, rerr, eerr = kx().verify_gate_up(x, L, gu, E, k, Ew=Ew, shared_logit=sl, shared_id=E,
                                                           h_sums=hs, sync=s)
            sync()
            assert list(rerr.cpu().numpy()[:3]) == [0, 0, 0] and list(eerr.cpu().numpy()[:3]) == [0, 0, 0]
            outs.append((ids.cpu().numpy(), coef.cpu().numpy(), util.host_bits(h), hs.cpu().numpy()))
        for a, b, name in zip(outs[0], outs[1], ("ids", "coef", "h", "h_sums")):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"{name} differs with the pool"


def test_verify_gate_up_pool_survives_other_shapes_on_one_buffer():
    """Launches that do not use the pool (K = 1024 gate_up with the same sync buffer) between K = 4096 launches that
    do: the pool launches keep alternating counter sets, so each gives the static split's bits."""
    import torch
    from strixite_amd import synthetic as syn
    M, E, k, I = 6, 64, 8, 512
    sy = kx().verify_layer_sync()
    g4 = syn.qweight(4, E * 2 * I, 4096, 128, seed=83)
    g1 = syn.qweight(4, E * 2 * I, 1024, 128, seed=84)
    for r, K in enumerate((4096, 1024, 4096, 1024, 1024, 4096, 4096, 1024, 4096)):
        print(f"alternate: launch {r} K={K}", flush=True)
        gu = g4 if K == 4096 else g1
        x = syn.activations(M, K, seed=200 + r)
        L = torch.randn((M, E), device="cuda") * 1.5
        outs = []
        for s in (None, sy):
            ids, coef, h, rerr, eerr = kx().verify_gate_up(x, L, gu, E, k, Ew=E, sync=s)
            sync()
            assert list(eerr.cpu().numpy()[:3]) == [0, 0, 0]
            outs.append((ids.cpu().numpy(), util.host_bits(h)))
        assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1]), f"launch {r}"
