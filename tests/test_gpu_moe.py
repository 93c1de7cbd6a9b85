"""Parity of the MoE path on cuda:0 through the C ABI: router (kernels/moe_router.hpp), route grouping
(kernels/moe_grouped.hpp:42-49), per-slot experts (kernels/linear_q4.hpp:32-58), grouped experts
(kernels/moe_grouped.hpp:51-62), SwiGLU, and the full BASELINE config-3 layer against the CPU oracle."""
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


# ---------------- router ----------------

@pytest.mark.parametrize("E,k", [(512, 10), (64, 32), (1000, 8), (1, 1), (130, 7)])
def test_router_ids_bit_exact(E, k):
    rng = np.random.default_rng(E + k)
    L = rng.standard_normal((9, E)).astype(np.float32)
    if E >= 8:
        L[2, [3, E - 1, E // 2]] = 9.0       # a three-way tie at the top: lowest index first
        L[4, :] = 0.5                         # everything tied
        L[5, :] = -0.0
        L[5, E - 1] = 0.0                     # -0 ties +0
        L[6, :] = rng.integers(0, 40, E)      # ties straddling the k-th value (a few dozen candidates)
        L[7, :] = np.round(L[7] * 2) / 2      # coarse levels
    ids, coef, err = kx().moe_router(util.f32_dev(L), E, k)
    sync()
    ref_ids, ref_coef, ref_err = orc.moe_router(L, E, k)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    util.assert_close(coef.cpu().numpy(), ref_coef, tol=1e-6, what="coef")
    assert err.cpu().numpy()[0] == 0


def test_router_bf16_logits_shared_slot_and_errors():
    import torch
    rng = np.random.default_rng(7)
    L = rng.standard_normal((4, 513)).astype(np.float32)
    L[1, 77] = np.nan
    Lb = util.f32_to_bf16(L)
    ld = 513
    shared = util.bf16_dev(Lb)[:, 512:]  # the shared gate in the row's last column, stride ld
    ids, coef, err = kx().moe_router(util.bf16_dev(Lb), 512, 10, shared=shared, shared_ld=ld, shared_id=512)
    sync()
    ref_ids, ref_coef, ref_err = orc.moe_router(util.bf16_to_f32(Lb), 512, 10, shared=util.bf16_to_f32(Lb[:, 512].copy()),
                                                shared_ld=1, shared_id=512)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    util.assert_close(coef.cpu().numpy(), ref_coef, tol=1e-6)
    assert list(err.cpu().numpy()[:3]) == [1, 1, 77] == list(ref_err)
    assert torch.isnan(coef[1]).all()


# ---------------- grouping ----------------

@pytest.mark.parametrize("M,A,E", [(300, 10, 40), (2048, 10, 512), (4000, 10, 512)])
def test_group_routes_invariants(M, A, E):
    """Up to 32,768 slots the grouping places them in LDS first and writes them out in order; above, straight into
    the workspace: both give a valid grouping."""
    rng = np.random.default_rng(3)
    ids = rng.integers(0, E, (M, A)).astype(np.int32)
    ids[:, 0] = 7                      # one bucket far over 64 slots
    ids[5, 3], ids[9, 1] = -1, E + 3   # invalid ids: bucket E, first one (slot 53) reported
    import torch
    ws, err = kx().group_routes(torch.from_numpy(ids).cuda(), E)
    sync()
    w = ws.cpu().numpy()
    S = M * A
    Tmax, WTmax = S // 16 + E + 2, S // 64 + E + 2
    off = w[4:4 + E + 2]
    slots = w[4 + E + 2:4 + E + 2 + S]
    tb = w[4 + E + 2 + S:][:Tmax]
    ts = w[4 + E + 2 + S + Tmax:][:Tmax]
    wb = w[4 + E + 2 + S + 2 * Tmax:][:WTmax]
    wst = w[4 + E + 2 + S + 2 * Tmax + WTmax:][:WTmax]
    flat = ids.ravel()
    bucket = np.where((flat >= 0) & (flat < E), flat, E)
    counts = np.bincount(bucket, minlength=E + 1)
    assert np.array_equal(off, np.concatenate([[0], np.cumsum(counts)]))
    assert sorted(slots.tolist()) == list(range(S))
    for b in range(E + 1):
        assert np.all(bucket[slots[off[b]:off[b + 1]]] == b)
    for R, n, tbk, tst in ((16, w[0], tb, ts), (64, w[3], wb, wst)):
        assert n == sum((c + R - 1) // R for c in counts)
        for b in range(E + 1):
            starts = tst[:n][tbk[:n] == b]
            assert list(starts) == list(range(off[b], off[b + 1], R))
    assert list(w[1:3]) == [S, E]
    assert list(err.cpu().numpy()[:3]) == [1, -1, 53]


def _ws_parts(w, S, E):
    """The defined parts of a route workspace (tile arrays past n_tiles / n_wtiles are never written)."""
    Tmax, WTmax = S // 16 + E + 2, S // 64 + E + 2
    o = 4 + E + 2
    t = o + S
    n, nw = w[0], w[3]
    tiles = np.concatenate([w[t:t + n], w[t + Tmax:t + Tmax + n], w[t + 2 * Tmax:t + 2 * Tmax + nw],
                            w[t + 2 * Tmax + WTmax:t + 2 * Tmax + WTmax + nw]])
    return {"head": w[:4], "off": w[4:o], "slots": w[o:o + S], "tiles": tiles}


@pytest.mark.parametrize("M,E,k,act", [(6, 512, 10, orc.F32), (1, 512, 10, orc.F32), (17, 64, 32, orc.BF16),
                                       (64, 1000, 8, orc.F32), (33, 130, 7, orc.BF16)])
def test_router_group_matches_two_calls(M, E, k, act):
    """One launch == moe_router + moe_group_routes: ids and coefficients bit for bit, the workspace's header, offsets
    and tiles equal, each bucket's slots the same set, and ids exact against the oracle; a non-finite row fails its
    token in both."""
    import torch
    rng = np.random.default_rng(M * 7 + E)
    L = rng.standard_normal((M, E)).astype(np.float32)
    L[0, [1, E // 2]] = 5.0  # a tie: lower index first
    if M > 3:
        L[3, E - 1] = np.nan
    Ld = util.f32_dev(L) if act == orc.F32 else util.bf16_dev(util.f32_to_bf16(L))
    ids2, coef2, rerr2 = kx().moe_router(Ld, E, k)
    ws2, eerr2 = kx().group_routes(ids2, E)
    ids, coef, ws, rerr, eerr = kx().router_group(Ld, E, k)
    sync()
    assert np.array_equal(ids.cpu().numpy(), ids2.cpu().numpy())
    assert np.array_equal(coef.cpu().numpy().view(np.uint32), coef2.cpu().numpy().view(np.uint32))
    assert np.array_equal(rerr.cpu().numpy(), rerr2.cpu().numpy())
    assert np.array_equal(eerr.cpu().numpy(), eerr2.cpu().numpy())
    a, b = _ws_parts(ws.cpu().numpy(), M * k, E), _ws_parts(ws2.cpu().numpy(), M * k, E)
    for key in ("head", "off", "tiles"):
        assert np.array_equal(a[key], b[key]), key
    off = a["off"]
    for e in range(E + 1):
        assert sorted(a["slots"][off[e]:off[e + 1]]) == sorted(b["slots"][off[e]:off[e + 1]])
    Lh = L if act == orc.F32 else util.bf16_to_f32(util.f32_to_bf16(L))
    ref_ids, _, _ = orc.moe_router(Lh, E, k)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)


@pytest.mark.parametrize("M,N,K", [(256, 512, 4096), (70, 100, 256), (64, 16, 32)])
def test_router_projection_prefill_mfma(M, N, K):
    """Prefill-width router projection (M >= 64, BF16 x: the MFMA path with the FP32 weight as three exact BF16
    terms) against the oracle's FP64 product, partial token and row tiles included; FP32 accuracy."""
    import torch
    rng = np.random.default_rng(M + N)
    x = util.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    y = kx().linear_f32w(util.bf16_dev(x), torch.from_numpy(W).cuda())
    sync()
    ref = orc.linear_f32w(x, W)
    got = y.cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


# ---------------- experts ----------------

def make_experts(seed, E, I, d, G=128):
    rng = np.random.default_rng(seed)
    return util.rand_qweight(rng, 4, E * 2 * I, d, G), util.rand_qweight(rng, 4, E * d, I, min(G, I)), rng


@pytest.mark.parametrize("act", [orc.BF16, orc.F32])
def test_per_slot_experts(act):
    import torch
    E, I, d, M, A = 12, 64, 256, 4, 3
    wgu, wdn, rng = make_experts(1, E, I, d)
    x = rng.standard_normal((M, d)).astype(np.float32)
    ids = np.stack([rng.choice(E, A, replace=False) for _ in range(M)]).astype(np.int32)
    coef = rng.random((M, A)).astype(np.float32)
    xh = x if act == orc.F32 else util.f32_to_bf16(x)
    dev = util.f32_dev(xh) if act == orc.F32 else util.bf16_dev(xh)
    ids_d = torch.from_numpy(ids).cuda()
    Wgu, Wdn = kx().QWeight.upload(wgu), kx().QWeight.upload(wdn)
    gu, _ = kx().experts_gather(dev, Wgu, E, ids_d)
    h, err = kx().experts_gather(dev, Wgu, E, ids_d, swiglu=True)
    y, err2 = kx().experts_combine(h, Wdn, E, ids_d, util.f32_dev(coef))
    sync()
    ref_gu, _ = orc.experts_gather(xh, wgu, E, ids)
    ref_h, _ = orc.experts_gather(xh, wgu, E, ids, swiglu=True)
    util.assert_close(util.host_bits(gu), ref_gu, what="gather")
    util.assert_close(util.host_bits(h), ref_h, what="gather_swiglu")
    ref_y, _ = orc.experts_combine(util.host_bits(h), wdn, E, ids, coef)  # the oracle on the GPU's h
    util.assert_close(util.host_bits(y), ref_y, what="combine")
    assert err.cpu().numpy()[0] == 0 and err2.cpu().numpy()[0] == 0


def test_per_slot_bad_id_poisons_and_flags():
    import torch
    E, I, d = 4, 32, 128
    wgu, wdn, rng = make_experts(2, E, I, d)
    x = util.bf16_dev(util.f32_to_bf16(rng.standard_normal((2, d)).astype(np.float32)))
    ids = torch.tensor([[1, 9], [0, 3]], dtype=torch.int32, device="cuda")
    h, err = kx().experts_gather(x, kx().QWeight.upload(wgu), E, ids, swiglu=True)
    y, err2 = kx().experts_combine(h.nan_to_num(), kx().QWeight.upload(wdn), E, ids,
                                   torch.ones((2, 2), device="cuda"))
    sync()
    assert list(err.cpu().numpy()[:3]) == [1, 9, 1] and list(err2.cpu().numpy()[:3]) == [1, 9, 1]
    assert torch.isnan(h[0, 1]).all() and not torch.isnan(h[0, 0]).any() and not torch.isnan(h[1]).any()
    assert torch.isnan(y[0]).all() and not torch.isnan(y[1]).any()


@pytest.mark.parametrize("M,A,E,I,d", [(6, 10, 64, 64, 512), (40, 4, 6, 32, 4096), (3, 2, 5, 128, 256)])
def test_grouped_matches_per_slot_oracle(M, A, E, I, d):
    """Grouped == per-slot semantics (kernels/moe_grouped.hpp:7-11), including buckets larger than the LDS batch."""
    import torch
    wgu, wdn, rng = make_experts(M + E, E, I, d)
    x = util.f32_to_bf16(rng.standard_normal((M, d)).astype(np.float32))
    ids = np.stack([rng.choice(E, A, replace=False) for _ in range(M)]).astype(np.int32)
    coef = rng.random((M, A)).astype(np.float32)
    ids_d = torch.from_numpy(ids).cuda()
    Wgu, Wdn = kx().QWeight.upload(wgu), kx().QWeight.upload(wdn)
    xd = util.bf16_dev(x)
    ws, err = kx().group_routes(ids_d, E)
    gu = kx().gather_grouped(xd, Wgu, E, ws, M, A)
    h = kx().gather_grouped(xd, Wgu, E, ws, M, A, swiglu=True)
    h2 = kx().swiglu(gu.view(M * A, 2 * I)).view(M, A, I)
    y = kx().combine_grouped(h, Wdn, E, ids_d, util.f32_dev(coef), ws)
    sync()
    ref_gu, _ = orc.experts_gather(x, wgu, E, ids)
    ref_h, _ = orc.experts_gather(x, wgu, E, ids, swiglu=True)
    util.assert_close(util.host_bits(gu), ref_gu, what="gather_grouped")
    util.assert_close(util.host_bits(h), ref_h, what="gather_swiglu_grouped")
    assert np.array_equal(util.host_bits(h), util.host_bits(h2))  # fused epilogue == gather then swiglu, bit for bit
    ref_y, _ = orc.experts_combine(util.host_bits(h), wdn, E, ids, coef)
    util.assert_close(util.host_bits(y), ref_y, what="combine_grouped")
    assert err.cpu().numpy()[0] == 0


@pytest.mark.parametrize("M,A,E,I,d", [(96, 4, 8, 512, 512), (40, 3, 5, 512, 2048), (64, 2, 3, 1024, 1024),
                                       (48, 2, 4, 2048, 512)])
def test_prefill_grouped_mfma_matches_oracle(M, A, E, I, d):
    """Prefill width (M >= 32 takes the 64-slot x 128-row MFMA kernel; the combine at I = 512 or 1024 the kernel
    with the tile's activations resident, at I = 2048 the 64-slot one): gather, SwiGLU gather and combine against the
    oracle, with one bucket far over 64 slots (several wide tiles), one of exactly 64, and an invalid id (NaN rows,
    error words from the grouping)."""
    import torch
    wgu, wdn, rng = make_experts(M * 31 + E, E, I, d)
    x = util.f32_to_bf16(rng.standard_normal((M, d)).astype(np.float32))
    ids = np.stack([rng.choice(E, A, replace=False) for _ in range(M)]).astype(np.int32)
    ids[: M // 2, 0] = 1                       # bucket 1: >= M/2 slots
    if M >= 64:
        ids[:, A - 1] = np.where(np.arange(M) < 64, 2, ids[:, A - 1])  # bucket 2 gets 64 more (duplicates allowed)
    ids[5, A - 1] = -1                         # an invalid slot
    coef = rng.random((M, A)).astype(np.float32)
    ids_d = torch.from_numpy(ids).cuda()
    Wgu, Wdn = kx().QWeight.upload(wgu), kx().QWeight.upload(wdn)
    xd = util.bf16_dev(x)
    ws, err = kx().group_routes(ids_d, E)
    gu = kx().gather_grouped(xd, Wgu, E, ws, M, A)
    h = kx().gather_grouped(xd, Wgu, E, ws, M, A, swiglu=True)
    y = kx().combine_grouped(h, Wdn, E, ids_d, util.f32_dev(coef), ws)
    sync()
    ref_gu, _ = orc.experts_gather(x, wgu, E, ids)
    ref_h, _ = orc.experts_gather(x, wgu, E, ids, swiglu=True)
    util.assert_close(util.host_bits(gu), ref_gu, what="prefill gather_grouped")
    util.assert_close(util.host_bits(h), ref_h, what="prefill gather_swiglu_grouped")
    ref_y, _ = orc.experts_combine(util.host_bits(h), wdn, E, ids, coef)
    util.assert_close(util.host_bits(y), ref_y, what="prefill combine_grouped")
    assert list(err.cpu().numpy()[:3]) == [1, -1, 5 * A + A - 1]


def test_grouped_bad_id_rows_are_nan():
    import torch
    M, A, E, I, d = 3, 2, 4, 32, 128
    wgu, wdn, rng = make_experts(9, E, I, d)
    x = util.bf16_dev(util.f32_to_bf16(rng.standard_normal((M, d)).astype(np.float32)))
    ids = torch.tensor([[0, 1], [2, 17], [3, 1]], dtype=torch.int32, device="cuda")
    ws, err = kx().group_routes(ids, E)
    h = kx().gather_grouped(x, kx().QWeight.upload(wgu), E, ws, M, A, swiglu=True)
    y = kx().combine_grouped(h, kx().QWeight.upload(wdn), E, ids, torch.ones((M, A), device="cuda"), ws)
    sync()
    assert list(err.cpu().numpy()[:3]) == [1, 17, 3]
    assert torch.isnan(h[1, 1]).all() and not torch.isnan(h[1, 0]).any()
    assert torch.isnan(y[1]).all() and not torch.isnan(y[0]).any() and not torch.isnan(y[2]).any()


# ---------------- BASELINE config 3 at full size ----------------

def test_config3_moe_verify_layer_full_size():
    """M = 6, d = 4096, E = 512, top-10, I = 1024, q4 G = 128: the whole layer against the oracle. The oracle routes
    the GPU's own router logits (ids bit-exact by construction of the comparison), and recomputes every expert from
    host copies of the touched experts' rows."""
    import torch
    from strixite_amd import synthetic as syn
    from strixite_amd.verify import MoeVerifyLayer
    E, d, I, k, M = 512, 4096, 1024, 10, 6
    Wr = syn.router_weight(E, d, seed=11)
    gu = syn.qweight(4, E * 2 * I, d, 128, seed=12)
    dn = syn.qweight(4, E * d, I, 128, seed=13)
    x = syn.activations(M, d, seed=14)
    layer = MoeVerifyLayer(Wr, gu, dn, E, k, M)
    y = layer.forward(x)
    sync()
    xh = util.host_bits(x)
    logits = layer.logits.cpu().numpy()
    util.assert_close(logits, orc.linear_f32w(xh, Wr.cpu().numpy()), what="router logits")
    ids, coef, err = orc.moe_router(logits, E, k)
    assert np.array_equal(layer.ids.cpu().numpy(), ids)
    util.assert_close(layer.coef.cpu().numpy(), coef, tol=1e-6, what="coef")
    touched = np.unique(ids)
    remap = {e: i for i, e in enumerate(touched)}
    U = len(touched)
    qs, ss, ms, qd, sd, md = [], [], [], [], [], []
    for e in touched:
        q, s, m = syn.host_rows(gu, e * 2 * I, (e + 1) * 2 * I)
        qs.append(q), ss.append(s), ms.append(m)
        q, s, m = syn.host_rows(dn, e * d, (e + 1) * d)
        qd.append(q), sd.append(s), md.append(m)
    hgu = orc.QWeight(4, np.concatenate(qs), np.concatenate(ss), np.concatenate(ms), U * 2 * I, d, 128)
    hdn = orc.QWeight(4, np.concatenate(qd), np.concatenate(sd), np.concatenate(md), U * d, I, 128)
    rid = np.vectorize(remap.get)(ids).astype(np.int32)
    ref_h, _ = orc.experts_gather(xh, hgu, U, rid, swiglu=True)
    util.assert_close(util.host_bits(layer.h), ref_h, what="h")
    ref_y, _ = orc.experts_combine(util.host_bits(layer.h), hdn, U, rid, layer.coef.cpu().numpy())
    util.assert_close(util.host_bits(y), ref_y, what="layer output")
    # the end-to-end view: routing from the oracle's own logits differs only at near-ties
    o_ids, _, _ = orc.moe_router(orc.linear_f32w(xh, Wr.cpu().numpy()), E, k)
    flips = int((np.sort(o_ids, 1) != np.sort(ids, 1)).any(1).sum())
    print(f"config3: U = {U} distinct experts; tokens whose routing flips from CPU logits: {flips}")
    assert flips <= 1


@pytest.mark.parametrize("d", [42, 4096])
def test_combine_grouped_row_counts(d):
    """combine_grouped's reduce over the slot partials: four outputs a thread when the row count allows (d a multiple
    of 4), one otherwise (d = 42), against the oracle's combine, with an invalid id's token NaN."""
    import torch
    M, A, E, I = 37, 3, 6, 128
    rng = np.random.default_rng(d)
    wdn = util.rand_qweight(rng, 4, E * d, I, 128)
    h = util.f32_to_bf16(rng.standard_normal((M, A, I)).astype(np.float32))
    ids = np.stack([rng.choice(E, A, replace=False) for _ in range(M)]).astype(np.int32)
    ids[5, 1] = E + 2
    coef = rng.random((M, A)).astype(np.float32)
    ids_d = torch.from_numpy(ids).cuda()
    ws, err = kx().group_routes(ids_d, E)
    y = kx().combine_grouped(util.bf16_dev(h), kx().QWeight.upload(wdn), E, ids_d, util.f32_dev(coef), ws)
    sync()
    yh = util.host_bits(y)
    assert np.isnan(util.as_f32(yh[5])).all()
    ok = [m for m in range(M) if m != 5]
    ref_y, _ = orc.experts_combine(h[ok], wdn, E, ids[ok], coef[ok])
    util.assert_close(yh[ok], ref_y, what=f"combine_grouped d={d}")
