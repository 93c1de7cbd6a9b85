"""Parity of the verify tail on cuda:0 through the C ABI: logits top-k (kernels/logits_topk.hpp), the MTP draft pick
(kernels/mtp_pick.hpp) and device acceptance (serve/engine.cpp:592-610 with serve/sampler.cpp's draw), against the
CPU oracle and the fixtures written from the compiled reference sampler."""
import os

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


def topk_gpu(L, n_valid, k, mask=None):
    import torch
    v, i, nan, raw = kx().logits_topk(util.f32_dev(L), n_valid, k,
                                      mask=None if mask is None else torch.from_numpy(mask.view(np.int32)).cuda())
    sync()
    return v.cpu().numpy(), i.cpu().numpy(), nan.cpu().numpy(), raw


@pytest.mark.parametrize("n,k", [(151936, 40), (151936, 20), (8192, 64), (300, 20), (7, 20), (1, 1), (40000, 33)])
def test_logits_topk_bit_exact(n, k):
    rng = np.random.default_rng(n + k)
    L = rng.standard_normal((6, n)).astype(np.float32)
    if n >= 300:
        L[1, 100:260] = 7.0                    # heavy ties at the top: the lowest ids
        L[2, n // 2] = np.nan                  # flagged, left out
        L[3, :] = -0.0
        L[3, n - 1] = 0.0                       # -0 ties +0 (value kept as stored)
        L[4, :] = np.round(L[4] * 4) / 4       # many ties throughout
    v, i, nan, _ = topk_gpu(L, n, k)
    rv, ri, rnan = orc.logits_topk(L, n, k)
    assert np.array_equal(i, ri)
    assert np.array_equal(v.view(np.uint32), rv.view(np.uint32))
    assert np.array_equal(nan, rnan)


def test_logits_topk_three_levels_and_ld():
    rng = np.random.default_rng(5)
    n = 3 * 1024 * 1024 + 17
    L = np.full((2, n + 5), np.inf, np.float32)  # padding past n_valid must never be read as a candidate
    L[:, :n] = rng.standard_normal((2, n)).astype(np.float32)
    v, i, nan, _ = topk_gpu(L, n, 40)
    rv, ri, rnan = orc.logits_topk(L, n, 40)
    assert np.array_equal(i, ri) and np.array_equal(nan, rnan)


def test_logits_topk_mask():
    rng = np.random.default_rng(6)
    n = 20000
    L = rng.standard_normal((3, n)).astype(np.float32)
    allowed = rng.random((3, n)) < 0.001
    allowed[2] = False
    allowed[2, [5, 9000]] = True          # fewer allowed than k: padding
    L[1, 3] = np.nan                       # flagged although masked out
    words = (n + 31) // 32
    mask = np.zeros((3, words), np.uint32)
    for r in range(3):
        for j in np.nonzero(allowed[r])[0]:
            mask[r, j >> 5] |= np.uint32(1 << (j & 31))
    v, i, nan, _ = topk_gpu(L, n, 20, mask)
    rv, ri, rnan = orc.logits_topk(L, n, 20, mask=mask)
    assert np.array_equal(i, ri) and np.array_equal(nan, rnan)
    assert list(i[2, :2]) == [9000, 5] or list(i[2, :2]) == [5, 9000]
    assert np.all(i[2, 2:] == np.iinfo(np.int32).max)


@pytest.mark.parametrize("n", [1, 2, 63, 1000, 65536, 248320])
def test_mtp_pick(n):
    import torch
    rng = np.random.default_rng(n)
    cases = [rng.standard_normal(n).astype(np.float32)]
    if n >= 63:
        t = cases[0].copy()
        t[[10, n - 3]] = 50.0               # tie at the top: lower id, second == best
        cases.append(t)
        t = cases[0].copy()
        t[7] = np.nan                       # flagged
        cases.append(t)
    cases.append(np.full(n, np.nan, np.float32))  # all NaN: best 0, flagged
    errs = [torch.tensor([i, 2 * i, 3 * i], dtype=torch.int32, device="cuda") for i in (1, 4, 7)]
    emb = torch.tensor([0x1234_5678_9ABC], dtype=torch.int64, device="cuda")
    ws = torch.zeros(kx().mtp_pick_ws_bytes(n), dtype=torch.uint8, device="cuda")  # shared by every call below
    for x in cases:
        xd = util.f32_dev(x)
        out = kx().mtp_pick(xd, *errs, emb)
        out_ws = kx().mtp_pick(xd, *errs, emb, ws=ws)
        # unaligned / non-multiple-of-4 rows take the scalar loads
        out_odd = kx().mtp_pick(xd[1:], *errs, emb, ws=ws) if n > 1 else None
        sync()
        assert bytes(out_ws.cpu().numpy()) == bytes(out.cpu().numpy()), "many-block pick differs"
        if out_odd is not None:
            p1 = kx().pick_from_bytes(out_odd)
            b1, bv1, sv1, nan1 = orc.top2(x[1:])
            assert (p1.best, p1.nan) == (b1, nan1)
            if not nan1:
                assert np.float32(p1.best_v) == np.float32(bv1) and np.float32(p1.second_v) == np.float32(sv1)
        p = kx().pick_from_bytes(out)
        b, bv, sv, nan = orc.top2(x)
        assert (p.best, p.nan) == (b, nan)
        if not nan:
            assert np.float32(p.best_v) == np.float32(bv) and np.float32(p.second_v) == np.float32(sv)
        assert list(p.err) == [1, 2, 3, 4, 8, 12, 7, 14, 21] and p.emb == 0x1234_5678_9ABC


def accept_gpu(X, drafts, seed, T, top_k, top_p, kc=40):
    """logits rows -> GPU top-kc -> GPU acceptance, the uniforms drawn on the host from the engine's mt19937_64."""
    import torch
    k = len(drafts)
    n = X.shape[1]
    _, _, nan, raw = topk_gpu(X, n, kc)
    rng = orc.Rng(seed)
    u = np.array([rng.canonical() for _ in range(k + 1)], np.float64)
    out = kx().mtp_accept(raw, torch.from_numpy(nan).cuda(), torch.from_numpy(np.asarray(drafts, np.int32)).cuda(),
                          torch.from_numpy(u).cuda(), T, top_k, top_p, n)
    sync()
    o = out.cpu().numpy()
    return int(o[0]), int(o[1]), o[2:]


def test_accept_matches_reference_fixture(golden_dir):
    f = np.load(os.path.join(golden_dir, "accept.npz"))
    for (T, k, p, seed), X, d, j, toks in zip(f["params"], f["x"], f["drafts"], f["j"], f["tokens"]):
        gj, st, gt = accept_gpu(X, d, int(seed), T, int(k), p)
        assert st == 0 and gj == j, (T, seed)
        assert np.array_equal(gt[:j + 1], toks[:j + 1])


@pytest.mark.parametrize("T,top_k,top_p", [(0.7, 40, 0.95), (0.0, 40, 0.95), (1.0, 20, 1.0), (0.3, 5, 0.5)])
def test_accept_random_against_oracle(T, top_k, top_p):
    rng = np.random.default_rng(int(T * 10) + top_k)
    for trial in range(12):
        X = (rng.standard_normal((6, 3000)) * 3).astype(np.float32)
        seed = 100 + trial
        r = orc.Rng(seed)
        seq = [orc.sample_row(r, X[j], 3000, T, top_k, top_p) for j in range(6)]
        target = trial % 6
        drafts = np.array(seq[:5], np.int32)
        if target < 5:
            drafts[target] = (seq[target] + 1) % 3000
        oj, ot, ost = orc.accept(orc.Rng(seed), X, drafts, 3000, T, top_k, top_p)
        gj, st, gt = accept_gpu(X, drafts, seed, T, top_k, top_p)
        assert (gj, st) == (oj, ost) == (target, 0)
        assert np.array_equal(gt[:gj + 1], ot[:oj + 1])


def test_accept_nan_row_status():
    X = np.random.default_rng(1).standard_normal((3, 500)).astype(np.float32)
    X[1, 42] = np.nan
    r = orc.Rng(3)
    first = orc.sample_row(r, X[0], 500, 0.7, 40, 0.95)
    gj, st, gt = accept_gpu(X, [first, 5], 3, 0.7, 40, 0.95)
    assert (gj, st) == (1, 2) and gt[0] == first


def test_config5_verify_tail_full_size():
    """h bf16 [6 x 4096] -> q8 LM head [151936 x 4096] -> logits (1e-3) -> top-40 (bit-exact on the GPU's logits) ->
    acceptance of 5 drafts for every accepted length 0..5, greedy and sampled (T 0.7, top-p 0.95)."""
    import torch
    from strixite_amd import synthetic as syn
    from strixite_amd.verify import VerifyTail
    V, d = 151936, 4096
    w = syn.qweight(8, V, d, 64, seed=21)
    h = syn.activations(6, d, seed=22)
    tail = VerifyTail(w, V, 40, 6)
    hq = orc.QWeight(8, *syn.host_rows(w, 0, V), V, d, 64)
    for mode, (T, tk, tp) in (("greedy", (0.0, 40, 0.95)), ("sampled", (0.7, 40, 0.95))):
        for target in range(6):
            seed = 500 + target
            drafts = torch.zeros(5, dtype=torch.int32, device="cuda")
            u = torch.zeros(6, dtype=torch.float64, device="cuda")
            tail.forward(h, drafts, u, T, tk, tp)  # logits first; drafts are built from them below
            sync()
            L = tail.logits[:6].cpu().numpy()
            if mode == "greedy" and target == 0:
                util.assert_close(L, orc.linear_q(util.host_bits(h), hq, out_act=orc.F32), what="lm head logits")
                rv, ri, _ = orc.logits_topk(L, V, 40)
                assert np.array_equal(tail.cands[:6, :, 1].cpu().numpy(), ri)
            r = orc.Rng(seed)
            seq = [orc.sample_row(r, L[j], V, T, tk, tp) for j in range(6)]
            dr = np.array(seq[:5], np.int32)
            if target < 5:
                dr[target] = (seq[target] + 7) % V
            rr = orc.Rng(seed)
            uu = np.array([rr.canonical() for _ in range(6)], np.float64)
            out = tail.forward(h, torch.from_numpy(dr).cuda(), torch.from_numpy(uu).cuda(), T, tk, tp)
            sync()
            o = out.cpu().numpy()
            assert (int(o[0]), int(o[1])) == (target, 0), (mode, target)
            assert list(o[2:2 + target + 1]) == seq[:target + 1]


def _two_launch_and_fused(L, n_valid, kc, drafts, u, T, top_k, top_p, ws, mask=None):
    """(cands, nan, out) of logits_topk + mtp_accept and of the one-launch verify_tail on the same device logits."""
    import torch
    Ld = util.f32_dev(L)
    md = None if mask is None else torch.from_numpy(mask.view(np.int32)).cuda()
    dd = None if drafts is None else torch.from_numpy(np.asarray(drafts, np.int32)).cuda()
    ud = None if u is None else torch.from_numpy(np.asarray(u, np.float64)).cuda()
    _, _, nan2, c2 = kx().logits_topk(Ld, n_valid, kc, mask=md)
    o2 = None
    if dd is not None:
        o2 = kx().mtp_accept(c2, nan2, dd, ud, T, top_k, top_p, n_valid)
    c1, nan1, o1 = kx().verify_tail(Ld, n_valid, kc, ws, drafts=dd, u=ud, temperature=T, top_k=top_k, top_p=top_p,
                                    mask=md)
    sync()
    res2 = (c2.cpu().numpy(), nan2.cpu().numpy(), None if o2 is None else o2.cpu().numpy())
    res1 = (c1.cpu().numpy(), nan1.cpu().numpy(), None if o1 is None else o1.cpu().numpy())
    return res2, res1


@pytest.mark.parametrize("n,kc", [(151936, 40), (248320, 20), (4097, 40), (300, 20), (1, 20), (40000, 64)])
def test_verify_tail_one_launch_matches_two(n, kc):
    """sx_verify_tail (top-k and acceptance in one launch) gives the candidates, NaN flags and accepted tokens of
    sx_logits_topk + sx_mtp_accept, bit for bit: ties, -0 / +0, a NaN row, greedy and sampled, launches back to back
    on one workspace (its counters must come back to zero)."""
    rng = np.random.default_rng(n + kc)
    rows = 6
    ws = kx().verify_tail_workspace(rows, n, kc)
    for trial in range(4):
        print(f"verify tail: n={n} kc={kc} trial {trial}", flush=True)
        L = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
        if n > 10:
            L[0, 5] = L[0, 9] = L[0].max() + 1  # a tie at the top
            L[2, 3], L[2, 4] = 0.0, -0.0
            L[2, :3] = -1e30
        if trial == 2 and n > 50:
            L[3, 17] = np.nan
        T, top_k, top_p = ((0.0, kc, 0.95), (0.7, min(40, kc), 0.95), (1.0, min(20, kc), 1.0), (0.3, 5, 0.5))[trial]
        ref = L.argmax(1) if T == 0 else np.zeros(rows, np.int64)
        drafts = [int(ref[j]) for j in range(5)] if T == 0 else list(rng.integers(0, n, 5))
        u = rng.random(rows)
        (c2, n2, o2), (c1, n1, o1) = _two_launch_and_fused(L, n, kc, drafts, u, T, top_k, top_p, ws)
        assert np.array_equal(c1, c2), "candidates differ"
        assert np.array_equal(n1, n2), "NaN flags differ"
        j = int(o2[0])
        assert (int(o1[0]), int(o1[1])) == (j, int(o2[1])), (o1[:2], o2[:2])
        assert np.array_equal(o1[2:2 + j + 1], o2[2:2 + j + 1])
    # top-k only (no drafts), with an allow-mask
    bits = (rng.random((rows, (n + 31) // 32, 32)) < 0.3).astype(np.uint64)
    words = (bits << np.arange(32, dtype=np.uint64)).sum(-1).astype(np.uint32)
    L = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    (c2, n2, _), (c1, n1, _) = _two_launch_and_fused(L, n, kc, None, None, 0.0, 1, 1.0, ws, mask=words)
    assert np.array_equal(c1, c2) and np.array_equal(n1, n2)
