"""BASELINE config 4 at full size on cuda:0 through the C ABI: the MoE layer at prefill width (M = 2048 tokens,
d = 4096, E = 512, top-10, I = 1024, q4 G = 128, routing skewed by a seeded Zipf(1.1) bias), and the dense linears at
prefill width (the route the reference's linear_q4_wmma / linear_q8_wmma callers take, kernels/linear_wmma.hpp:22-25).

The oracle recomputes the router logits in full, the routing bit-exact on the GPU's logits, the grouping invariants
on all 20,480 slots, h of every token on 128 seeded features and in full for 32 seeded tokens, and y for 256 seeded
tokens (every expert those tokens touch)."""
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


def test_config4_prefill_layer_full_size():
    import torch
    from strixite_amd import synthetic as syn
    E, d, I, k, M = 512, 4096, 1024, 10, 2048
    print("config 4: building inputs", flush=True)
    Wr = syn.router_weight(E, d, seed=61)
    gu = syn.qweight(4, E * 2 * I, d, 128, seed=62)
    dn = syn.qweight(4, E * d, I, 128, seed=63)
    bias = syn.zipf_router_bias(E, seed=64)
    x = syn.activations(M, d, seed=65)

    print("config 4: router projection + Zipf bias + routing + grouping", flush=True)
    logits = kx().linear_f32w(x, Wr)
    raw = logits.clone()
    logits.add_(bias)
    ids, coef, rerr = kx().moe_router(logits, E, k)
    ws, eerr = kx().group_routes(ids, E)
    print("config 4: grouped gate_up + SwiGLU, grouped down + combine", flush=True)
    h = kx().gather_grouped(x, gu, E, ws, M, k, swiglu=True)
    y = kx().combine_grouped(h, dn, E, ids, coef, ws)
    sync()
    # the grouped kernels order their loads and waits by hand: a second run must give the same bits (a wait that
    # lets a load land after its use shows up as run-to-run differences long before it breaks a tolerance)
    print("config 4: the grouped kernels again (run-to-run identical)", flush=True)
    h2 = kx().gather_grouped(x, gu, E, ws, M, k, swiglu=True)
    y2 = kx().combine_grouped(h, dn, E, ids, coef, ws)
    sync()
    assert torch.equal(h.view(torch.int16), h2.view(torch.int16)), "grouped gate_up differs between two runs"
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), "grouped down + combine differs between two runs"
    # a second grouping places the slots of a bucket in another order (the counting sort's atomics): a slot's results
    # must not depend on its place in its tile
    print("config 4: regrouped (slot order within the buckets changes)", flush=True)
    ws3, _ = kx().group_routes(ids, E)
    h3 = kx().gather_grouped(x, gu, E, ws3, M, k, swiglu=True)
    y3 = kx().combine_grouped(h3, dn, E, ids, coef, ws3)
    sync()
    assert torch.equal(h.view(torch.int16), h3.view(torch.int16)), "grouped gate_up depends on the slot order"
    assert torch.equal(y.view(torch.int16), y3.view(torch.int16)), "grouped down + combine depends on the slot order"
    del h2, y2, h3, y3, ws3

    xh = util.host_bits(x)
    util.assert_close(raw.cpu().numpy(), orc.linear_f32w(xh, Wr.cpu().numpy()), tol=1e-5, what="router logits")
    L = logits.cpu().numpy()
    ref_ids, ref_coef, _ = orc.moe_router(L, E, k)
    g_ids = ids.cpu().numpy()
    assert np.array_equal(g_ids, ref_ids), "expert ids differ from the oracle on the same logits"
    util.assert_close(coef.cpu().numpy(), ref_coef, tol=1e-6, what="coef")
    assert rerr.cpu().numpy()[0] == 0 and eerr.cpu().numpy()[0] == 0

    # grouping: the workspace layout of kernels/moe_grouped.hip:63-81 on 20,480 slots
    S = M * k
    w = ws.cpu().numpy()
    Tmax, WTmax = S // 16 + E + 2, S // 64 + E + 2
    off = w[4:4 + E + 2]
    slots = w[4 + E + 2:4 + E + 2 + S]
    counts = np.bincount(g_ids.ravel(), minlength=E + 1)
    assert list(w[1:3]) == [S, E]
    assert np.array_equal(off, np.concatenate([[0], np.cumsum(counts)]))
    assert np.array_equal(np.sort(slots), np.arange(S))
    for b in range(E):
        assert np.all(g_ids.ravel()[slots[off[b]:off[b + 1]]] == b)
    t = 4 + E + 2 + S
    for R, n, tb, ts in ((16, w[0], w[t:t + Tmax], w[t + Tmax:t + 2 * Tmax]),
                         (64, w[3], w[t + 2 * Tmax:t + 2 * Tmax + WTmax], w[t + 2 * Tmax + WTmax:t + 2 * Tmax + 2 * WTmax])):
        assert n == sum((c + R - 1) // R for c in counts)
        for b in np.flatnonzero(counts):
            assert list(ts[:n][tb[:n] == b]) == list(range(off[b], off[b + 1], R))
    print(f"config 4: {int((counts[:E] > 0).sum())} experts used, buckets 0..{int(counts[:E].max())} slots, "
          f"{int((counts[:E] > 64).sum())} over one 64-slot tile", flush=True)
    assert counts[:E].max() > 128  # Zipf: a hot head of experts over two wide tiles

    # h and y for a seeded sample of tokens, against the oracle on the touched experts' rows
    toks = np.sort(np.random.default_rng(66).choice(M, 32, replace=False))
    sub = g_ids[toks]
    touched = np.unique(sub)
    U = len(touched)
    rid = np.searchsorted(touched, sub).astype(np.int32)
    print(f"config 4: checking h and y of {len(toks)} tokens over {U} experts", flush=True)
    cat = lambda wt, rows: [np.concatenate(p) for p in zip(*[syn.host_rows(wt, e * rows, (e + 1) * rows) for e in touched])]
    hgu = orc.QWeight(4, *cat(gu, 2 * I), U * 2 * I, d, 128)
    ref_h, _ = orc.experts_gather(xh[toks], hgu, U, rid, swiglu=True)
    gh = util.host_bits(h)[toks]
    util.assert_close(gh, ref_h, roundings=4, what="config 4 h (sampled tokens)")
    del hgu
    del gh

    # h of every token and slot on 128 seeded features: the gate and up rows of those features of all 512 experts
    J = np.sort(np.random.default_rng(67).choice(I, 128, replace=False))
    rows = (np.arange(E)[:, None] * 2 * I + np.concatenate([J, I + J])[None, :]).ravel()
    print(f"config 4: checking h of all {M} tokens on {len(J)} features", flush=True)
    ridx = torch.from_numpy(rows).cuda()
    qsub = gu.q.view(E * 2 * I, d // 2)[ridx].cpu().numpy().ravel()
    ssub = gu.scale.view(E * 2 * I, d // 128)[ridx].cpu().numpy().view(np.uint16).ravel()
    msub = gu.minv.view(E * 2 * I, d // 128)[ridx].cpu().numpy().view(np.uint16).ravel()
    hsub = orc.QWeight(4, qsub, ssub, msub, len(rows), d, 128)
    ref_hj, _ = orc.experts_gather(xh, hsub, E, g_ids, swiglu=True)
    util.assert_close(util.host_bits(h)[:, :, J], ref_hj, roundings=4, what="config 4 h (all tokens, sampled features)")
    del hsub, qsub, ssub, msub, ref_hj

    # y of 256 seeded tokens from the GPU's h, against the oracle on the down rows of the experts they touch
    ytoks = np.sort(np.random.default_rng(68).choice(M, 256, replace=False))
    ysub = g_ids[ytoks]
    ytouched = np.unique(ysub)
    print(f"config 4: checking y of {len(ytoks)} tokens over {len(ytouched)} experts", flush=True)
    yrid = np.searchsorted(ytouched, ysub).astype(np.int32)
    hdn = orc.QWeight(4, *[np.concatenate(p) for p in zip(*[syn.host_rows(dn, e * d, (e + 1) * d) for e in ytouched])],
                      len(ytouched) * d, I, 128)
    ref_y, _ = orc.experts_combine(util.host_bits(h)[ytoks], hdn, len(ytouched), yrid, coef.cpu().numpy()[ytoks])
    util.assert_close(util.host_bits(y)[ytoks], ref_y, what="config 4 y (sampled tokens)")


@pytest.mark.parametrize("bits,G,act,out_act,M,K", [(4, 128, orc.BF16, orc.BF16, 2048, 4096),
                                                     (4, 128, orc.BF16, orc.F32, 2000, 2048),
                                                     (4, 128, orc.BF16, orc.BF16, 257, 512),
                                                     (8, 64, orc.BF16, orc.F32, 2048, 4096),
                                                     (8, 64, orc.BF16, orc.BF16, 300, 1280),
                                                     (8, 64, orc.BF16, orc.BF16, 256, 4352),
                                                     (8, 64, orc.BF16, orc.F32, 200, 768),
                                                     (4, 128, orc.F32, orc.F32, 2048, 4096),
                                                     (4, 128, orc.BF16, orc.F32, 130, 1024),
                                                     (4, 128, orc.BF16, orc.BF16, 512, 4096),
                                                     (8, 64, orc.BF16, orc.BF16, 100, 2048),
                                                     (8, 64, orc.BF16, orc.F32, 513, 256)])
def test_dense_linear_prefill_width(bits, G, act, out_act, M, K):
    """linear_q4 / linear_q8 at prefill width (the route *_wmma callers take; q4 G = 128 and q8 G = 64 with BF16 x on
    the MFMA tiles: K split over a block's waves up to 512 tokens, whole K a block above; a partial last tile of tokens
    and of rows included; K = 4352 past the tiles' limit on qmm) against the oracle."""
    N = 384
    rng = np.random.default_rng(bits * 10 + act)
    w = util.rand_qweight(rng, bits, N, K, G)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x = x if act == orc.F32 else util.f32_to_bf16(x)
    print(f"dense prefill q{bits} G{G} act={act} out={out_act}", flush=True)
    xd = util.f32_dev(x) if act == orc.F32 else util.bf16_dev(x)
    y = kx().linear(xd, kx().QWeight.upload(w), out_act=out_act)
    sync()
    ref = orc.linear_q(x, w, out_act=out_act)
    util.assert_close(util.host_bits(y), ref, what=f"dense q{bits} M={M}")


def test_f32_x_prefill_keeps_full_precision():
    """The *_wmma entry points of the integration shim forward to linear_q4 / linear_q8, which keep FP32 x exact (three
    BF16 planes) at every width; the reference's wmma contract rounds x to BF16 first (kernels/linear_wmma.hpp:3-6).
    This pins the choice: the result is within FP32 rounding of the exact-x oracle and measurably apart from the
    oracle on BF16-rounded x."""
    M, N, K = 512, 256, 2048
    rng = np.random.default_rng(77)
    w = util.rand_qweight(rng, 4, N, K, 128)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = kx().linear(util.f32_dev(x), kx().QWeight.upload(w), out_act=orc.F32)
    sync()
    got = util.host_bits(y)
    exact = orc.linear_q(x, w, out_act=orc.F32)
    rounded = orc.linear_q(util.bf16_to_f32(util.f32_to_bf16(x)), w, out_act=orc.F32)
    e_exact, e_round = util.max_abs_norm_err(got, exact), util.max_abs_norm_err(got, rounded)
    print(f"F32 x: error vs exact x {e_exact:.3g}, vs BF16-rounded x {e_round:.3g}", flush=True)
    assert e_exact < 1e-5 and e_round > 20 * e_exact


@pytest.mark.parametrize("bits,G", [(4, 128), (8, 64)])
def test_dense_prefill_bench_shape(bits, G):
    """The dense prefill linears at the benchmarked shape (4096 x 4096, M = 2048, BF16 in and out) on the MFMA tiles:
    every output feature of 256 seeded tokens, and every token on 128 seeded output features, against the oracle."""
    import torch
    from strixite_amd import synthetic as syn
    N = K = 4096
    M = 2048
    w = syn.qweight(bits, N, K, G, seed=70 + bits)
    x = syn.activations(M, K, seed=71 + bits)
    print(f"dense prefill q{bits} at 4096 x 4096, M = 2048", flush=True)
    y = kx().linear(x, w)
    sync()
    xh, yh = util.host_bits(x), util.host_bits(y)
    toks = np.sort(np.random.default_rng(72).choice(M, 256, replace=False))
    hw = orc.QWeight(bits, *syn.host_rows(w, 0, N), N, K, G)
    util.assert_close(yh[toks], orc.linear_q(xh[toks], hw), what=f"dense q{bits} (256 tokens, all features)")
    feats = np.sort(np.random.default_rng(73).choice(N, 128, replace=False))
    per, groups = K * bits // 8, K // G
    fw = orc.QWeight(bits, hw.q.reshape(N, per)[feats].ravel(), hw.scale.reshape(N, groups)[feats].ravel(),
                     hw.minv.reshape(N, groups)[feats].ravel(), len(feats), K, G)
    util.assert_close(yh[:, feats], orc.linear_q(xh, fw), what=f"dense q{bits} (all tokens, 128 features)")


@pytest.mark.parametrize("bits,G", [(4, 128), (8, 64)])
def test_staged_stores_match_direct_stores(bits, G):
    """The MFMA tiles store BF16 outputs through LDS as 16-byte vectors when y is 16-byte aligned (and the row count a
    multiple of 8), and one value at a time otherwise: the two store paths write the same bits."""
    import torch
    M, N, K = 300, 384, 1024
    rng = np.random.default_rng(90 + bits)
    w = kx().QWeight.upload(util.rand_qweight(rng, bits, N, K, G))
    xd = util.bf16_dev(util.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32)))
    print(f"staged vs direct stores q{bits}", flush=True)
    y = kx().linear(xd, w)
    buf = torch.empty(M * N + 1, dtype=torch.bfloat16, device="cuda")
    y2 = buf[1:].view(M, N)  # 2 bytes past a 16-byte boundary: the direct path
    kx().linear(xd, w, y=y2)
    sync()
    assert np.array_equal(util.host_bits(y), util.host_bits(y2))


@pytest.mark.parametrize("bits,G,M,N,K,out_act", [(4, 128, 2048, 4096, 1024, orc.BF16), (8, 64, 2048, 4096, 512, orc.BF16),
                                                  (4, 128, 2000, 4104, 1024, orc.BF16), (8, 64, 2000, 4104, 512, orc.F32),
                                                  (4, 128, 2000, 4096, 512, orc.F32), (8, 64, 2048, 4100, 512, orc.BF16)])
def test_wide_tiles_match_64_token_tiles(bits, G, M, N, K, out_act):
    """Where its grid fills the chip (here: all M tokens at once) the dense linear takes 128 tokens a wave; each half
    of the tokens alone takes gg_kernel's 64-token tiles. Both do the same arithmetic for every output: the same bits
    (a partial last token tile, a partial last row block, BF16 staged and BF16 / F32 direct stores included)."""
    import torch
    rng = np.random.default_rng(M + N + K + bits)
    w = kx().QWeight.upload(util.rand_qweight(rng, bits, N, K, G))
    xd = util.bf16_dev(util.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32)))
    print(f"wide vs 64-token tiles q{bits} M={M} N={N} K={K} out={out_act}", flush=True)
    y = kx().linear(xd, w, out_act=out_act)
    h = M // 2
    y0 = kx().linear(xd[:h].contiguous(), w, out_act=out_act)
    y1 = kx().linear(xd[h:].contiguous(), w, out_act=out_act)
    sync()
    assert np.array_equal(util.host_bits(y), np.concatenate([util.host_bits(y0), util.host_bits(y1)]))


@pytest.mark.parametrize("bits,G,M,N,K", [(4, 128, 100, 100, 512), (8, 64, 60, 72, 256), (4, 128, 511, 200, 1536),
                                          (8, 64, 300, 40, 4096)])
def test_dense_k_split_ragged(bits, G, M, N, K):
    """The K-split tiles (up to 512 tokens) on ragged shapes: output rows not a multiple of 64, one K step a wave
    (K = 512 q4, 256 q8), a quarter of K not a multiple of the ring, against the oracle."""
    rng = np.random.default_rng(M + N + K)
    w = util.rand_qweight(rng, bits, N, K, G)
    x = util.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    print(f"dense k-split q{bits} M={M} N={N} K={K}", flush=True)
    y = kx().linear(util.bf16_dev(x), kx().QWeight.upload(w), out_act=orc.F32)
    sync()
    util.assert_close(util.host_bits(y), orc.linear_q(x, w, out_act=orc.F32), what=f"k-split q{bits} M={M} N={N}")
