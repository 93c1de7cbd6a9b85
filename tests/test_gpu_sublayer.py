"""Parity of the served model's MoE sublayer pieces on cuda:0 through the C ABI: the BF16-weight router projection
(kernels/linear.hpp linear_bf16w, kernels/linear_wmma.hpp linear_bf16w_wmma), the shared-expert add and its inject
form (kernels/moe_router.hpp:45-63), and the whole verify sublayer at the config-3 shape with a separate shared expert
(runtime/qwen4exp.cpp:1132-1163: projection -> routing -> experts -> shared expert -> moe_shared_add_inject)."""
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


def dev(a):
    return util.f32_dev(a) if a.dtype == np.float32 else util.bf16_dev(a)


# ---------------- linear_bf16w ----------------

@pytest.mark.parametrize("M,N,K,act,out_act", [
    (6, 513, 4096, orc.BF16, orc.F32),    # the served router at verify width (rows kernel)
    (1, 513, 2560, orc.BF16, orc.F32),    # decode, the real model's d
    (6, 100, 4096, orc.F32, orc.F32),
    (5, 70, 1000, orc.BF16, orc.BF16),    # K % 8 == 0, BF16 out
    (3, 17, 1003, orc.F32, orc.F32),      # K % 8 != 0: the generic kernel
    (256, 513, 4096, orc.BF16, orc.F32),  # prefill width: MFMA, exact products
    (70, 130, 512, orc.F32, orc.F32),     # MFMA with F32 x split into three BF16 terms, partial tiles
    (64, 64, 96, orc.BF16, orc.BF16),
])
def test_linear_bf16w_matches_oracle(M, N, K, act, out_act):
    rng = np.random.default_rng(M * 1000 + N + K)
    W = util.f32_to_bf16((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    x = rng.standard_normal((M, K)).astype(np.float32)
    x = x if act == orc.F32 else util.f32_to_bf16(x)
    print(f"linear_bf16w M={M} N={N} K={K} act={act} out={out_act}", flush=True)
    y = kx().linear_bf16w(dev(x), util.bf16_dev(W).view(__import__("torch").int16), out_act=out_act)
    sync()
    ref = orc.linear_bf16w(x, W, out_act=out_act)
    util.assert_close(util.host_bits(y), ref, what=f"linear_bf16w M={M} N={N} K={K}")


@pytest.mark.parametrize("M,act", [(6, orc.F32), (128, orc.F32), (200, orc.BF16)])
def test_linear_bf16w_wmma_rounds_x_to_bf16(M, act):
    """linear_bf16w_wmma: y = bf16(x) * W^T with FP32 accumulation (kernels/linear_wmma.hpp:25-27): against the oracle
    on x rounded to BF16 first; for F32 x that differs from linear_bf16w on the unrounded x."""
    import torch
    N, K = 96, 1024
    rng = np.random.default_rng(M + 7)
    W = util.f32_to_bf16((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    x = rng.standard_normal((M, K)).astype(np.float32)
    xin = x if act == orc.F32 else util.f32_to_bf16(x)
    y = kx().linear_bf16w(dev(xin), util.bf16_dev(W).view(torch.int16), out_act=orc.F32, wmma=True)
    sync()
    xr = util.f32_to_bf16(x) if act == orc.F32 else xin
    ref = orc.linear_bf16w(xr, W, out_act=orc.F32)
    util.assert_close(y.cpu().numpy(), ref, what="linear_bf16w_wmma")
    if act == orc.F32:  # the rounding of x is visible: the product of the unrounded x differs
        assert not np.array_equal(orc.linear_bf16w(x, W), ref)


def test_linear_bf16w_rejects_overlap_and_bad_dtypes():
    import strixite_amd as sx
    import torch
    x = torch.zeros((4, 64), dtype=torch.bfloat16, device="cuda")
    W = torch.zeros((8, 64), dtype=torch.int16, device="cuda")
    with pytest.raises(sx.SxError, match="overlaps"):
        kx().linear_bf16w(x, W, y=x.view(-1)[:32].view(4, 8))
    with pytest.raises(sx.SxError, match="output dtype"):
        kx().linear_bf16w(x.float(), W, out_act=orc.BF16)
    with pytest.raises(sx.SxError, match="multiple of 64"):
        kx().linear_bf16w(torch.zeros((4, 96), dtype=torch.bfloat16, device="cuda"),
                          torch.zeros((8, 96), dtype=torch.int16, device="cuda"), wmma=True)


# ---------------- moe_shared_add / moe_shared_add_inject ----------------

@pytest.mark.parametrize("act", [orc.F32, orc.BF16])
@pytest.mark.parametrize("inject", [False, True])
def test_shared_add_matches_oracle(act, inject):
    """y += sigmoid(gate) * s (and the four-stream inject of the stored y) against the oracle, with the gate logit in
    the last column of the router's logit rows (stride E + 1), one token's gate NaN and another's +inf: NaN rows,
    error words {1, a bad token, gate_index}."""
    import torch
    M, N, E = 6, 4096, 512
    rng = np.random.default_rng(act * 2 + inject)
    y = rng.standard_normal((M, N)).astype(np.float32)
    s = rng.standard_normal((M, N)).astype(np.float32)
    logits = rng.standard_normal((M, E + 1)).astype(np.float32) * 2
    logits[2, E] = np.nan
    logits[4, E] = np.inf
    if act == orc.BF16:
        y, s = util.f32_to_bf16(y), util.f32_to_bf16(s)
    xh = w_in = None
    if inject:
        xh = rng.standard_normal((M, 4 * N)).astype(np.float32)
        xh = xh if act == orc.F32 else util.f32_to_bf16(xh)
        w_in = rng.standard_normal((M, 4)).astype(np.float32)
    yd, sd, Ld = dev(y), dev(s), util.f32_dev(logits)
    err = torch.zeros(4, dtype=torch.int32, device="cuda")
    xd = None if xh is None else dev(xh)
    kx().moe_shared_add(yd, sd, Ld[:, E:], E, err, x=xd, w_in=None if w_in is None else util.f32_dev(w_in))
    sync()
    ref_y, ref_x, ref_err = orc.moe_shared_add(y, s, logits.ravel()[E:], E + 1, E, x=xh, w_in=w_in)
    # first writer wins: either bad token may be named (the oracle, sequential, names the first)
    e = err.cpu().numpy()[:3]
    assert list(ref_err) == [1, 2, E] and e[0] == 1 and e[1] in (2, 4) and e[2] == E
    util.assert_close(util.host_bits(yd), ref_y, tol=1e-6, what="shared add y")
    if inject:
        util.assert_close(util.host_bits(xd), ref_x, tol=1e-6, what="inject x")
        got = util.as_f32(util.host_bits(xd)).reshape(M, 4, N)
        assert np.isnan(got[2]).all() and not np.isnan(got[0]).any()


# ---------------- the verify sublayer with a separate shared expert (config-3 shape) ----------------

def test_verify_sublayer_with_shared_expert_config3_shape():
    """M = 6, d = 4096, 512 routed experts top-10 + a separate shared expert (I = 1024 everywhere, q4 G = 128), BF16
    router weight [513, 4096] with the shared gate in row 512 (the served model's layout): projection (linear_bf16w,
    F32 logits) -> routing + gate_up + SwiGLU -> down + combine -> shared gate_up (linear_q4) -> SwiGLU -> shared down
    -> moe_shared_add_inject into 4 residual streams. Each stage against the oracle on the GPU's own inputs to it;
    routing bit-exact on the GPU's logits."""
    import torch
    from strixite_amd import synthetic as syn
    E, d, I, k, M, H = 512, 4096, 1024, 10, 6, 4
    rng = np.random.default_rng(33)
    Wr = util.f32_to_bf16((rng.standard_normal((E + 1, d)) * 0.02).astype(np.float32))
    gu = syn.qweight(4, E * 2 * I, d, 128, seed=34)
    dn = syn.qweight(4, E * d, I, 128, seed=35)
    sgu = syn.qweight(4, 2 * I, d, 128, seed=36)
    sdn = syn.qweight(4, d, I, 128, seed=37)
    x = syn.activations(M, d, seed=38)
    streams = syn.activations(M, H * d, seed=39)
    w_in = torch.rand((M, H), device="cuda")
    Wr_d = util.bf16_dev(Wr).view(torch.int16)

    logits = kx().linear_bf16w(x, Wr_d, out_act=orc.F32)
    ids, coef, h, rerr, eerr = kx().verify_gate_up(x, logits, gu, E, k)
    y, eerr2 = kx().verify_down(h, dn, ids, coef, E)
    sh_gu = kx().linear(x, sgu)
    sh_h = kx().swiglu(sh_gu)
    sh_y = kx().linear(sh_h, sdn)
    y_before = y.clone()
    x_out = streams.clone()
    kx().moe_shared_add(y, sh_y, logits[:, E:], E, rerr, x=x_out, w_in=w_in)
    sync()

    xh = util.host_bits(x)
    L = logits.cpu().numpy()
    util.assert_close(L, orc.linear_bf16w(xh, Wr, out_act=orc.F32), what="router logits (BF16 weight)")
    ref_ids, ref_coef, _ = orc.moe_router(L, E, k)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    util.assert_close(coef.cpu().numpy(), ref_coef, tol=1e-6, what="coef")
    assert rerr.cpu().numpy()[0] == 0 and eerr.cpu().numpy()[0] == 0 and eerr2.cpu().numpy()[0] == 0

    touched = np.unique(ref_ids)
    U = len(touched)
    rid = np.searchsorted(touched, ref_ids).astype(np.int32)
    cat = lambda w, rows: [np.concatenate(p) for p in zip(*[syn.host_rows(w, e * rows, (e + 1) * rows) for e in touched])]
    hgu = orc.QWeight(4, *cat(gu, 2 * I), U * 2 * I, d, 128)
    hdn = orc.QWeight(4, *cat(dn, d), U * d, I, 128)
    ref_h, _ = orc.experts_gather(xh, hgu, U, rid, swiglu=True)
    util.assert_close(util.host_bits(h), ref_h, roundings=4, what="routed h")
    ref_y, _ = orc.experts_combine(util.host_bits(h), hdn, U, rid, coef.cpu().numpy())
    util.assert_close(util.host_bits(y_before), ref_y, what="routed y")

    hs = orc.QWeight(4, *syn.host_rows(sgu, 0, 2 * I), 2 * I, d, 128)
    util.assert_close(util.host_bits(sh_gu), orc.linear_q(xh, hs), what="shared gate_up")
    util.assert_close(util.host_bits(sh_h), orc.swiglu(util.host_bits(sh_gu)), tol=1e-6, what="shared swiglu")
    hd = orc.QWeight(4, *syn.host_rows(sdn, 0, d), d, I, 128)
    util.assert_close(util.host_bits(sh_y), orc.linear_q(util.host_bits(sh_h), hd), what="shared down")
    ref_y2, ref_x2, ref_err = orc.moe_shared_add(util.host_bits(y_before), util.host_bits(sh_y), L.ravel()[E:], E + 1,
                                                 E, x=util.host_bits(streams), w_in=w_in.cpu().numpy())
    assert list(ref_err) == [0, 0, 0] and rerr.cpu().numpy()[0] == 0
    util.assert_close(util.host_bits(y), ref_y2, tol=1e-6, what="y + shared")
    util.assert_close(util.host_bits(x_out), ref_x2, tol=1e-6, what="streams after inject")
