"""The draft side on cuda:0 through the C ABI: the draft head's Q4 copy of the Q8 LM head (formats/q4_from_q8.hpp,
made on the device) byte-identical to the compiled reference's fixture and to the oracle at the served size, and the
draft head's logits and top-2 pick (runtime/qwen4exp.cpp:1540-1560 + kernels/mtp_pick.hpp) against the oracle."""
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


def upload8(w):
    return kx().QWeight.upload(w)


@pytest.mark.parametrize("tag", ["g64_g64", "g64_g128", "g64_g32", "g128_g64"])
def test_q4_from_q8_device_matches_reference_fixture(golden_dir, tag):
    f = np.load(os.path.join(golden_dir, "q4_from_q8.npz"))
    N, K = (int(v) for v in f["shape"])
    G8, G4 = (int(t[1:]) for t in tag.split("_"))
    w8 = orc.QWeight(8, f[tag + "_q8"], f[tag + "_s8"], f[tag + "_m8"], N, K, G8)
    w4, err = kx().quantize_q4_from_q8(upload8(w8), G4)
    sync()
    assert np.array_equal(w4.q.cpu().numpy(), f[tag + "_q4"])
    assert np.array_equal(w4.scale.cpu().numpy().view(np.uint16), f[tag + "_s4"])
    assert np.array_equal(w4.minv.cpu().numpy().view(np.uint16), f[tag + "_m4"])
    assert err.cpu().numpy()[0] == 0


def test_q4_from_q8_device_served_size():
    """The served draft head: the first 65,536 rows of a Q8 LM head (d = 4096, Q8 G = 64) into Q4 G = 64, byte for
    byte against the oracle."""
    from strixite_amd import synthetic as syn
    V, d, rows = 151936, 4096, 65536
    print("q4_from_q8: 65536 x 4096 rows of a 151936-row Q8 head", flush=True)
    head = syn.qweight(8, V, d, 64, seed=21)
    w4, err = kx().quantize_q4_from_q8(head, 64, rows=rows)
    sync()
    ref = orc.q4_from_q8(orc.QWeight(8, *syn.host_rows(head, 0, rows), rows, d, 64), 64)
    assert np.array_equal(w4.q.cpu().numpy(), ref.q)
    assert np.array_equal(w4.scale.cpu().numpy().view(np.uint16), ref.scale)
    assert np.array_equal(w4.minv.cpu().numpy().view(np.uint16), ref.minv)
    assert err.cpu().numpy()[0] == 0


def test_q4_from_q8_nonfinite_scale_reported():
    """A Q8 group with an infinite scale dequantizes to non-finite values (the reference throws): the error word names
    the row and the group's first column, and that group's scale, min and codes are zero."""
    rng = np.random.default_rng(8)
    w8 = util.rand_qweight(rng, 8, 8, 256, 64)
    w8.scale[3 * 4 + 2] = 0x7F80  # +inf, row 3, group 2 (k 128..191)
    w4, err = kx().quantize_q4_from_q8(upload8(w8), 64)
    sync()
    assert list(err.cpu().numpy()[:3]) == [1, 3, 128]
    s4 = w4.scale.cpu().numpy().view(np.uint16).reshape(8, 4)
    assert s4[3, 2] == 0 and w4.minv.cpu().numpy().view(np.uint16).reshape(8, 4)[3, 2] == 0
    assert not w4.q.cpu().numpy().reshape(8, 128)[3, 64:96].any()
    ok = [r for r in range(8) if r != 3]
    ref = orc.q4_from_q8(orc.QWeight(8, w8.q.reshape(8, 256)[ok].ravel(), w8.scale.reshape(8, 4)[ok].ravel(),
                                     w8.minv.reshape(8, 4)[ok].ravel(), 7, 256, 64), 64)
    assert np.array_equal(w4.q.cpu().numpy().reshape(8, 128)[ok].ravel(), ref.q)


def test_draft_head_logits_and_pick():
    """DraftHead: Q4 copy of the first 4096 rows of a Q8 head, h BF16 [1, 4096] -> FP32 logits (1e-3 of the oracle's on
    the same Q4 copy) -> the pick (best id, values, NaN flag) equal to the oracle's top-2 of those logits, with the
    forward's error words copied into the record."""
    import torch
    from strixite_amd import synthetic as syn
    from strixite_amd.draft import DraftHead
    V, d, mv = 8192, 4096, 4096
    head = syn.qweight(8, V, d, 64, seed=31)
    dh = DraftHead(head, mv)
    h = syn.activations(1, d, seed=32)
    rerr = torch.tensor([0, 0, 0, 0], dtype=torch.int32, device="cuda")
    eerr = torch.tensor([1, 7, 9, 0], dtype=torch.int32, device="cuda")
    dh.forward(h, expert_err=eerr)
    p = dh.top2()
    L = dh.logits.cpu().numpy()
    w4 = orc.q4_from_q8(orc.QWeight(8, *syn.host_rows(head, 0, mv), mv, d, 64), 64)
    ref_L = orc.linear_q(util.host_bits(h), w4, out_act=orc.F32)
    util.assert_close(L, ref_L, what="draft logits")
    b, bv, sv, nan = orc.top2(L[0])
    assert (p.best, p.nan) == (b, nan) and p.best_v == bv and p.second_v == sv
    assert list(p.err)[3:6] == [1, 7, 9] and list(p.err)[:3] == [0, 0, 0]


@pytest.mark.parametrize("bits,G,N,K", [(4, 64, 65536, 4096), (4, 64, 1000, 4096), (8, 64, 4100, 2048),
                                        (4, 128, 37, 1024), (4, 128, 50, 256)])
def test_mtp_head_pick_matches_linear_then_pick(bits, G, N, K):
    """sx_mtp_head_pick (the GEMV with the pick fused, or for K = 256 the GEMV then sx_mtp_pick_ws) against
    sx_linear_q4 / q8 then the single-block sx_mtp_pick: the logits and the 64-byte pick bit for bit, on plain
    weights, on a tie at the top (two equal rows far apart: the lower id wins) and on a NaN row (flagged). Every call
    shares one workspace (the count each call leaves at zero)."""
    import torch
    rng = np.random.default_rng(N + K + bits)
    base = util.rand_qweight(rng, bits, N, K, G)
    rb, gpr = K // (2 if bits == 4 else 1), K // G
    cases = [base]
    if N >= 8:
        t = util.rand_qweight(rng, bits, N, K, G)
        for a in (t.q, t.scale, t.minv):
            w = len(a) // N
            a[(N - 3) * w:(N - 2) * w] = a[5 * w:6 * w]
        # every other row scaled down, so rows 5 and N - 3 are on top
        t.scale.reshape(N, gpr)[np.arange(N) % 2 == 0] = util.f32_to_bf16(np.float32(1e-4))
        t.scale.reshape(N, gpr)[[5, N - 3]] = util.f32_to_bf16(np.float32(0.5))
        t.minv.reshape(N, gpr)[:] = 0
        cases.append(t)
        t = util.rand_qweight(rng, bits, N, K, G)
        t.scale[(N // 2) * gpr] = 0x7FC0  # NaN: row N / 2
        cases.append(t)
    # x > 0: with zero mins the scaled-up rows' logits are the largest
    x = util.bf16_dev(util.f32_to_bf16(np.abs(rng.standard_normal((1, K))).astype(np.float32) + 0.1))
    errs = [torch.tensor([i, 2 * i, 3 * i, 0], dtype=torch.int32, device="cuda") for i in (1, 4, 7)]
    emb = torch.tensor([0x1234_5678_9ABC], dtype=torch.int64, device="cuda")
    ws = torch.zeros(kx().mtp_pick_ws_bytes(N), dtype=torch.uint8, device="cuda")
    for ci, hw in enumerate(cases):
        print(f"bits={bits} G={G} N={N} K={K} case {ci}", flush=True)
        w = kx().QWeight.upload(hw)
        ref_L = kx().linear(x, w, out_act=kx().ACT_F32)
        ref_p = kx().mtp_pick(ref_L[0], *errs, emb)
        L = torch.full((N,), 7.0, dtype=torch.float32, device="cuda")
        p = kx().mtp_head_pick(x, w, L, *errs, emb, ws)
        sync()
        assert np.array_equal(L.cpu().numpy().view(np.uint32), ref_L[0].cpu().numpy().view(np.uint32)), "logits"
        assert bytes(p.cpu().numpy()) == bytes(ref_p.cpu().numpy()), "pick"
        got = kx().pick_from_bytes(p)
        if ci == 1:
            assert got.best == 5 and got.best_v == got.second_v and not got.nan
        if ci == 2:
            assert got.nan == 1
    assert not ws[-16:].any().item(), "the count is back at zero"
