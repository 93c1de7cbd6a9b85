"""Parity of the dense dequantizing GEMV/GEMM (linear_q4 / linear_q8, kernels/linear_q4.hpp:26-30,
linear_q8.hpp:13-14) against the CPU oracle, through the C ABI on cuda:0."""
import numpy as np
import pytest

from oracle import oracle as orc
from tests import util

pytestmark = pytest.mark.gpu

F32, BF16 = orc.F32, orc.BF16


def run(bits, N, K, G, M, act, out_act, seed=0):
    import torch
    from strixite_amd import kernels as kx
    rng = np.random.default_rng(seed)
    w = util.rand_qweight(rng, bits, N, K, G)
    x = rng.standard_normal((M, K)).astype(np.float32)
    xh = x if act == F32 else util.f32_to_bf16(x)
    ref = orc.linear_q(xh, w, out_act=out_act)
    xd = util.f32_dev(xh) if act == F32 else util.bf16_dev(xh)
    y = kx.linear(xd, kx.QWeight.upload(w), out_act=out_act)
    torch.cuda.synchronize()
    return util.host_bits(y), ref


@pytest.mark.parametrize("bits,G", [(4, 128), (8, 64), (8, 128), (4, 64), (4, 32), (8, 32)])
@pytest.mark.parametrize("M", [1, 6, 17])
def test_linear_groups_and_rows(bits, G, M):
    got, ref = run(bits, 80, 512, G, M, BF16, F32, seed=M + G)
    util.assert_close(got, ref, what=f"q{bits} G{G} M{M}")


@pytest.mark.parametrize("act,out_act", [(F32, F32), (BF16, BF16), (BF16, F32)])
@pytest.mark.parametrize("bits", [4, 8])
def test_linear_dtypes_partial_tile(act, out_act, bits):
    got, ref = run(bits, 37, 384 if bits == 4 else 320, 128 if bits == 4 else 64, 5, act, out_act, seed=3)
    util.assert_close(got, ref, what=f"q{bits} act {act}->{out_act}")


def test_config1_dense_q4_gemv_f32():
    # x fp32 [1 x 4096], W 4096 x 4096 q4 G = 128, y fp32
    got, ref = run(4, 4096, 4096, 128, 1, F32, F32, seed=0)
    util.assert_close(got, ref, what="config 1")


@pytest.mark.parametrize("bits,G", [(4, 128), (8, 64)])
def test_config2_verify_width(bits, G):
    # x bf16 [6 x 4096], W 12288 x 4096, fp32 out
    got, ref = run(bits, 12288, 4096, G, 6, BF16, F32, seed=1)
    util.assert_close(got, ref, what=f"config 2 q{bits}")


@pytest.mark.parametrize("bits,K", [(4, 512), (4, 1024), (4, 4096), (4, 8192), (8, 256), (8, 1024), (8, 4096)])
@pytest.mark.parametrize("M,act,out_act", [(1, F32, F32), (5, BF16, BF16), (16, BF16, F32), (3, F32, F32)])
def test_linear_k_split_path(bits, K, M, act, out_act):
    """The decode / verify-width kernel (K split over a block's waves, dense_ks.hip) on the shapes it takes - q4 G = 128
    and q8 G = 64 with 4 .. 64 spans, M <= 16, at most a 16-row tile a block - and its neighbours the general kernel
    takes (FP32 x too long for its LDS, more tiles than blocks): a partial last tile, a run of tiles a block."""
    G = 128 if bits == 4 else 64
    N = 3000 if K == 1024 else 200
    got, ref = run(bits, N, K, G, M, act, out_act, seed=K + M)
    util.assert_close(got, ref, what=f"q{bits} K{K} M{M} act {act}->{out_act}")


def test_linear_rejects_misaligned_x():
    import torch
    from strixite_amd import kernels as kx, SxError
    w = kx.QWeight.upload(util.rand_qweight(np.random.default_rng(0), 4, 16, 128, 128))
    x = torch.zeros(2 * 128 + 1, dtype=torch.bfloat16, device="cuda")[1:].view(2, 128)
    with pytest.raises(SxError, match="16-byte aligned"):
        kx.linear(x, w)


@pytest.mark.parametrize("bits,K,G", [(4, 96, 32), (4, 64, 64), (4, 320, 64), (8, 96, 32), (8, 32, 32)])
def test_linear_k_not_a_whole_span(bits, K, G):
    """K that ends inside the kernels' 64-byte row span (the reference allows any K % G == 0)."""
    got, ref = run(bits, 24, K, G, 3, BF16, F32, seed=K)
    util.assert_close(got, ref, what=f"q{bits} K{K} G{G}")
