"""The allocation-free logits top-k (sx_logits_topk_noalloc, the library's fixed device scratch) against
sx_logits_topk with a caller's workspace, through the C ABI on cuda:0: bit-identical candidates and NaN flags on two
calls in a row, the second smaller than the first (the scratch keeps the first call's contents), and a shape whose
scratch need exceeds the fixed size is refused before any launch."""
import numpy as np
import pytest

from tests import util

pytestmark = pytest.mark.gpu


def _case(rng, rows, n, k, with_mask):
    import torch
    from strixite_amd import kernels as kx
    L = rng.standard_normal((rows, n)).astype(np.float32)
    L[0, n // 3] = np.nan
    L[rows - 1, : min(n, 300)] = 5.0  # ties at the top
    Ld = util.f32_dev(L)
    mask = None
    if with_mask:
        m = rng.integers(0, 2**32, (rows, (n + 31) // 32), dtype=np.uint64).astype(np.uint32)
        mask = torch.from_numpy(m.view(np.int32)).cuda()
    ref = kx.logits_topk(Ld, n, k, mask=mask)
    got = kx.logits_topk_noalloc(Ld, n, k, mask=mask)
    torch.cuda.synchronize()
    assert torch.equal(ref[3], got[3]), f"candidates differ at rows={rows} n={n} k={k}"
    assert torch.equal(ref[2], got[2]), f"NaN flags differ at rows={rows} n={n} k={k}"


@pytest.mark.parametrize("with_mask", [False, True])
def test_noalloc_topk_matches_workspace_entry(with_mask):
    rng = np.random.default_rng(7 + with_mask)
    print(f"noalloc top-k: rows=6 n=151936 k=40 mask={with_mask}", flush=True)
    _case(rng, 6, 151936, 40, with_mask)   # config 5's shape: three levels
    print(f"noalloc top-k: rows=3 n=20000 k=20 mask={with_mask}", flush=True)
    _case(rng, 3, 20000, 20, with_mask)    # a smaller second call on the same scratch


def test_noalloc_topk_refuses_oversized_shape():
    import ctypes
    import strixite_amd as sx
    L = sx.lib()
    n = ctypes.c_size_t()
    assert L.sx_logits_topk_workspace_bytes(65535, 151936, 64, ctypes.byref(n)) == 0
    assert n.value > sx_scratch_bytes()
    p = ctypes.c_void_p(256)  # never dereferenced: the size check comes first
    rc = L.sx_logits_topk_noalloc(p, 65535, 151936, 151936, 64, p, p, None, 0, None)
    assert rc == sx.SX_EINVAL and b"scratch" in L.sx_last_error()


def sx_scratch_bytes():
    import os
    import re
    hdr = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                            "strixite_amd.h")).read()
    m = re.search(r"#define SX_TOPK_SCRATCH_BYTES \((\d+)u << (\d+)\)", hdr)
    return int(m.group(1)) << int(m.group(2))
