"""Shared helpers for the tests: seeded synthetic weights in the reference layout and bf16 bit conversions."""
import numpy as np

from oracle import oracle as orc


def f32_to_bf16(a):
    """Round-to-nearest-even FP32 -> BF16 bits (uint16), NaN kept quiet: formats/q4.cpp:12-19's conversion."""
    a = np.ascontiguousarray(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7F800000) == 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    keep = ((u >> np.uint64(16)) | np.where((u & 0x7FFFFF) != 0, np.uint64(0x40), np.uint64(0))) & 0xFFFF
    return np.where(nan, keep, r).astype(np.uint16)


def bf16_to_f32(b):
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def rand_qweight(rng, bits, N, K, G):
    """Uniform codes, scale = bf16(|N(0, 0.02)|), min = bf16(-(2^bits - 1) / 2 * scale): zero-mean weights."""
    q = rng.integers(0, 256, N * K // (2 if bits == 4 else 1), dtype=np.uint8)
    s = np.abs(rng.standard_normal(N * (K // G)) * 0.02).astype(np.float32)
    sb = f32_to_bf16(s)
    half = 7.5 if bits == 4 else 127.5
    mb = f32_to_bf16(-half * bf16_to_f32(sb))
    return orc.QWeight(bits, q, sb, mb, N, K, G)


def max_abs_norm_err(got, ref):
    """max |got - ref| / max |ref|: the north star's 1e-3 tolerance measure."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


# ---------------- device helpers (GPU tests) ----------------

def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def bf16_dev(bits_u16):
    """numpy uint16 BF16 bits -> torch.bfloat16 tensor on cuda:0 (the same bits)."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits_u16).view(np.int16)).cuda().view(torch.bfloat16)


def f32_dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def host_bits(t):
    """A device activation tensor back to numpy: float32, or BF16 bits as uint16."""
    import torch
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def as_f32(a):
    return bf16_to_f32(a) if a.dtype == np.uint16 else np.asarray(a, np.float32)


def bf16_ulp(r):
    """One BF16 unit in the last place at |r| (8 significant bits): 2^(floor(log2 |r|) - 7); zero maps to the smallest
    normal's ulp."""
    a = np.maximum(np.abs(np.asarray(r, np.float64)), 2.0 ** -126)
    return np.exp2(np.floor(np.log2(a)) - 7)


def assert_close(got, ref, tol=1e-3, what="", roundings=1, max_off_frac=1e-3, max_bias=1e-4):
    """The north star's bar, plus two checks that catch a systematic error the per-element bound would let through.

    1. Per element: max |got - ref| <= tol * max |ref| (FP32 outputs). BF16 outputs (uint16 bits) may also differ by the
       roundings to BF16 along the way: + roundings * 2^-8 |ref| per element (1: the store; SwiGLU of stored gate and
       up: gate, up, silu and the product, 4). A BF16 reference was rounded once more on its own side: two FP32 values
       a hair apart can round to neighbouring BF16 values, up to 2 x 2^-8 |ref| apart.
    2. At most max_off_frac of the elements (at least one) differ by more than one BF16 ulp of the reference plus
       tol / 10 of max |ref| (a value that differs only by summation order is off by far less).
    3. The mean signed error over all elements is below max_bias * max |ref|, widened for small arrays by three
       standard errors of unbiased BF16 rounding (2^-8 mean |ref| / sqrt(n)): a bias of 1 % in every element fails."""
    g = as_f32(got).astype(np.float64)
    r = as_f32(ref).astype(np.float64)
    assert g.shape == r.shape, (g.shape, r.shape)
    if not np.array_equal(np.isnan(g), np.isnan(r)):
        bad = np.argwhere(np.isnan(g) != np.isnan(r))
        raise AssertionError(f"{what}: NaN pattern differs: {int(np.isnan(g).sum())} NaN on the GPU, "
                             f"{int(np.isnan(r).sum())} in the oracle, first at {bad[:4].tolist()}")
    ok = ~np.isnan(r)
    if not ok.any():
        return
    scale = max(np.max(np.abs(r[ok])), 1e-30)
    if np.asarray(got).dtype == np.uint16:
        roundings += 1 if np.asarray(ref).dtype == np.uint16 else 0
        bound = tol * scale + roundings * 2.0 ** -8 * np.abs(r[ok])
    else:
        bound = tol * scale
    diff = g[ok] - r[ok]
    err = np.abs(diff)
    worst = float(np.max(err / scale))
    assert np.all(err <= bound), f"{what}: max-abs-normalised error {worst:.3g} over tolerance {tol}"
    off = int(np.count_nonzero(err > bf16_ulp(r[ok]) + 0.1 * tol * scale))
    allowed = max(1, int(max_off_frac * err.size))
    assert off <= allowed, (f"{what}: {off} of {err.size} elements ({off / err.size:.2%}) differ by more than one "
                            f"BF16 ulp; at most {allowed} allowed")
    bias = float(np.mean(diff)) / scale
    limit = max_bias + 3 * 2.0 ** -8 * float(np.mean(np.abs(r[ok]))) / scale / np.sqrt(err.size)
    assert abs(bias) <= limit, f"{what}: mean signed error {bias:.3g} of max |ref| (limit {limit:.3g})"
