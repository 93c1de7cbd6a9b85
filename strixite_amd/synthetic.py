"""Seeded synthetic inputs in the reference's formats, generated on the device (bench.py, smoke and the GPU tests).

Weights follow BASELINE.json's configs with the reference's actual format (formats/q4.hpp:3-6, q8.hpp:3-11): uniform
codes, scale = bf16(|N(0, 0.02)|), min = bf16(-(2^bits - 1) / 2 * scale) so the weights are zero-mean. torch's
device generator (Philox) makes them from the seed; the CPU oracle gets host copies of the same bytes.
"""
import torch

from .kernels import QWeight


def qweight(bits, N, K, G, seed, device="cuda"):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    nbytes = N * K // (2 if bits == 4 else 1)
    q = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=device, generator=g)
    s = (torch.randn(N * (K // G), device=device, generator=g) * 0.02).abs().to(torch.bfloat16)
    half = 7.5 if bits == 4 else 127.5
    m = (-half * s.float()).to(torch.bfloat16)
    return QWeight(bits, q, s.view(torch.int16), m.view(torch.int16), N, K, G)


def activations(M, K, seed, dtype=torch.bfloat16, device="cuda"):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.randn(M, K, device=device, generator=g).to(dtype)


def router_weight(E, K, seed, device="cuda"):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.randn(E, K, device=device, generator=g) * 0.02


def zipf_router_bias(E, seed, s=1.1, scale=0.3, device="cuda"):
    """BASELINE config 4's routing skew: a bias added to the router logits, -scale * s * ln(rank + 1) for the
    experts in a seeded random order of ranks (a Zipf(s) prior in log space). scale = 0.3 against logits of standard
    deviation ~1.3 (x ~ N(0, 1), Wr ~ N(0, 0.02), d = 4096) gives buckets of 0..~450 of 20,480 slots at top-10."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(E, generator=g)
    bias = torch.empty(E, dtype=torch.float32)
    bias[perm] = -scale * s * torch.log(torch.arange(E, dtype=torch.float32) + 1.0)
    return bias.to(device)


def host_rows(w, r0, r1):
    """Host numpy copy (q, scale, minv) of weight rows [r0, r1): for the oracle on the rows a test touches."""
    r0, r1 = int(r0), int(r1)  # numpy integers would overflow int32 on the byte offsets of large weights
    per = w.K // (2 if w.bits == 4 else 1)
    groups = w.K // w.G
    q = w.q[r0 * per:r1 * per].cpu().numpy()
    s = w.scale[r0 * groups:r1 * groups].cpu().numpy().view("uint16")
    m = w.minv[r0 * groups:r1 * groups].cpu().numpy().view("uint16")
    return q, s, m
