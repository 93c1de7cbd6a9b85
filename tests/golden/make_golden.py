"""Writes the golden fixtures in this folder from the reference's own host code, compiled by oracle/Makefile into
oracle/_ref/libstrix_ref.so (formats/q4.cpp, formats/q8.cpp, serve/sampler.cpp from /root/reference).

Run in the build container (the reference tree is not on the GPU box):  python tests/golden/make_golden.py
Each fixture holds seeded inputs and the reference's outputs, nothing else:
  formats.npz  quantize_q4 / quantize_q8 + dequantize (formats/q4.cpp:44-134, q8.cpp:40-127), G = 32, 64, 128
  top2.npz     serve/sampler.cpp:79-101 top2 on random rows, ties, -inf and single-logit rows
  sampler.npz  Sampler::sample (serve/sampler.cpp:103-328), one call per row in sequence, for several parameter sets
  accept.npz   the engine's accept loop (serve/engine.cpp:592-610) driven by the reference Sampler, drafts built so
               the accepted length is each of 0..5, greedy and sampled (T 0.7, top-k 40, top-p 0.95)
  q4_from_q8.npz  formats/q4_from_q8.cpp quantize_q4_from_q8 (the MTP draft head's Q4 copy) of seeded Q8 weights:
               Q8 groups 64 and 128 into Q4 groups 32, 64, 128, with constant, one-code and wide groups
  strixw_small.strixw  a file written by formats/strixw.cpp's StrixwWriter from oracle/strixw.py's sample_plan()
               (every encoding, metadata, parts)
  strixw_hash.npz  strix_hash64 (formats/strixw.cpp:253-274) of seeded buffers of every length 0..300 and some long ones
Run with fixture names (e.g. `make_golden.py q4_from_q8`) to write only those.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as orc  # noqa: E402


def formats():
    out = {}
    rng = np.random.default_rng(1)
    for bits in (4, 8):
        for G in (32, 64, 128):
            N, K = 6, 384
            w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
            w[1, :G] = 0.125           # a constant group: s = 0, codes 0
            w[2, G:2 * G] = -3.5e-3    # constant negative group
            w[3, :G] *= 1000.0          # a wide group
            qw, deq = orc.ref_quantize(bits, w, G)
            tag = f"q{bits}_g{G}"
            out[tag + "_w"] = w
            out[tag + "_q"] = qw.q
            out[tag + "_scale"] = qw.scale
            out[tag + "_min"] = qw.minv
            out[tag + "_deq"] = deq
    np.savez_compressed(os.path.join(HERE, "formats.npz"), **out)


def top2():
    rng = np.random.default_rng(2)
    rows = []
    for n in (1, 2, 3, 63, 64, 65, 200, 1000):
        rows.append(rng.standard_normal(n).astype(np.float32))
    r = rng.standard_normal(300).astype(np.float32)
    r[17] = r[250] = 9.0  # a tie for the best: the lower id wins, second == best
    rows.append(r)
    r = rng.standard_normal(130).astype(np.float32)
    r[5] = 4.0
    r[100] = r[129] = 3.0  # a tie for second
    rows.append(r)
    rows.append(np.full(70, -np.inf, np.float32))
    r = rng.standard_normal(129).astype(np.float32)
    r[0] = 0.0
    r[64] = -0.0
    r[:] = np.minimum(r, 0.0)
    rows.append(r)
    n = max(len(x) for x in rows)
    X = np.full((len(rows), n), np.nan, np.float32)
    lens = np.array([len(x) for x in rows], np.int64)
    exp = np.zeros((len(rows), 4), np.float64)
    for i, x in enumerate(rows):
        X[i, :len(x)] = x
        b, bv, sv, nan = orc.ref_top2(x)
        exp[i] = (b, bv, sv, nan)
    np.savez_compressed(os.path.join(HERE, "top2.npz"), x=X, n=lens, expect=exp)


SAMPLER_PARAMS = [  # temperature, top_k, top_p, seed
    (0.0, 40, 0.95, 11),
    (0.7, 40, 0.95, 12),
    (0.7, 20, 0.95, 13),
    (1.0, 20, 1.0, 14),
    (0.7, 100, 0.9, 15),
    (1.0, 0, 1.0, 16),
    (0.7, 0, 0.95, 17),
    (0.3, 5, 0.5, 18),
]


def sampler():
    rng = np.random.default_rng(3)
    V, R = 512, 16
    out = {"params": np.array(SAMPLER_PARAMS, np.float64)}
    for pi, (T, k, p, seed) in enumerate(SAMPLER_PARAMS):
        X = (rng.standard_normal((R, V)) * 2.5).astype(np.float32)
        X[3, 7] = X[3, 400] = X[3].max() + 1.0  # a tie at the top
        s = orc.RefSampler(T, k, p, int(seed), V)
        ids = np.array([s.sample(X[r]) for r in range(R)], np.int32)
        out[f"x{pi}"] = X
        out[f"ids{pi}"] = ids
        # the same params through sample_candidates (the logits_topk path) when the sampler takes candidates
        if T == 0 or 1 <= k <= 20:
            s2 = orc.RefSampler(T, k, p, int(seed), V)
            cids = []
            for r in range(R):
                order = sorted(range(V), key=lambda i: (-X[r, i], i))[:20]
                cids.append(s2.sample_candidates(X[r, order], np.array(order, np.int32)))
            out[f"cand_ids{pi}"] = np.array(cids, np.int32)
    np.savez_compressed(os.path.join(HERE, "sampler.npz"), **out)


def accept():
    rng = np.random.default_rng(4)
    V, k = 1024, 5
    cases = []
    for mode, (T, tk, tp) in (("greedy", (0.0, 40, 0.95)), ("sampled", (0.7, 40, 0.95))):
        for target in range(k + 1):
            seed = 1000 + 10 * target + (1 if mode == "sampled" else 0)
            X = (rng.standard_normal((k + 1, V)) * 3.0).astype(np.float32)
            # what the sampler draws at each row in sequence (the same seed replays the same draws)
            s = orc.RefSampler(T, tk, tp, seed, V)
            seq = [s.sample(X[r]) for r in range(k + 1)]
            drafts = np.array(seq[:k], np.int32)
            if target < k:
                drafts[target] = (seq[target] + 1 + int(rng.integers(0, V - 1))) % V
                if drafts[target] == seq[target]:
                    drafts[target] = (drafts[target] + 1) % V
                drafts[target + 1:] = rng.integers(0, V, k - target - 1)
            # the engine loop with a fresh reference sampler: accept while the sample equals the draft; the last row
            # (all accepted) is sampled as the next step's token
            s = orc.RefSampler(T, tk, tp, seed, V)
            toks = []
            j = 0
            while True:
                v = s.sample(X[j])
                toks.append(v)
                if j == k or v != drafts[j]:
                    break
                j += 1
            assert j == target, (mode, target, j)
            cases.append((T, tk, tp, seed, X, drafts, j, np.array(toks + [-1] * (k + 1 - len(toks)), np.int32)))
    np.savez_compressed(os.path.join(HERE, "accept.npz"),
                        params=np.array([c[:4] for c in cases], np.float64),
                        x=np.stack([c[4] for c in cases]), drafts=np.stack([c[5] for c in cases]),
                        j=np.array([c[6] for c in cases], np.int64), tokens=np.stack([c[7] for c in cases]))


def q4_from_q8():
    rng = np.random.default_rng(5)
    out = {}
    for G8, G4 in ((64, 64), (64, 128), (64, 32), (128, 64)):
        N, K = 24, 512
        q = rng.integers(0, 256, N * K, dtype=np.uint8)
        s = (np.abs(rng.standard_normal(N * (K // G8))) * 0.02).astype(np.float32)
        sb = (s.view(np.uint32) >> 16).astype(np.uint16)  # truncated to BF16: any BF16 scale will do
        mb = ((-127.5 * (sb.astype(np.uint32) << 16).view(np.float32)).view(np.uint32) >> 16).astype(np.uint16)
        q.reshape(N, K)[1, :G8] = 77                       # one code in a group: a constant Q4 group (s = 0)
        q.reshape(N, K)[2, :] = rng.integers(0, 2, K)      # two codes only
        sb.reshape(N, K // G8)[3, 0] = 0                   # zero scale: constant dequantized values
        sb.reshape(N, K // G8)[4, 0] = 0x4100              # a wide group (scale 8.0)
        w8 = orc.QWeight(8, q, sb, mb, N, K, G8)
        r = orc.ref_q4_from_q8(w8, G4)
        tag = f"g{G8}_g{G4}"
        out[tag + "_q8"], out[tag + "_s8"], out[tag + "_m8"] = q, sb, mb
        out[tag + "_q4"], out[tag + "_s4"], out[tag + "_m4"] = r.q, r.scale, r.minv
    out["shape"] = np.array([24, 512], np.int64)
    np.savez_compressed(os.path.join(HERE, "q4_from_q8.npz"), **out)


def strixw():
    from oracle import strixw as sw
    meta, specs, payloads = sw.sample_plan(seed=7)
    sw.ref_write(os.path.join(HERE, "strixw_small.strixw"), meta, specs, payloads)
    rng = np.random.default_rng(8)
    lens = list(range(301)) + [1023, 4096, 4099, 65536 + 13]
    data = rng.integers(0, 256, sum(lens), dtype=np.uint8)
    hashes = np.zeros(len(lens), dtype=np.uint64)
    at = 0
    for i, n in enumerate(lens):
        hashes[i] = sw.ref_hash64(data[at:at + n].tobytes())
        at += n
    np.savez_compressed(os.path.join(HERE, "strixw_hash.npz"), data=data, lens=np.array(lens, dtype=np.int64),
                        hash=hashes)


if __name__ == "__main__":
    if not orc.ref_available():
        orc.build()
    todo = sys.argv[1:] or ["formats", "top2", "sampler", "accept", "q4_from_q8", "strixw"]
    for name in todo:
        globals()[name]()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
