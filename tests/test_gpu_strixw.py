"""strixw files onto cuda:0 (sx_strixw_load through StrixwDevice): the data region must arrive byte for byte, every
view must point at its component, and the kernels must give on loaded weights exactly what they give on the same
bytes uploaded directly.

Files are written by the oracle's restatement of the reference's StrixwWriter (oracle/strixw.py, byte-identical to
the reference's output in the CPU tests) plus the reference-written fixture tests/golden/strixw_small.strixw.
"""
import os

import numpy as np
import pytest

from oracle import oracle as orc
from oracle import strixw as ow
from tests import util

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
SMALL = os.path.join(HERE, "golden", "strixw_small.strixw")
L = "model.language_model.layers.0.mlp."


def sw():
    from strixite_amd import strixw
    return strixw


def check_region(dev, path):
    """The device data region equals the file's bytes from the data offset on."""
    import torch
    torch.cuda.synchronize()
    blob = np.fromfile(path, dtype=np.uint8)
    got = dev.data.cpu().numpy()
    want = blob[dev.file.data_offset:]
    assert got.shape == want.shape
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} bytes differ, first at region offset {bad[:1]}"


def test_load_fixture_and_views():
    import torch
    dev = sw().StrixwDevice(SMALL, read_threads=3)
    print(f"loaded {dev.data_bytes()} bytes in {dev.load_seconds * 1e3:.2f} ms", flush=True)
    check_region(dev, SMALL)
    blob = open(SMALL, "rb").read()
    f = dev.file
    head = dev.q8("lm_head.weight", [300, 256])
    c = f.get("lm_head.weight").components
    assert head.q.cpu().numpy().tobytes() == blob[c[0].offset:c[0].offset + c[0].bytes]
    assert head.scale.cpu().numpy().tobytes() == blob[c[1].offset:c[1].offset + c[1].bytes]
    assert head.G == 64 and head.q.data_ptr() % 256 == 0
    gu = dev.qw(L + "experts_gate_up", [5 * 128, 256])
    assert gu.bits == 4 and gu.G == 128
    r = dev.bf16(L + "router", [5, 256])
    assert r.dtype == torch.bfloat16 and tuple(r.shape) == (5, 256)
    n = dev.f32("model.language_model.norm.weight", [256])
    cn = f.get("model.language_model.norm.weight").components[0]
    assert np.array_equal(n.cpu().numpy(), np.frombuffer(blob[cn.offset:cn.offset + 1024], np.float32))
    pos = dev.i64("positions", [3, 5])
    assert pos.dtype == torch.int64
    import strixite_amd as sx
    with pytest.raises(sx.SxError, match="is q8 \\[300, 256\\], expected q4"):
        dev.q4("lm_head.weight", [300, 256])
    with pytest.raises(sx.SxError, match="expected q4 or q8 row-major"):
        dev.qw("q6.weight", [4, 128])


def test_load_rejects_small_destination():
    import ctypes
    import torch
    import strixite_amd as sx
    f = sw().StrixwFile(SMALL)
    dst = torch.empty(f.data_bytes() - 1, dtype=torch.uint8, device="cuda")
    secs = ctypes.c_double()
    rc = sx.lib().sx_strixw_load(f._h, dst.data_ptr(), dst.numel(), 4, ctypes.byref(secs), None)
    assert rc == sx.SX_EINVAL and b"the data region is" in sx.lib().sx_last_error()


def test_load_many_chunks(tmp_path):
    """A file whose data region spans several rounds of the staging ring (tensors of odd sizes, one larger than a
    staging slot), loaded with 5 reader threads."""
    rng = np.random.default_rng(5)
    specs = [dict(name="big", enc=ow.Q8, shape=[150_000 + 7, 2048], G=64),  # ~307 MiB of codes
             dict(name="odd", enc=ow.BF16, shape=[1, 12345]),
             dict(name="tail", enc=ow.Q4, shape=[33, 128], G=32)]
    payloads = [[rng.integers(0, 256, b, dtype=np.uint8).tobytes() for _, b in ow.components(s["enc"], s["shape"],
                                                                                            s.get("G", 0))]
                for s in specs]
    p = tmp_path / "big.strixw"
    ow.write(p, {"k": "v"}, specs, payloads)
    del payloads
    dev = sw().StrixwDevice(p, read_threads=5)
    gb = dev.data_bytes() / 1e9
    print(f"loaded {gb:.3f} GB in {dev.load_seconds:.3f} s ({gb / dev.load_seconds:.2f} GB/s)", flush=True)
    check_region(dev, p)


def layer_file(path, E, d, I, V, seed):
    """A one-layer file: router BF16 [E + 1, d] (the shared expert's gate last), stacked q4 experts (the shared one as
    expert E), a q8 LM head. Returns the host weights as written."""
    rng = np.random.default_rng(seed)
    Ew = E + 1
    wr = util.f32_to_bf16((rng.standard_normal((Ew, d)) * 0.05).astype(np.float32))
    gu = util.rand_qweight(rng, 4, Ew * 2 * I, d, 128)
    dn = util.rand_qweight(rng, 4, Ew * d, I, 128)
    head = util.rand_qweight(rng, 8, V, d, 64)
    specs = [dict(name=L + "router", enc=ow.BF16, shape=[Ew, d]),
             dict(name=L + "experts_gate_up", enc=ow.Q4, shape=[Ew * 2 * I, d], G=128, experts=Ew),
             dict(name=L + "experts_down", enc=ow.Q4, shape=[Ew * d, I], G=128, experts=Ew),
             dict(name="lm_head.weight", enc=ow.Q8, shape=[V, d], G=64)]
    qparts = lambda w: [w.q.tobytes(), w.scale.tobytes(), w.minv.tobytes()]
    ow.write(path, {"arch": "qwen4exp"}, specs, [[wr.tobytes()], qparts(gu), qparts(dn), qparts(head)])
    return wr, gu, dn, head


def test_verify_layer_on_loaded_weights(tmp_path):
    """The one-launch MoE sublayer and the LM head on weights loaded from a file give bit-identical outputs to the
    same bytes uploaded directly, and the LM head matches the oracle."""
    import torch
    from strixite_amd import kernels as kx
    E, d, I, V, k, M = 8, 4096, 1024, 1000, 4, 6
    p = tmp_path / "layer.strixw"
    wr, gu, dn, head = layer_file(p, E, d, I, V, seed=9)
    dev = sw().StrixwDevice(p)
    lw = (dev.bf16(L + "router", [E + 1, d]), dev.qw(L + "experts_gate_up", [(E + 1) * 2 * I, d]),
          dev.qw(L + "experts_down", [(E + 1) * d, I]))
    direct = (torch.from_numpy(wr.view(np.int16)).cuda().view(torch.bfloat16), kx.QWeight.upload(gu),
              kx.QWeight.upload(dn))
    x = util.bf16_dev(util.f32_to_bf16(np.random.default_rng(1).standard_normal((M, d)).astype(np.float32)))
    outs = []
    for Wr, G, D in (lw, direct):
        sync = kx.verify_layer_sync()
        r = kx.verify_layer(x, Wr, G, D, E, k, sync, shared=True, shared_id=E, Ew=E + 1)
        torch.cuda.synchronize()
        outs.append([util.host_bits(t) if t.dtype == torch.bfloat16 else t.cpu().numpy() for t in r[:5]])
    for a, b, name in zip(outs[0], outs[1], ("logits", "ids", "coef", "h", "y")):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), name
    hq = dev.q8("lm_head.weight", [V, d])
    logits = kx.linear(x, hq, out_act=0)
    torch.cuda.synchronize()
    ref = orc.linear_q(util.host_bits(x), head, out_act=orc.F32)
    util.assert_close(logits.cpu().numpy(), ref, what="LM head on loaded weights")
