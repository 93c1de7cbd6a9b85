"""The C-ABI library without a GPU: it loads, exports every symbol include/strixite_amd.h declares, and its host-side
precondition checks answer before any launch (CPU only)."""
import ctypes
import os
import re

import pytest

import strixite_amd as sx

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "strixite_amd.h")


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(sx.LIB_PATH):
        from strixite_amd import build
        build.build(verbose=False)
    return sx.lib()


def declared():
    text = open(HEADER).read()
    return set(re.findall(r"^\s*(?:int|const char \*|uint64_t|void)\s*(sx_\w+)\s*\(", text, re.M))


def test_header_and_python_signatures_agree():
    assert declared() == set(sx.SIGNATURES), declared() ^ set(sx.SIGNATURES)


def declared_arity():
    """name -> number of parameters, parsed from the header's prototypes."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:int|const char \*|uint64_t|void)\s*(sx_\w+)\s*\(([^;]*?)\)\s*;", text, re.M | re.S):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_python_argtypes_match_header_arity():
    """Each ctypes signature has as many arguments as the C prototype (a dropped pointer would shift the rest)."""
    ar = declared_arity()
    assert set(ar) == declared()
    for name, n in ar.items():
        assert len(sx.SIGNATURES[name]) == n, f"{name}: {len(sx.SIGNATURES[name])} argtypes, header has {n}"


def test_every_declared_symbol_is_exported(L):
    for name in declared():
        assert hasattr(L, name), name
    assert b"gfx950" in L.sx_version()


def test_precondition_errors_name_the_problem(L):
    w = sx.QView(None, None, None, 16, 128, 128)
    rc = L.sx_linear_q4(None, ctypes.byref(w), None, 1, sx.ACT_BF16, sx.ACT_BF16, None)
    assert rc == sx.SX_EINVAL and b"null pointer" in L.sx_last_error()
    # a weight view with a bad group size (kernels/linear_q4.hip:418)
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p).value
    w = sx.QView(p, p, p, 16, 128, 48)
    rc = L.sx_linear_q8(ctypes.c_void_p(p), ctypes.byref(w), ctypes.c_void_p(p + 32), 1, sx.ACT_BF16, sx.ACT_BF16, None)
    assert rc == sx.SX_EINVAL and b"group size 48" in L.sx_last_error()
    # k above the router's 32 (kernels/moe_router.hpp:37)
    rc = L.sx_moe_router(ctypes.c_void_p(p), 512, 1, 512, 33, None, 0, 0, ctypes.c_void_p(p), ctypes.c_void_p(p + 8),
                         sx.ACT_F32, ctypes.c_void_p(p + 16), None)
    assert rc == sx.SX_EINVAL and b"k = 33" in L.sx_last_error()


def test_route_workspace_layout_contract(L):
    # kernels/moe_grouped.hip:63-81: [4 header] [E + 2 offsets] [S slots] [2 x Tmax] [2 x WTmax], Tmax = S/16 + E + 2,
    # WTmax = S/64 + E + 2.
    for M, A, E in [(6, 10, 512), (2048, 10, 512), (1, 1, 1), (3, 11, 513)]:
        S = M * A
        n = ctypes.c_size_t()
        assert L.sx_moe_route_workspace_bytes(M, A, E, ctypes.byref(n)) == 0
        assert n.value == 4 * (4 + E + 2 + S + 2 * (S // 16 + E + 2) + 2 * (S // 64 + E + 2))
    assert L.sx_moe_route_workspace_bytes(1, 1, 1024, ctypes.byref(n)) == sx.SX_EINVAL


def test_topk_workspace_and_reports(L):
    n = ctypes.c_size_t()
    assert L.sx_logits_topk_workspace_bytes(6, 151936, 40, ctypes.byref(n)) == 0
    g1 = (151936 + 4095) // 4096  # first-level groups of 4096 logits
    assert n.value == 2 * 6 * g1 * 40 * 8 + 6 * g1 * 4
    e = (ctypes.c_uint32 * 3)(1, 700, 5)
    assert L.sx_report_expert_error(e, b"layer 3") == sx.SX_EINVAL
    assert b"expert id 700 at slot 5" in L.sx_last_error()
    e = (ctypes.c_uint32 * 3)(0, 0, 0)
    assert L.sx_report_router_error(e, b"x") == sx.SX_OK


def test_pick_workspace_contract(L):
    # the many-block pick's workspace: a 16-byte top-2 for each of up to 256 blocks and the count
    n = ctypes.c_size_t()
    assert L.sx_mtp_pick_ws_bytes(65536, ctypes.byref(n)) == 0 and n.value == 256 * 16 + 16
    assert L.sx_mtp_pick_ws_bytes(0, ctypes.byref(n)) == sx.SX_EINVAL
    buf = (ctypes.c_uint8 * 8192)()
    p = ctypes.cast(buf, ctypes.c_void_p).value
    p16 = (p + 15) // 16 * 16
    P = lambda o=0: ctypes.c_void_p(p16 + o)
    rc = L.sx_mtp_pick_ws(P(), 1000, P(), P(), P(), P(), P(), P(64), 4000, None)
    assert rc == sx.SX_EINVAL and b"need 4112" in L.sx_last_error()
    rc = L.sx_mtp_pick_ws(P(), 1000, P(), P(), P(), P(), P(), P(8), 4112, None)
    assert rc == sx.SX_EINVAL and b"16-byte aligned" in L.sx_last_error()
    w = sx.QView(p16, p16, p16, 16, 128, 64)
    rc = L.sx_mtp_head_pick(P(), ctypes.byref(w), 5, P(), P(), P(), P(), P(), P(), P(64), 4112, None)
    assert rc == sx.SX_EINVAL and b"bits = 5" in L.sx_last_error()
    rc = L.sx_mtp_head_pick(P(), ctypes.byref(w), 4, P(1024), P(), P(), P(), P(), P(), P(64), 100, None)
    assert rc == sx.SX_EINVAL and b"need 4112" in L.sx_last_error()


def test_engine_draft_and_commit_rules():
    """serve/engine.cpp:574-581 (a draft is kept when its top-1 margin reaches mtp_margin and it is no end token; NaN is
    an error) and :612-645 (keep every verify row when all drafts were accepted, else the verified token and the
    accepted drafts)."""
    from strixite_amd import MtpPick
    from strixite_amd.draft import commit_after_accept, draft_continues
    p = MtpPick(best=5, best_v=3.0, second_v=1.0, nan=0)
    assert draft_continues(p, 2.0, {7, 8}) and not draft_continues(p, 2.5, {7, 8})
    assert not draft_continues(MtpPick(best=7, best_v=9.0, second_v=1.0, nan=0), 2.0, {7, 8})
    with pytest.raises(RuntimeError):
        draft_continues(MtpPick(best=0, best_v=0.0, second_v=0.0, nan=1), 2.0, set())
    assert commit_after_accept(5, 5) == ("keep_verify", 6)
    assert [commit_after_accept(j, 5) for j in range(5)] == [("keep_verify_prefix", j + 1) for j in range(5)]
    with pytest.raises(ValueError):
        commit_after_accept(6, 5)
