"""The drop-in boundary without a GPU: strixite_amd/integration/strix_kernels_shim.cpp defines, with identical
signatures, every operator that the reference's kernels/*.hpp headers declare for the source files the integration
recipe removes from strix_kernels, and nothing else outside its anonymous namespace; and every C-ABI
entry point it calls is declared in include/strixite_amd.h.

Two checks: a comparison of the parsed declarations (types and order of the parameters, return type, default
arguments left out), and a compile of the shim against the reference's own headers with hipcc -fsyntax-only.
strixite's common/hip_runtime.hpp includes <format>, which this image's GCC 11 lacks and which none of the headers the
shim reaches uses, so the compile puts a directory holding an empty `format` header first on the include path.
Skipped when the reference tree is absent (the GPU box)."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
SHIM = os.path.join(ROOT, "strixite_amd", "integration", "strix_kernels_shim.cpp")
HEADER = os.path.join(ROOT, "include", "strixite_amd.h")
INTEGRATION = os.path.join(ROOT, "INTEGRATION.md")

# the reference sources the recipe takes out of strix_kernels, and the headers declaring what they define
REPLACED = {
    "kernels/linear.hip": "kernels/linear.hpp",
    "kernels/linear_q4.hip": "kernels/linear_q4.hpp",
    "kernels/linear_q56.hip": ("kernels/linear_q5.hpp", "kernels/linear_q6.hpp"),
    "kernels/linear_q8.hip": "kernels/linear_q8.hpp",
    "kernels/linear_wmma.hip": "kernels/linear_wmma.hpp",
    "kernels/moe_router.hip": "kernels/moe_router.hpp",
    "kernels/moe_grouped.hip": "kernels/moe_grouped.hpp",
    "kernels/swiglu.hip": "kernels/swiglu.hpp",
    "kernels/logits_topk.hip": "kernels/logits_topk.hpp",
    "kernels/mtp_pick.hip": "kernels/mtp_pick.hpp",
}

pytestmark = pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "kernels")), reason="reference tree absent")


def strip_comments(t):
    t = re.sub(r"/\*.*?\*/", "", t, flags=re.S)
    return re.sub(r"//[^\n]*", "", t)


def norm_params(params):
    """Parameter types in order: names, default values and spacing dropped ('const uint32_t e[3]' -> pointer)."""
    out = []
    for p in [p.strip() for p in params.split(",") if p.strip()]:
        p = p.split("=")[0].strip()
        p = re.sub(r"\[\d*\]$", "*", re.sub(r"\s*(\w+)\s*(\[\d*\])$", r" \2", p)) if "[" in p else p
        toks = re.findall(r"[A-Za-z_]\w*|[*&]", p)
        # a trailing identifier after a complete type is the parameter's name
        if len(toks) >= 2 and re.match(r"[A-Za-z_]", toks[-1]) and toks[-2] not in ("const", "unsigned", "signed"):
            toks = toks[:-1]
        out.append(" ".join(toks))
    return tuple(out)


def declarations(path):
    t = strip_comments(open(path).read())
    decls = set()
    for m in re.finditer(r"(?m)^\s*([A-Za-z_][\w:]*(?:\s*[*&])*)\s+([A-Za-z_]\w*)\s*\(([^;{}]*)\)\s*;", t):
        decls.add((m.group(1).strip(), m.group(2), norm_params(m.group(3))))
    return decls


def shim_definitions():
    t = strip_comments(open(SHIM).read())
    body = t[t.index("namespace strix::kernels {"):]
    # drop the anonymous namespace (helpers that are not part of the interface)
    a = body.index("namespace {")
    depth, i = 0, a
    while True:
        if body[i] == "{":
            depth += 1
        elif body[i] == "}":
            depth -= 1
            if depth == 0:
                break
        i += 1
    body = body[:a] + body[i + 1:]
    defs = set()
    for m in re.finditer(r"(?m)^([A-Za-z_][\w:]*(?:\s*[*&])*)\s+([A-Za-z_]\w*)\s*\(([^;{}]*)\)\s*\{", body):
        defs.add((m.group(1).strip(), m.group(2), norm_params(m.group(3))))
    return defs


def expected():
    want = set()
    for hdrs in REPLACED.values():
        for h in (hdrs if isinstance(hdrs, tuple) else (hdrs,)):
            want |= declarations(os.path.join(REF, h))
    return want


def test_shim_defines_exactly_the_replaced_operators():
    want, have = expected(), shim_definitions()
    missing = sorted(want - have)
    extra = sorted(have - want)
    assert not missing, "declared in the reference headers but not defined by the shim: " + repr(missing)
    assert not extra, "defined by the shim but declared by no replaced header: " + repr(extra)


def test_shim_calls_only_declared_entry_points():
    hdr = open(HEADER).read()
    declared = set(re.findall(r"^\s*(?:int|const char \*)\s*(sx_\w+)\s*\(", hdr, re.M))
    called = set(re.findall(r"\b(sx_[a-z_0-9]+)\s*\(", strip_comments(open(SHIM).read())))
    called -= {"sx_qview", "sx_stream"}
    assert called <= declared, sorted(called - declared)


def test_recipe_names_the_reference_target_and_sources():
    """The recipe edits strix_kernels' strix_hip_sources list (CMakeLists.txt:193-197) and removes exactly the
    replaced sources, each of which that list holds."""
    cm = open(os.path.join(REF, "CMakeLists.txt")).read()
    m = re.search(r"strix_hip_sources\(strix_kernels([^)]*)\)", cm)
    listed = set(m.group(1).split())
    doc = open(INTEGRATION).read()
    assert "strix_hip_sources(strix_kernels" in doc
    for src in REPLACED:
        assert src in listed, f"{src} is not in the reference's strix_kernels sources"
        assert src in doc, f"the recipe does not name {src}"


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc absent")
def test_shim_compiles_against_reference_headers(tmp_path):
    (tmp_path / "format").write_text("")
    cmd = ["hipcc", "-std=c++20", "-fsyntax-only", "--offload-arch=gfx950", f"-I{tmp_path}", f"-I{REF}",
           f"-I{os.path.join(ROOT, 'include')}", SHIM]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
